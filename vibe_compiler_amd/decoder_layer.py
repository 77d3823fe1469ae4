"""Decoder layer (Llama-style) composed from the gfx950 backend's regions.

This is the order of regions a lowered Llama decoder block runs through the
backend, each one a C-ABI call of ``libwafer_hip.so`` on the caller's stream:

    h    = RMSNorm(x) * w_in                          wafer_hip_rmsnorm
    qkv  = h . Wqkv^T        [T, (Hq + 2 Hkv) D]      wafer_hip_gemm_mfma (bf16 / f16 MFMA)
    q,k  = RoPE(q), RoPE(k) -> head-major [H, T, D]  wafer_hip_head_permute_rope
    a    = causal GQA attention(q, k, v)              wafer_hip_attention_prefill_strided (FA; V read
                                                      from the QKV rows, a written token-major [T, Hq D])
    x1   = x + a . Wo^T                               wafer_hip_gemm_mfma, wafer_hip_add_rmsnorm (Add
    h2   = RMSNorm(x1) * w_post                         and the norm in one pass)
    act  = silu(h2 . Wg^T) * (h2 . Wu^T)              wafer_hip_gemm_mfma_swiglu
    y    = x1 + act . Wd^T                            wafer_hip_gemm_mfma_residual (the Add in the
                                                      GEMM's epilogue)

The fused SwiGLU GEMM gives the same bits as the unfused sequence (gate and
up GEMMs with narrow outputs, then the silu_mul region): its epilogue rounds
each product to the storage format first and then applies the region's own
arithmetic.

The math is the reference's CPU reference of the decoder block
(test/Tools/Inputs/wafer_pytorch_xla_capture.py:1183-1260: rms_norm with
reciprocal-sqrt of the mean square plus eps, q/k/v/o/gate/up/down linear
layers as x . W^T, rotate-half RoPE with inv_freq = 1/theta^(2i/D), causal
softmax attention with scale 1/sqrt(D), SwiGLU MLP) and of the board case
built on the Hugging Face decoder layer
(test/Board/PyTorch/wafer_pytorch_board_cases.py:817-866, the llama-2-7b-block
case, F16 or BF16).  Storage between regions is the layer's dtype (bf16 or
f16), every region computes in f32; results match an f32 torch evaluation of
the same layer within the attention tolerance, not bit for bit.

Weights are kept in the nn.Linear orientation [out, in] (rhs Transpose for
the GEMM), so no re-layout pass runs per call; the gate and up weights are
packed once, in the constructor, into the [2*ffn, hidden] operand of the
fused SwiGLU GEMM (32-row groups of 16 gate and 16 up rows).  All buffers are
allocated once in the constructor; ``forward`` launches only.
"""
from __future__ import annotations

import math

from . import backend as B

ADD = B.EW["Add"]  # TargetElementwiseOperation::Add

class DecoderLayer:
    """One decoder layer on one GPU, bf16 or f16 weights resident in HBM."""

    def __init__(self, hip: "B.Context", weights: dict, tokens: int, hidden: int = 4096,
                 q_heads: int = 32, kv_heads: int = 8, head_dim: int = 128, ffn: int = 14336,
                 eps: float = 1e-5, theta: float = 1e4, dtype=None):
        import torch

        dt = torch.bfloat16 if dtype is None else dtype
        if dt not in (torch.bfloat16, torch.float16):
            raise ValueError("DecoderLayer: dtype must be torch.bfloat16 or torch.float16")
        self.dtype = dt
        self.fmt = B.BF16 if dt == torch.bfloat16 else B.F16

        self.hip, self.T, self.hidden = hip, tokens, hidden
        self.Hq, self.Hkv, self.D, self.ffn = q_heads, kv_heads, head_dim, ffn
        self.eps, self.theta = eps, theta
        if q_heads * head_dim != hidden:
            raise ValueError("q_heads * head_dim must equal hidden")
        if ffn % 32:
            raise ValueError("ffn must be a multiple of 32 (gate/up packing)")
        dev = torch.device("cuda", hip.device)

        def w(name, shape):
            t = weights[name]
            if tuple(t.shape) != shape or t.dtype != dt or t.device != dev:
                raise ValueError(f"weight {name}: expected {dt} {shape} on {dev}, got {t.dtype} {tuple(t.shape)}")
            return t.contiguous()

        qkv_n = (q_heads + 2 * kv_heads) * head_dim
        self.w_in = w("input_norm", (hidden,))
        self.w_post = w("post_norm", (hidden,))
        self.wqkv = w("wqkv", (qkv_n, hidden))
        self.wo = w("wo", (hidden, hidden))
        self.wg = w("wgate", (ffn, hidden))
        self.wu = w("wup", (ffn, hidden))
        self.wd = w("wdown", (hidden, ffn))
        self.wgu = torch.empty((2 * ffn, hidden), dtype=dt, device=dev)
        hip.interleave_gate_up(self.wg, self.wu, self.wgu)

        T = tokens
        e = lambda *s: torch.empty(s, dtype=dt, device=dev)
        self.h = e(T, hidden)
        self.qkv = e(T, qkv_n)
        # Q and K head-major in one buffer: one permute+RoPE call over their
        # Hq + Hkv heads, which sit side by side in each QKV row
        self.qk = e(q_heads + kv_heads, T, head_dim)
        self.q, self.k = self.qk[:q_heads], self.qk[q_heads:]
        self.attn = e(T, hidden)
        # [1, heads, T, D] views: V inside the QKV rows, O inside the token-major attention rows
        self.v_view = self.qkv[:, (q_heads + kv_heads) * head_dim:].view(T, kv_heads, head_dim).permute(1, 0, 2)[None]
        self.attn_view = self.attn.view(T, q_heads, head_dim).permute(1, 0, 2)[None]
        self.proj = e(T, hidden)
        self.x1 = e(T, hidden)
        self.act = e(T, ffn)
        self.pos = torch.arange(T, dtype=torch.int32, device=dev)

    def forward(self, x, y):
        """x, y: [tokens, hidden] device tensors of the layer's dtype (y may
        not alias x)."""
        hip, T, Hd, D = self.hip, self.T, self.hidden, self.D
        Hq, Hkv, F, fmt = self.Hq, self.Hkv, self.ffn, self.fmt
        qkv_n = self.qkv.shape[1]
        hip.rmsnorm(x, self.w_in, self.h, self.eps, fmt=fmt)
        hip.gemm_mfma(self.h, self.wqkv, self.qkv, T, Hd, qkv_n, in_fmt=fmt, out_fmt=fmt, rhs_t=True)
        hip.head_permute_rope(self.qkv, self.qk, T, Hq + Hkv, D, qkv_n, self.pos, self.theta, fmt=fmt)
        # V read in place from the QKV rows and O written token-major: head
        # slices addressed by strides, no re-layout steps
        hip.attention_prefill_strided(self.q.view(1, Hq, T, D), self.k.view(1, Hkv, T, D), self.v_view,
                                      self.attn_view, 1.0 / math.sqrt(D), causal=True, fmt=fmt)
        hip.gemm_mfma(self.attn, self.wo, self.proj, T, Hd, Hd, in_fmt=fmt, out_fmt=fmt, rhs_t=True)
        hip.add_rmsnorm(x, self.proj, self.w_post, self.x1, self.h, self.eps, fmt=fmt)
        hip.gemm_mfma_swiglu(self.h, self.wgu, self.act, T, Hd, F, in_fmt=fmt)
        hip.gemm_mfma_residual(self.act, self.wd, self.x1, y, T, F, Hd, in_fmt=fmt, rhs_t=True)
        return y


def flops(tokens: int = 1024, hidden: int = 4096, q_heads: int = 32, kv_heads: int = 8, head_dim: int = 128,
          ffn: int = 14336) -> int:
    """Algorithmic FLOPs of one layer: 2*T*(weights) for the projections plus
    4*Hq*D*(causal visible pairs) for attention."""
    weights = hidden * (q_heads + 2 * kv_heads) * head_dim + hidden * hidden + 3 * hidden * ffn
    return 2 * tokens * weights + 4 * q_heads * head_dim * (tokens * (tokens + 1) // 2)


def random_weights(torch, gen, hidden=4096, q_heads=32, kv_heads=8, head_dim=128, ffn=14336, std=0.02,
                   dtype=None):
    """~N(0, std) weights (bf16 unless dtype says otherwise) in the layout
    DecoderLayer takes; norm weights 1."""
    dev = gen.device
    dt = torch.bfloat16 if dtype is None else dtype
    r = lambda *s: (torch.randn(s, device=dev, generator=gen) * std).to(dt)
    return {
        "input_norm": torch.ones(hidden, dtype=dt, device=dev),
        "post_norm": torch.ones(hidden, dtype=dt, device=dev),
        "wqkv": r((q_heads + 2 * kv_heads) * head_dim, hidden),
        "wo": r(hidden, hidden),
        "wgate": r(ffn, hidden),
        "wup": r(ffn, hidden),
        "wdown": r(hidden, ffn),
    }
