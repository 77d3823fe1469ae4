"""GPU parity for the reference's long attention board cases and its NCx
external-layout attention case (test/Board/PyTorch/wafer_pytorch_board_cases.py:
1073-1083 attention-prefill-llama-2-7b, 1486-1493 attention-prefill-28-heads-2048-ncx,
1494-1498 attention-prefill-28-heads-4096), FP16 and BF16 storage.

* Long shapes: every head against float32 softmax attention on the GPU, two
  sampled heads against the CPU oracle's FA (oracle_attention_prefill), both
  under the reference's attention policy plus rtol 0.006 / atol 0.008
  (tests/similarity.py).
* NCx: with --external-layout ncx the program's Q / K / V arrive, and its
  output leaves, in the NCx physical layout
  (lib/Wafer/Transforms/Tile/LayoutOptimization.cpp:2426-2492).  The
  inputs are packed to NCx by the CPU oracle's codec, unpacked on the GPU
  (wafer_hip_unpack), attended (wafer_hip_attention_prefill) and the output
  packed back to NCx (wafer_hip_pack).  The NCx output must equal, byte for
  byte, the oracle's NCx packing of the dense entry's output on the logical
  tensors.
"""
import math
import sys

import numpy as np
import pytest

from tests.similarity import attention_gate

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

F16, BF16 = 2, 3
NCX = 3


def say(*a):
    print("[gpu-long]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def hip():
    from vibe_compiler_amd import backend

    ctx = backend.Context(0)
    yield ctx
    ctx.close()


@pytest.fixture(scope="module")
def B():
    from vibe_compiler_amd import backend

    return backend


def back(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def tdt(fmt):
    return torch.bfloat16 if fmt == BF16 else torch.float16


def bits(t):
    return back(t.contiguous().view(torch.int16)).view(np.uint16)


def f32_attention_all_heads(q, k, v, scale, causal=True):
    """float32 softmax attention head by head on the GPU (no transposed bf16 bmm operands)."""
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    S = q.shape[2]
    mask = torch.ones((S, S), dtype=torch.bool, device="cuda").tril() if causal else None
    g = q.shape[1] // k.shape[1]
    for h in range(q.shape[1]):
        qf = q[0, h].float()
        kf = k[0, h // g].float().t().contiguous()
        s = torch.matmul(qf, kf) * scale
        if mask is not None:
            s = s.masked_fill(~mask, float("-inf"))
        out[0, h] = torch.matmul(torch.softmax(s, -1), v[0, h // g].float())
    return out


def check_long(hip, oracle, fmt, H, S, seed, heads=(0, -1)):
    D = 128
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q, k, v = (torch.randn((1, H, S, D), generator=gen, device="cuda").to(tdt(fmt)) for _ in range(3))
    scale = 1.0 / math.sqrt(D)
    o = torch.full_like(q, float("nan"))
    hip.attention_prefill(q, k, v, o, scale, causal=True, fmt=fmt)
    got = back(o.float())
    attention_gate(got, back(f32_attention_all_heads(q, k, v, scale)), what=f"{H}x{S} all heads vs torch f32")
    for h in heads:
        sel = slice(h, h + 1) if h >= 0 else slice(H - 1, H)
        qs, ks, vs = (bits(t[:, sel]) for t in (q, k, v))
        ref = oracle.attention_prefill(qs, ks, vs, scale, causal=True, block_k=64, fmt=fmt)
        attention_gate(got[:, sel], oracle.to_float(fmt, ref).reshape(ref.shape), what=f"{H}x{S} head {h} vs oracle")
    return q, k, v, o


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
def test_attention_prefill_llama_2_7b(hip, oracle, fmt):
    """attention-prefill-llama-2-7b: 32 heads x 4096 (max_position_embeddings)
    x 128, causal; FP16 is the case's configured dtype."""
    say("llama-2-7b prefill", fmt)
    check_long(hip, oracle, fmt, 32, 4096, 1073 + fmt)


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
def test_attention_prefill_28_heads_4096(hip, oracle, fmt):
    say("28 heads 4096", fmt)
    check_long(hip, oracle, fmt, 28, 4096, 1494 + fmt)


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
def test_attention_prefill_28_heads_2048_ncx(hip, B, oracle, fmt):
    say("28 heads 2048 ncx", fmt)
    H, S, D = 28, 2048, 128
    shape = [1, H, S, D]
    nbytes = B.physical_bytes(fmt, NCX, shape)
    rng = np.random.default_rng(1486 + fmt)

    def logical_bits(scale):
        x = (rng.standard_normal(shape) * scale).astype(np.float32)
        if fmt == BF16:
            return oracle.f32_to_bf16(x).reshape(shape)
        return x.astype(np.float16).view(np.uint16)

    q, k, v = logical_bits(1.0), logical_bits(1.0), logical_bits(1.0)
    template = np.zeros(nbytes, dtype=np.uint8)
    ncx_in = [oracle.pack(fmt, NCX, shape, t, template) for t in (q, k, v)]
    # the NCx program: unpack the external inputs, attend, pack the output
    dense = []
    for st in ncx_in:
        t = torch.empty(shape, dtype=tdt(fmt), device="cuda")
        hip.unpack(fmt, NCX, shape, torch.from_numpy(st).cuda(), t)
        dense.append(t)
    scale = 1.0 / math.sqrt(D)
    o = torch.empty(shape, dtype=tdt(fmt), device="cuda")
    hip.attention_prefill(dense[0], dense[1], dense[2], o, scale, causal=True, fmt=fmt)
    o_ncx = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    hip.pack(fmt, NCX, shape, o, o_ncx)
    got_ncx = back(o_ncx)
    # the dense entry on the logical tensors, packed by the oracle's codec
    qd, kd, vd = (torch.from_numpy(t.view(np.int16)).cuda().view(tdt(fmt)) for t in (q, k, v))
    od = torch.empty(shape, dtype=tdt(fmt), device="cuda")
    hip.attention_prefill(qd, kd, vd, od, scale, causal=True, fmt=fmt)
    ref_ncx = oracle.pack(fmt, NCX, shape, bits(od), template)
    assert np.array_equal(got_ncx, ref_ncx), "NCx output differs from the packed dense output"
    assert np.array_equal(bits(o), bits(od))
    # and the attention itself against the oracle on two heads
    for h in (0, H - 1):
        ref = oracle.attention_prefill(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1], scale, causal=True, block_k=64,
                                       fmt=fmt)
        out_h = oracle.unpack(fmt, NCX, shape, got_ncx).reshape(shape)[:, h:h + 1]
        attention_gate(oracle.to_float(fmt, out_h).reshape(out_h.shape), oracle.to_float(fmt, ref).reshape(ref.shape),
                       what=f"ncx head {h} vs oracle")
