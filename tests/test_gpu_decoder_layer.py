"""GPU tests of the decoder-layer composite and of the
token-major <-> head-major re-layout it uses.

The re-layout is bit-exact against torch's permute.  The layer is checked
against a plain float32 torch evaluation of the same layer (the math of the
reference's CPU decoder-block reference,
test/Tools/Inputs/wafer_pytorch_xla_capture.py:1183-1260) on the same bf16
weights and input.  The backend stores every intermediate in bf16 while the
reference keeps float32 throughout, so the bound is a tolerance:

  at BASELINE config 4, the attention policy (cosine >= 0.9999, relative
  L2 <= 0.01) on the layer's update d = y - x (the residual stream itself
  would hide errors) and on y;
  on the small T=256, hidden-1024 layer, whose update has fewer terms per
  output and so a larger relative share of bf16 storage rounding: cosine >=
  0.9998 and relative L2 <= 0.02 on the update, relative L2 <= 0.01 on y.
Measured: T=256 small layer cos 0.99993 / relL2 0.012 (update), 0.0026 (y);
BASELINE config 4 cos 0.99998 / relL2 0.0062 (update), 0.0057 (y).

The layer is also composed from the CPU oracle's regions (formal-order bf16
GEMMs, RMSNorm, RoPE, online-softmax attention with 64-key blocks, SiLU-mul,
managed Add), which round every intermediate to bf16 where the backend does,
and the backend's output on sampled tokens is held to the attention gate
against it (test_decoder_layer_vs_oracle_composition).
"""
import math

import pytest

from tests.decoder_reference import reference_layer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from vibe_compiler_amd import backend

    ctx = backend.Context(0)
    yield ctx
    ctx.close()


@pytest.fixture(scope="module")
def torch():
    import torch

    return torch


# ------------------------------------------------------ head permute + RoPE
@pytest.mark.parametrize("tokens,heads,head_dim,stride,offset,fmt", [
    (1024, 32, 128, 6144, 0, "bf16"),      # the layer's Q
    (1024, 8, 128, 6144, 4096, "bf16"),    # the layer's K
    (1024, 40, 128, 6144, 0, "bf16"),      # the layer's Q and K together (head groups of 8)
    (77, 3, 64, 200, 8, "bf16"),           # ragged: odd tokens and heads, head groups of 1
    (300, 6, 32, 192, 0, "f16"),
    (64, 5, 16, 96, 16, "f32"),
    (64, 3, 256, 800, 0, "bf16"),         # head_dim above 128: the per-thread kernel
])
def test_head_permute_rope_bit_exact(hip, torch, tokens, heads, head_dim, stride, offset, fmt):
    """The fused kernel against head_permute followed by rope, bit for bit
    (the same rotation expressions; only the cos/sin sharing differs)."""
    from vibe_compiler_amd import backend as B

    F, dt = {"bf16": (B.BF16, torch.bfloat16), "f16": (B.F16, torch.float16), "f32": (B.F32, torch.float32)}[fmt]
    gen = torch.Generator(device="cuda").manual_seed(tokens * 31 + heads)
    src = torch.randn(tokens * stride + offset, generator=gen, device="cuda").to(dt)
    pos = (torch.randperm(4 * tokens, generator=gen, device="cuda")[:tokens]).to(torch.int32)
    ref = torch.empty(heads, tokens, head_dim, dtype=dt, device="cuda")
    hip.head_permute(src, ref, tokens, heads, head_dim, stride, 0, fmt=F, src_offset=offset)
    hip.rope(ref.view(heads * tokens, 1, head_dim), ref.view(heads * tokens, 1, head_dim), pos.repeat(heads),
             1e4, fmt=F)
    out = torch.full((heads * tokens * head_dim + 32,), 7.0, dtype=dt, device="cuda")
    hip.head_permute_rope(src, out, tokens, heads, head_dim, stride, pos, 1e4, fmt=F, src_offset=offset)
    torch.cuda.synchronize()
    got = out[: heads * tokens * head_dim].view(heads, tokens, head_dim)
    iv = torch.int32 if fmt == "f32" else torch.int16
    assert torch.equal(got.view(iv), ref.view(iv))
    assert torch.all(out[heads * tokens * head_dim:] == 7.0)


# ------------------------------------------------------------- head permute
@pytest.mark.parametrize("fmt_name,T,H,D,extra", [("BF16", 256, 8, 128, 0), ("BF16", 64, 3, 64, 256),
                                                  ("F32", 32, 4, 128, 64), ("F16", 16, 2, 8, 8)])
def test_head_permute_bit_exact(hip, torch, fmt_name, T, H, D, extra):
    from vibe_compiler_amd import backend as B

    fmt = getattr(B, fmt_name)
    dt = {"BF16": torch.bfloat16, "F32": torch.float32, "F16": torch.float16}[fmt_name]
    stride = H * D + extra
    gen = torch.Generator(device="cuda").manual_seed(7)
    src = torch.randn((T, stride), device="cuda", generator=gen).to(dt)
    hm = torch.full((H, T, D), -1.0, device="cuda", dtype=dt)
    hip.head_permute(src, hm, T, H, D, stride, 0, fmt=fmt)
    want = src[:, :H * D].reshape(T, H, D).permute(1, 0, 2).contiguous()
    assert torch.equal(hm.view(torch.int16 if dt != torch.float32 else torch.int32),
                       want.view(torch.int16 if dt != torch.float32 else torch.int32))
    back = torch.zeros((T, stride), device="cuda", dtype=dt)
    hip.head_permute(hm, back, T, H, D, stride, 1, fmt=fmt)
    torch.cuda.synchronize()
    assert torch.equal(back[:, :H * D], src[:, :H * D])
    assert torch.count_nonzero(back[:, H * D:]) == 0  # padding columns untouched


def test_head_permute_rejects_bad_arguments(hip, torch):
    from vibe_compiler_amd import backend as B

    x = torch.zeros((4, 64), device="cuda", dtype=torch.bfloat16)
    y = torch.zeros((4, 64), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(B.WaferHipError):
        hip.head_permute(x, y, 4, 2, 32, 32, 0)      # token_stride < heads*head_dim
    with pytest.raises(B.WaferHipError):
        hip.head_permute(x, y, 4, 2, 4, 64, 0)       # head_dim of 8 bytes
    with pytest.raises(B.WaferHipError):
        hip.head_permute(x, y, 4, 2, 32, 64, 2)      # direction


# --------------------------------------------------------------- the layer
def stats(torch, got, ref):
    g, r = got.double().flatten(), ref.double().flatten()
    cos = (g @ r / (g.norm() * r.norm())).item()
    rel = ((g - r).norm() / r.norm()).item()
    return cos, rel


@pytest.mark.parametrize("T,Hd,Hq,Hkv,F", [(256, 1024, 8, 2, 2048),
                                            (1024, 4096, 32, 8, 14336)])
def test_decoder_layer_vs_torch_f32(hip, torch, T, Hd, Hq, Hkv, F):
    from vibe_compiler_amd import decoder_layer as DL

    print(f"decoder layer T={T} hidden={Hd} heads={Hq}/{Hkv} ffn={F}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20260803)
    W = DL.random_weights(torch, gen, hidden=Hd, q_heads=Hq, kv_heads=Hkv, head_dim=128, ffn=F)
    x = torch.randn((T, Hd), device="cuda", generator=gen).to(torch.bfloat16)
    layer = DL.DecoderLayer(hip, W, T, hidden=Hd, q_heads=Hq, kv_heads=Hkv, head_dim=128, ffn=F)
    y = torch.empty_like(x)
    layer.forward(x, y)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    ref = reference_layer(torch, x, W, 1e-5, 1e4, Hq, Hkv, 128)
    cos_d, rel_d = stats(torch, y.float() - x.float(), ref - x.float())
    _, rel_y = stats(torch, y.float(), ref)
    print(f"update cos {cos_d:.6f} relL2 {rel_d:.5f}; output relL2 {rel_y:.6f}", flush=True)
    if T == 1024:  # the attention policy
        assert cos_d >= 0.9999 and rel_d <= 0.01
    else:
        assert cos_d >= 0.9998 and rel_d <= 0.02
    assert rel_y <= 0.01
    # determinism: a second forward gives the same bits
    y2 = torch.empty_like(x)
    layer.forward(x, y2)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))



def test_decoder_layer_vs_oracle_composition(hip, torch, oracle):
    """BASELINE config 4 against the CPU oracle's composition of the same
    regions, on sampled tokens.  K and V are formed for every token (the
    sampled tokens attend to all earlier ones); Q, attention, the output
    projection, the residual Adds, RMSNorm and the SwiGLU FFN only for the
    sampled tokens.  Every intermediate is bf16, as in the backend, so the
    two differ only by accumulation order (MFMA vs k-order fma, tree vs
    sequential row sums) and FA's lazy rescale.  Gate: the reference's
    similarity acceptance (cosine >= 0.9999, relative L2 <= 0.01) on y and on
    the update y - x, and elementwise |y - y_oracle| <= 4 bf16 ulps at the
    largest |y_oracle| of the sample.  The policy's elementwise rtol 0.006
    cannot apply here: y = x1 + down is formed from bf16 values of the
    residual stream, which reach |x1| ~ 8 where one bf16 ulp is 2^-5, and a
    one-ulp difference in x1 survives into a y that cancellation has made
    small."""
    import numpy as np

    from tests.similarity import stats as sim_stats
    from vibe_compiler_amd import decoder_layer as DL

    T, Hd, Hq, Hkv, D, F = 1024, 4096, 32, 8, 128, 14336
    eps, theta = 1e-5, 1e4
    print("decoder layer vs oracle composition (config 4, sampled tokens)", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20260805)
    W = DL.random_weights(torch, gen, hidden=Hd, q_heads=Hq, kv_heads=Hkv, head_dim=D, ffn=F)
    x = torch.randn((T, Hd), device="cuda", generator=gen).to(torch.bfloat16)
    layer = DL.DecoderLayer(hip, W, T, hidden=Hd, q_heads=Hq, kv_heads=Hkv, head_dim=D, ffn=F)
    y = torch.empty_like(x)
    layer.forward(x, y)
    torch.cuda.synchronize()
    u16 = lambda t: t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    xb, yb = u16(x), u16(y)
    Wn = {k: u16(v) for k, v in W.items()}
    BF = oracle.BF16
    gemm = lambda a, w, n: oracle.gemm_formal(BF, BF, a, w, a.shape[0], a.shape[1], n,
                                              rhs_t=True).reshape(a.shape[0], n)
    h = oracle.rmsnorm(xb, Wn["input_norm"], eps)
    wqkv = Wn["wqkv"]
    kv = gemm(h, np.ascontiguousarray(wqkv[Hq * D:]), 2 * Hkv * D)
    pos = np.arange(T, dtype=np.int32)
    k = oracle.rope(np.ascontiguousarray(kv[:, :Hkv * D]).reshape(T, Hkv, D), pos, theta)
    v = np.ascontiguousarray(kv[:, Hkv * D:]).reshape(T, Hkv, D)
    idx = np.array([0, 1, 63, 64, 200, 511, 777, 1023])
    q = oracle.rope(gemm(np.ascontiguousarray(h[idx]), np.ascontiguousarray(wqkv[:Hq * D]), Hq * D)
                    .reshape(len(idx), Hq, D), idx.astype(np.int32), theta)
    o = np.zeros((len(idx), Hq, D), np.uint16)
    for i, t in enumerate(idx):
        kt = np.ascontiguousarray(k[:t + 1].transpose(1, 0, 2))[None]
        vt = np.ascontiguousarray(v[:t + 1].transpose(1, 0, 2))[None]
        o[i] = oracle.attention_prefill(q[i][None, :, None, :], kt, vt, 1.0 / math.sqrt(D),
                                        causal=False, block_k=64)[0, :, 0, :]
    add = 8  # TargetElementwiseOperation::Add
    x1 = oracle.elementwise(add, BF, np.ascontiguousarray(xb[idx]), gemm(o.reshape(len(idx), Hd), Wn["wo"], Hd))
    h2 = oracle.rmsnorm(x1, Wn["post_norm"], eps)
    act = oracle.silu_mul(gemm(h2, Wn["wgate"], F), gemm(h2, Wn["wup"], F))
    yo = oracle.elementwise(add, BF, x1, gemm(act, Wn["wdown"], Hd))
    got = oracle.bf16_to_f32(yb[idx]).reshape(len(idx), Hd).astype(np.float64)
    exp = oracle.bf16_to_f32(yo).reshape(len(idx), Hd).astype(np.float64)
    xf = oracle.bf16_to_f32(xb[idx]).reshape(len(idx), Hd).astype(np.float64)
    cos_d, rel_d, _ = sim_stats(got - xf, exp - xf)
    print(f"vs oracle: update cos {cos_d:.7f} relL2 {rel_d:.5f}", flush=True)
    cos_y, rel_y, mx = sim_stats(got, exp)
    print(f"vs oracle: y cos {cos_y:.7f} relL2 {rel_y:.5f} max|d| {mx:.4f}", flush=True)
    assert cos_y >= 0.9999 and rel_y <= 0.01
    assert cos_d >= 0.9999 and rel_d <= 0.01
    ulp = 2.0 ** (math.floor(math.log2(np.abs(exp).max())) - 7)
    assert mx <= 4 * ulp, (mx, ulp)


# ------------------------------------------- llama-2-7b-block, F16 and BF16
# test/Board/PyTorch/wafer_pytorch_board_cases.py:817-866 with the
# configuration test/Tools/Inputs/hf/llama-2-7b-block-config.json: hidden
# 4096, 32 query and 32 KV heads of 128, intermediate 11008, RMSNorm eps 1e-5,
# RoPE theta 1e4, float16 (the case also runs bfloat16, :817-829);
# hidden_states [1, 16, 4096] ~ N(0, 1) * 0.125; the HF comparison policy
# (:28-30): rtol 0.002, atol 0.004, cosine >= 0.9999, relative L2 <= 0.01
# (make_similarity_policy, test/Board/PyTorch/wafer_pytorch_board_common.py:
# 59-71).  Weights ~ N(0, 0.02) (the configuration's initializer_range), norm
# weights 1.
L2B = dict(T=16, Hd=4096, Hq=32, Hkv=32, D=128, F=11008, eps=1e-5, theta=1e4)
HF_RTOL, HF_ATOL = 0.002, 0.004
# storage format: (torch dtype name, oracle format, mantissa bits, smallest normal exponent)
L2B_FORMATS = {"f16": ("float16", 2, 10, -14), "bf16": ("bfloat16", 3, 7, -126)}


def llama_2_7b_block_inputs(torch, name="f16"):
    """Weights and input of the block in the named storage format, drawn on
    the CPU (seeded), so the same tensors can be formed without a GPU."""
    from vibe_compiler_amd import decoder_layer as DL

    c = L2B
    dt = getattr(torch, L2B_FORMATS[name][0])
    gen = torch.Generator().manual_seed(817)
    W = DL.random_weights(torch, gen, hidden=c["Hd"], q_heads=c["Hq"], kv_heads=c["Hkv"], head_dim=c["D"],
                          ffn=c["F"], dtype=dt)
    x = (torch.randn((c["T"], c["Hd"]), generator=gen) * 0.125).to(dt)
    return W, x


@pytest.fixture(scope="module", params=["f16", "bf16"])
def llama_2_7b_block(hip, torch, request):
    """(format name, weights, input, backend output, layer) of the block, run
    once per storage format."""
    from vibe_compiler_amd import decoder_layer as DL

    c = L2B
    name = request.param
    print(f"llama-2-7b-block {name} [1,16,4096]", flush=True)
    W, x = llama_2_7b_block_inputs(torch, name)
    W = {k: v.cuda() for k, v in W.items()}
    x = x.cuda()
    layer = DL.DecoderLayer(hip, W, c["T"], hidden=c["Hd"], q_heads=c["Hq"], kv_heads=c["Hkv"], head_dim=c["D"],
                            ffn=c["F"], eps=c["eps"], theta=c["theta"], dtype=x.dtype)
    y = torch.empty_like(x)
    layer.forward(x, y)
    torch.cuda.synchronize()
    y2 = torch.empty_like(x)
    layer.forward(x, y2)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "second forward differs"
    return name, W, x, y, layer


def hf_policy(actual, expected, what):
    """The HF comparison policy as the reference applies it: cosine >= 0.9999
    and relative L2 <= 0.01 decide; the elementwise rtol / atol count is a
    diagnostic (make_similarity_policy keeps rtol / atol for point
    diagnostics only).  Returns the count of elements outside rtol / atol."""
    import numpy as np

    from tests.similarity import stats as sim_stats

    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    cos, rel, mx = sim_stats(a, e)
    bad = int((np.abs(a - e) > HF_ATOL + HF_RTOL * np.abs(e)).sum())
    print(f"{what}: cos {cos:.7f} relL2 {rel:.6f} max|d| {mx:.5f} outside rtol/atol {bad}/{a.size}", flush=True)
    assert cos >= 0.9999 and rel <= 0.01, what
    return bad


def test_llama_2_7b_block_vs_oracle_composition(torch, oracle, llama_2_7b_block):
    """The block against the CPU oracle's composition of the same regions
    over all 16 tokens (formal-order GEMMs, RMSNorm, RoPE, online-softmax
    attention in 64-key blocks, SiLU-mul, managed Add; every intermediate
    rounded to the storage format where the backend rounds it): the HF policy
    on y and on the update y - x, every element within 4 ulps of the storage
    format at the largest |y|, and the down projection with its residual Add
    (fed the backend's own x1 and SwiGLU output) within one ulp of the
    product plus one of the sum.  The two sides differ only in accumulation
    order (MFMA against k-order); one-ulp differences in the early
    intermediates spread through the later GEMMs, so in F16 about 0.3 % of
    the outputs fall outside rtol 0.002 / atol 0.004 here (the oracle
    composition itself has about 1.5 % outside against Hugging Face's float16
    layer)."""
    import numpy as np

    from tests.similarity import stats as sim_stats

    name, W, x, y, layer = llama_2_7b_block
    _, FMT, MB, EMIN = L2B_FORMATS[name]
    c = L2B
    T, Hd, Hq, Hkv, D, F = c["T"], c["Hd"], c["Hq"], c["Hkv"], c["D"], c["F"]
    u16 = lambda t: t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    xb, yb = u16(x), u16(y)
    Wn = {k: u16(v) for k, v in W.items()}
    gemm = lambda a, w, n: oracle.gemm_formal(FMT, FMT, a, w, a.shape[0], a.shape[1], n,  # noqa: E731
                                              rhs_t=True).reshape(a.shape[0], n)
    h = oracle.rmsnorm(xb, Wn["input_norm"], c["eps"], fmt=FMT)
    qkv = gemm(h, Wn["wqkv"], (Hq + 2 * Hkv) * D)
    pos = np.arange(T, dtype=np.int32)
    q = oracle.rope(np.ascontiguousarray(qkv[:, :Hq * D]).reshape(T, Hq, D), pos, c["theta"], fmt=FMT)
    k = oracle.rope(np.ascontiguousarray(qkv[:, Hq * D:(Hq + Hkv) * D]).reshape(T, Hkv, D), pos, c["theta"],
                    fmt=FMT)
    v = np.ascontiguousarray(qkv[:, (Hq + Hkv) * D:]).reshape(T, Hkv, D)
    hm = lambda t: np.ascontiguousarray(t.reshape(T, -1, D).transpose(1, 0, 2))[None]  # noqa: E731
    o = oracle.attention_prefill(hm(q), hm(k), hm(v), 1.0 / math.sqrt(D), causal=True, block_k=64, fmt=FMT)
    o = np.ascontiguousarray(o[0].transpose(1, 0, 2)).reshape(T, Hq * D)
    add = 8  # TargetElementwiseOperation::Add
    x1 = oracle.elementwise(add, FMT, xb, gemm(o, Wn["wo"], Hd))
    h2 = oracle.rmsnorm(x1, Wn["post_norm"], c["eps"], fmt=FMT)
    act = oracle.silu_mul(gemm(h2, Wn["wgate"], F), gemm(h2, Wn["wup"], F), fmt=FMT)
    yo = oracle.elementwise(add, FMT, x1, gemm(act, Wn["wdown"], Hd))
    f = lambda b: oracle.to_float(FMT, b).reshape(b.shape).astype(np.float64)  # noqa: E731
    got, exp, xf = f(yb), f(yo), f(xb)
    hf_policy(got, exp, f"llama-2-7b-block {name} y vs oracle")
    cos_d, rel_d, _ = sim_stats(got - xf, exp - xf)
    print(f"update vs oracle: cos {cos_d:.7f} relL2 {rel_d:.6f}", flush=True)
    assert cos_d >= 0.9999 and rel_d <= 0.01
    ulp = lambda a: 2.0 ** (np.floor(np.log2(np.maximum(np.abs(a), 2.0 ** EMIN))) - MB)  # noqa: E731
    assert np.abs(got - exp).max() <= 4 * ulp(np.abs(exp).max())
    # the last GEMM and its residual Add on the backend's own inputs: at most
    # one ulp of the narrowed product (accumulation order) carried through
    # the Add's own rounding
    x1g, actg = u16(layer.x1), u16(layer.act)
    down = gemm(actg, Wn["wdown"], Hd)
    yl = f(oracle.elementwise(add, FMT, x1g, down))
    assert np.all(np.abs(got - yl) <= ulp(f(down)) + ulp(yl))


def test_llama_2_7b_block_vs_hugging_face(torch, llama_2_7b_block):
    """The block against the official Hugging Face LlamaDecoderLayer run as
    the board case runs it for its expected output (the case's dtype, eval,
    CPU), with the same weights and input: the HF policy on y and the
    cosine / relative-L2 acceptance on the update y - x.  Elementwise,
    against the float32 evaluation of the same layer, the backend has no
    more elements outside rtol 0.002 / atol 0.004 than Hugging Face's own
    output in the same dtype."""
    pytest.importorskip("transformers")
    import numpy as np

    from tests.decoder_reference import hf_layer
    from tests.similarity import stats as sim_stats

    name, W, x, y, _ = llama_2_7b_block
    c = L2B
    Wc = {k: v.cpu() for k, v in W.items()}
    ref = hf_layer(torch, x.cpu(), Wc, c["eps"], c["theta"], c["Hq"], c["Hkv"], c["D"], c["F"], x.dtype)
    assert ref.dtype == x.dtype and torch.isfinite(ref).all()
    got = y.float().cpu().numpy().astype(np.float64)
    exp = ref.float().numpy().astype(np.float64)
    xf = x.float().cpu().numpy().astype(np.float64)
    hf_policy(got, exp, f"llama-2-7b-block {name} y vs HF")
    cos_d, rel_d, _ = sim_stats(got - xf, exp - xf)
    print(f"update vs HF {name}: cos {cos_d:.7f} relL2 {rel_d:.6f}", flush=True)
    assert cos_d >= 0.9999 and rel_d <= 0.01
    f32 = reference_layer(torch, x.cpu(), Wc, c["eps"], c["theta"], c["Hq"], c["Hkv"], c["D"]).double().numpy()
    bad_gpu = hf_policy(got, f32, f"llama-2-7b-block {name} y vs float32 layer")
    bad_hf = hf_policy(exp, f32, f"HF {name} vs float32 layer")
    assert bad_gpu <= bad_hf, (bad_gpu, bad_hf)
