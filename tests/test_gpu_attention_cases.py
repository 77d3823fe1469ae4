"""GPU parity for the reference's own attention cases
(test/Board/PyTorch/wafer_pytorch_board_cases.py:937-1130, 1478-1516): FP16
and BF16 storage, head_dim 64 / 128 and the head_dim-16 probability-rounding
case, additive F32, boolean padding, fully-masked and sliding-window masks,
a valid-KV prefix, a lower-right causal decode, GQA, and the score-region
rounding flags, through wafer_hip_attention_prefill_masked and
wafer_hip_attention_prefill, against the CPU oracle's masked FA
(oracle_attention_prefill_ex) on identical inputs.

Tolerance: the reference's attention policy (cosine >= 0.9999, relative L2
<= 0.01) plus elementwise rtol 0.006 / atol 0.008; fully-masked rows exactly
+0; bit-exact where two calls run the same kernel walk over the same keys.
"""
import ctypes
import math
import sys
import zlib

import numpy as np
import pytest

from tests.similarity import attention_gate

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

F16, BF16 = 2, 3


def say(*a):
    print("[gpu-case]", *a, flush=True)
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


def u16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).cuda()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def back(t):
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def store(oracle, fmt, x):
    x = np.asarray(x, np.float32)
    if fmt == BF16:
        return oracle.f32_to_bf16(x).reshape(x.shape)
    return x.astype(np.float16).view(np.uint16)


def inputs(oracle, rng, fmt, Hq, Hkv, Sq, Skv, D, Bn=1):
    q = store(oracle, fmt, rng.standard_normal((Bn, Hq, Sq, D)) * 0.125)
    k = store(oracle, fmt, rng.standard_normal((Bn, Hkv, Skv, D)) * 0.125)
    v = store(oracle, fmt, rng.standard_normal((Bn, Hkv, Skv, D)))
    return q, k, v


def band(Sq, Skv, diag, window=None):
    i = np.arange(Sq)[:, None]
    j = np.arange(Skv)[None, :]
    vis = j <= i + diag
    if window is not None:
        vis &= j > i + diag - window
    return vis


def run_masked(hip, fmt, q, k, v, scale, **kw):
    Bn, Hq, Sq, D = q.shape
    o = torch.full((Bn, Hq, Sq, D), 0x7E00, dtype=torch.int16, device="cuda")
    dkw = dict(kw)
    for name in ("bias", "keep"):
        if dkw.get(name) is not None:
            dkw[name] = dev(dkw[name])
    hip.attention_prefill_masked(u16(q), u16(k), u16(v), o, scale, fmt=fmt, **dkw)
    return back(o)


def tof(oracle, fmt, a):
    return oracle.to_float(fmt, a).reshape(a.shape)


# (name, Hq, Hkv, Sq, Skv, valid, D, mode): the board cases at their own shapes
CASES = [
    ("attention-noncausal", 1, 1, 1024, 33, None, 64, "none"),
    ("attention-noncausal-additive", 1, 1, 1024, 33, None, 64, "additive"),
    ("attention-padding", 1, 1, 1024, 33, None, 64, "padding"),
    ("attention-valid-kv-prefix", 1, 1, 1025, 1031, 1024, 64, "causal"),
    ("attention-sliding-window", 1, 1, 1025, 1031, None, 64, "sliding"),
    ("attention-sliding-window-flags", 1, 1, 1025, 1031, None, 64, "window"),
    ("attention-causal-decode-two-tokens", 1, 1, 2, 1026, None, 64, "lower-right"),
    ("attention-probability-rounding-1024", 2, 2, 1024, 33, None, 16, "none"),
    ("attention-probability-rounding-1025", 2, 2, 1025, 33, None, 16, "none"),
    ("attention-probability-rounding-1031", 2, 2, 1031, 33, None, 16, "none"),
    ("attention-prefill", 1, 1, 1024, 1024, None, 64, "causal"),
    ("attention-prefill-tail-1025", 1, 1, 1025, 1025, None, 64, "causal"),
    ("attention-prefill-tail-1031", 1, 1, 1031, 1031, None, 64, "causal"),
    ("attention-gqa", 32, 8, 1024, 1024, None, 128, "causal"),
    ("attention-gqa-tail-1025", 32, 8, 1025, 1025, None, 128, "causal"),
]


def case_kwargs(rng, Sq, L, mode):
    kw = dict(kv_len=L)
    if mode == "additive":
        kw["bias"] = (rng.standard_normal((1, 1, Sq, L)) * 0.125).astype(np.float32)
    elif mode == "padding":
        keep = np.zeros((1, 1, 1, L), np.uint8)
        keep[..., :L - 7] = 1
        kw["keep"] = keep
    elif mode == "causal":
        kw.update(causal=True, diagonal=0)
    elif mode == "lower-right":
        kw.update(causal=True, diagonal=L - Sq)
    elif mode == "sliding":
        kw["keep"] = band(Sq, L, L - Sq, 64)[None, None].astype(np.uint8)
    elif mode == "window":
        kw.update(causal=True, diagonal=L - Sq, window=64)
    return kw


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_reference_attention_case(hip, oracle, case, fmt):
    name, Hq, Hkv, Sq, Skv, valid, D, mode = case
    say(name, "fmt", fmt)
    rng = np.random.default_rng(zlib.crc32(name.encode()) + fmt)
    q, k, v = inputs(oracle, rng, fmt, Hq, Hkv, Sq, Skv, D)
    L = Skv if valid is None else valid
    kw = case_kwargs(rng, Sq, L, mode)
    scale = 1.0 / math.sqrt(D)
    ref = oracle.attention_prefill_ex(q, k, v, scale, fmt=fmt, **kw)
    got = run_masked(hip, fmt, q, k, v, scale, **kw)
    attention_gate(tof(oracle, fmt, got), tof(oracle, fmt, ref), what=f"{name} masked")
    if mode in ("causal", "none") and valid is None:
        # the plain entry: head_dim 128 takes its own kernel, the rest the
        # masked kernels with the causal flag alone
        o = torch.full(q.shape, 0x7E00, dtype=torch.int16, device="cuda")
        hip.attention_prefill(u16(q), u16(k), u16(v), o, scale, causal=mode == "causal", fmt=fmt)
        attention_gate(tof(oracle, fmt, back(o)), tof(oracle, fmt, ref), what=f"{name} plain")


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("D", [128, 64, 16])
def test_fully_masked_is_exact_zero(hip, oracle, fmt, D):
    """attention-fully-masked (q 1024, kv 33): every output exactly +0; and a
    causal diagonal that hides the first rows' keys zeroes exactly those."""
    say("fully masked", fmt, D)
    rng = np.random.default_rng(21 + D)
    q, k, v = inputs(oracle, rng, fmt, 1, 1, 1024, 33, D)
    got = run_masked(hip, fmt, q, k, v, 0.125, keep=np.zeros((1, 1, 1, 33), np.uint8))
    assert not got.any()
    got = run_masked(hip, fmt, q, k, v, 0.125, causal=True, diagonal=-5)
    assert not got[:, :, :5].any() and got[:, :, 5:].any(axis=-1).all()
    ref = oracle.attention_prefill_ex(q, k, v, 0.125, causal=True, diagonal=-5, fmt=fmt)
    attention_gate(tof(oracle, fmt, got), tof(oracle, fmt, ref), what="diagonal -5")
    got = run_masked(hip, fmt, q, k, v, 0.125, causal=True, diagonal=-(1 << 40))
    assert not got.any()


@pytest.mark.parametrize("D", [128, 64, 32])
def test_general_operands_and_rounding(hip, oracle, D):
    """Per-(batch, head, query) additive mask, a per-batch boolean padding mask
    broadcast over heads and queries, GQA, batch 2, and both score-rounding
    flags on scores near 512 (an f16 ulp of 0.5: the rounding is visible)."""
    say("general operands", D)
    fmt = F16
    rng = np.random.default_rng(31 + D)
    Bn, Hq, Hkv, Sq, Skv = 2, 4, 2, 150, 140
    qi = rng.integers(-1, 2, (Bn, Hq, Sq, D))
    ki = rng.integers(-1, 2, (Bn, Hkv, Skv, D))
    qi[..., :8], ki[..., :8] = 8, 8
    q, k = store(oracle, fmt, qi), store(oracle, fmt, ki)
    v = store(oracle, fmt, rng.standard_normal((Bn, Hkv, Skv, D)))
    bias = (rng.standard_normal((Bn, Hq, Sq, Skv)) * 0.3).astype(np.float32)
    keep = np.ones((Bn, 1, 1, Skv), np.uint8)
    keep[0, ..., 100:] = 0
    keep[1, ..., :3] = 0
    for flags in (dict(), dict(round_scaled=True), dict(round_scaled=True, round_biased=True)):
        ref = oracle.attention_prefill_ex(q, k, v, 1.0, bias=bias, keep=keep, fmt=fmt, **flags)
        got = run_masked(hip, fmt, q, k, v, 1.0, bias=bias, keep=keep, **flags)
        attention_gate(tof(oracle, fmt, got), tof(oracle, fmt, ref), what=f"D{D} {flags}")
    # causal lower-right with a window and the bias, BF16
    qb, kb, vb = inputs(oracle, rng, BF16, Hq, Hkv, Sq, Skv, D, Bn=Bn)
    kw = dict(causal=True, diagonal=Skv - Sq, window=37, bias=bias)
    ref = oracle.attention_prefill_ex(qb, kb, vb, 0.2, fmt=BF16, **kw)
    got = run_masked(hip, BF16, qb, kb, vb, 0.2, **kw)
    attention_gate(tof(oracle, BF16, got), tof(oracle, BF16, ref), what=f"D{D} window")


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("D", [128, 64, 16])
def test_valid_prefix_never_reads_the_tail(hip, oracle, fmt, D):
    """K/V heads kv_capacity tokens apart with NaN past kv_len: the output is
    bit-identical to the same call on the contiguous valid prefix."""
    say("valid prefix", fmt, D)
    rng = np.random.default_rng(41 + D)
    Hq, Hkv, Sq, cap, L = 4, 2, 200, 300, 229
    q, k, v = inputs(oracle, rng, fmt, Hq, Hkv, Sq, cap, D)
    nan = 0x7E00 if fmt == F16 else 0x7FC0
    k[:, :, L:] = nan
    v[:, :, L:] = nan
    kw = dict(causal=True, diagonal=L - Sq)
    got = run_masked(hip, fmt, q, k, v, 0.09, kv_len=L, **kw)
    sliced = run_masked(hip, fmt, q, np.ascontiguousarray(k[:, :, :L]), np.ascontiguousarray(v[:, :, :L]), 0.09, **kw)
    assert np.array_equal(got, sliced)
    ref = oracle.attention_prefill_ex(q, k, v, 0.09, kv_len=L, fmt=fmt, **kw)
    attention_gate(tof(oracle, fmt, got), tof(oracle, fmt, ref), what="valid prefix")


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
def test_config1_shape_f16_and_masked_bf16(hip, oracle, fmt):
    """The headline shape [1, 16, 2048, 128] causal through the masked entry
    and through the plain entry (the dedicated head_dim-128 kernel, F16 and
    BF16), each against the oracle."""
    say("config-1 shape masked", fmt)
    rng = np.random.default_rng(51)
    q, k, v = inputs(oracle, rng, fmt, 16, 16, 2048, 2048, 128)
    scale = 1.0 / math.sqrt(128)
    ref = oracle.attention_prefill_ex(q, k, v, scale, causal=True, fmt=fmt)
    got = run_masked(hip, fmt, q, k, v, scale, causal=True)
    attention_gate(tof(oracle, fmt, got), tof(oracle, fmt, ref), what="config-1 masked")
    o = torch.full(q.shape, 0x7E00, dtype=torch.int16, device="cuda")
    hip.attention_prefill(u16(q), u16(k), u16(v), o, scale, causal=True, fmt=fmt)
    attention_gate(tof(oracle, fmt, back(o)), tof(oracle, fmt, ref), what="config-1 plain")


def test_diagonal_past_the_keys_is_noncausal(hip, oracle):
    """A causal diagonal at or beyond kv_len hides nothing: bit-identical to
    the non-causal call (same kernel, same key walk)."""
    rng = np.random.default_rng(61)
    for D in (128, 64, 16):
        q, k, v = inputs(oracle, rng, BF16, 2, 1, 130, 77, D)
        a = run_masked(hip, BF16, q, k, v, 0.1)
        b = run_masked(hip, BF16, q, k, v, 0.1, causal=True, diagonal=77)
        c = run_masked(hip, BF16, q, k, v, 0.1, causal=True, diagonal=1 << 40)
        assert np.array_equal(a, b) and np.array_equal(a, c), D


def test_masked_entry_rejects_bad_arguments(hip, B):
    t = torch.zeros(64 * 64, dtype=torch.int16, device="cuda").view(1, 1, 64, 64)
    L = hip._L

    def call(m, D=64, fmt=B.F16):
        src = torch.zeros(64 * D, dtype=torch.int16, device="cuda")
        dst = torch.zeros(64 * D, dtype=torch.int16, device="cuda")
        p = src.data_ptr()
        return L.wafer_hip_attention_prefill_masked(hip._bind(), fmt, p, p, p, dst.data_ptr(), 1, 1, 1, 64, 64, D,
                                                    0.1, ctypes.byref(m))

    ok = B.AttentionMask()
    assert call(ok) == 0
    hip.synchronize()
    bad = B.AttentionMask()
    bad.flags = 16
    assert call(bad) == -1
    bad = B.AttentionMask()
    bad.kv_capacity = 10  # < kv_len
    assert call(bad) == -1
    bad = B.AttentionMask()
    bad.flags = B.ATT_WINDOW
    bad.window = 0
    assert call(bad) == -1
    bad = B.AttentionMask()
    bad.bias_strides[1] = -1
    assert call(bad) == -1
    assert call(B.AttentionMask(), D=96) == -3
    assert call(B.AttentionMask(), fmt=B.F32) == -3
    with pytest.raises(ValueError):  # a mask that does not broadcast: caught before the C call
        hip.attention_prefill_masked(t, t, t, t, 0.1, fmt=B.F16, bias=torch.zeros(2, 1, 1, 64, device="cuda"))
    with pytest.raises(ValueError):
        hip.attention_prefill_masked(t, t, t, t, 0.1, fmt=B.F16, keep=torch.zeros(1, 1, 1, 63, device="cuda",
                                                                                    dtype=torch.uint8))
    with pytest.raises(ValueError):
        hip.attention_prefill_masked(t, t, t, t, 0.1, fmt=B.F16, bias=torch.zeros(1, 1, 1, 64, device="cuda",
                                                                                  dtype=torch.float16))


# ------------------------------------------------------------------ FD decode, F16 storage
@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("Bn,Hq,Hkv,L,cap,chunks", [
    (1, 32, 32, 1024, 1024, 16),     # attention-decode-kv-cache: Llama-2-7b, 1023 past + 1
    (1, 32, 32, 4095, 4096, 16),     # attention-decode-kv-cache-long-4096 (valid prefix of the cache)
    (2, 8, 2, 1000, 1024, 16), (3, 8, 1, 100, 128, 5), (1, 16, 4, 777, 800, 1),
    (64, 8, 4, 2048, 2048, 16), (48, 16, 8, 600, 600, 4), (64, 4, 2, 513, 513, 16), (64, 4, 4, 300, 300, 3),
])
def test_fd_decode_storage_formats(hip, oracle, fmt, Bn, Hq, Hkv, L, cap, chunks):
    """FD on both storage formats: the chunk grid (small batch*kv_heads) and
    the one-workgroup-per-(batch, kv head) path (large), GQA 1..8, ragged
    chunks, a valid prefix of a larger cache; against the oracle's FD."""
    say("fd decode", fmt, Bn, Hq, Hkv, L, cap, chunks)
    rng = np.random.default_rng(L + chunks + fmt)
    D = 128
    q = store(oracle, fmt, rng.standard_normal((Bn, Hq, 1, D)) * 0.125)
    k = store(oracle, fmt, rng.standard_normal((Bn, Hkv, cap, D)) * 0.125)
    v = store(oracle, fmt, rng.standard_normal((Bn, Hkv, cap, D)))
    scale = 1.0 / math.sqrt(D)
    ref = oracle.attention_decode(q, k, v, scale, chunks=chunks, kv_len=L, block_k=64, fmt=fmt)
    o = torch.full((Bn, Hq, 1, D), 0x7E00, dtype=torch.int16, device="cuda")
    hip.attention_decode(u16(q), u16(k), u16(v), o, scale, chunks=chunks, kv_len=L, fmt=fmt)
    got = back(o)
    attention_gate(tof(oracle, fmt, got), tof(oracle, fmt, ref), what="FD")
    o2 = torch.full((Bn, Hq, 1, D), 0x7E00, dtype=torch.int16, device="cuda")
    hip.attention_decode_noalloc(u16(q), u16(k), u16(v), o2, scale, chunks=chunks, kv_len=L, fmt=fmt)
    assert np.array_equal(back(o2), got)


# ---------------------------------------------------------------- strided FA
@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("Bn,Hq,Hkv,S,causal", [(1, 32, 8, 1024, True), (2, 4, 2, 300, True), (1, 2, 1, 130, False),
                                                 (1, 32, 32, 16, True)])
def test_strided_prefill_equals_dense(hip, B, oracle, fmt, Bn, Hq, Hkv, S, causal):
    """wafer_hip_attention_prefill_strided on head slices of token-major
    projection rows (Q, K, V inside one [B, S, (Hq + 2 Hkv) 128] buffer, O
    written into token-major [B, S, Hq 128] rows) gives the bits of the dense
    entry on the re-laid-out tensors (same kernel walk); the first head
    against the oracle."""
    say("strided prefill", fmt, Bn, Hq, Hkv, S, causal)
    D = 128
    dt = torch.bfloat16 if fmt == BF16 else torch.float16
    gen = torch.Generator(device="cuda").manual_seed(Bn * 1000 + Hq * 10 + S)
    n = (Hq + 2 * Hkv) * D
    qkv = torch.randn(Bn, S, n, generator=gen, device="cuda").to(dt)
    qv = qkv[:, :, :Hq * D].view(Bn, S, Hq, D).permute(0, 2, 1, 3)
    kv_ = qkv[:, :, Hq * D:(Hq + Hkv) * D].view(Bn, S, Hkv, D).permute(0, 2, 1, 3)
    vv = qkv[:, :, (Hq + Hkv) * D:].view(Bn, S, Hkv, D).permute(0, 2, 1, 3)
    out = torch.full((Bn, S, Hq * D + 8), 5.0, dtype=dt, device="cuda")  # padded rows
    ov = out[:, :, :Hq * D].view(Bn, S, Hq, D).permute(0, 2, 1, 3)
    scale = 1 / math.sqrt(D)
    hip.attention_prefill_strided(qv, kv_, vv, ov, scale, causal=causal, fmt=fmt)
    od = torch.empty(Bn, Hq, S, D, dtype=dt, device="cuda")
    hip.attention_prefill(qv.contiguous(), kv_.contiguous(), vv.contiguous(), od, scale, causal=causal, fmt=fmt)
    torch.cuda.synchronize()
    assert torch.equal(ov.contiguous().view(torch.int16), od.view(torch.int16))
    assert torch.all(out[:, :, Hq * D:] == 5.0)  # the row padding is untouched
    bits = lambda t: back(t[:1, :1].contiguous().view(torch.int16))
    ref = oracle.attention_prefill(bits(qv), bits(kv_), bits(vv), scale, causal=causal, block_k=64, fmt=fmt)
    attention_gate(tof(oracle, fmt, bits(ov)), tof(oracle, fmt, ref), what="strided head 0")


def test_strided_prefill_rejections(hip, B):
    say("strided prefill rejections")
    D = 128
    q = torch.zeros(1, 2, 64, D, dtype=torch.bfloat16, device="cuda")
    q64 = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(B.WaferHipError) as e:  # head_dim 64: not served by this entry
        hip.attention_prefill_strided(q64, q64, q64, q64.clone(), 0.1)
    assert e.value.status == -3
    with pytest.raises(B.WaferHipError) as e:  # F32 storage
        hip.attention_prefill_strided(q, q, q, q.clone(), 0.1, fmt=B.F32)
    assert e.value.status == -3
    big = torch.zeros(64, 2 * D + 4, dtype=torch.bfloat16, device="cuda")  # row stride 260: not a multiple of 8
    v = big[:, :2 * D].view(64, 2, D).permute(1, 0, 2)[None]
    with pytest.raises(B.WaferHipError) as e:
        hip.attention_prefill_strided(q, q, v, q.clone(), 0.1)
    assert e.value.status == -1
    with pytest.raises(ValueError):  # head_dim must have unit stride
        hip.attention_prefill_strided(q, q, q.transpose(2, 3), q.clone(), 0.1)


# --------------------------------------------- invisible keys are excluded
@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("D", [16, 128])
def test_invisible_nan_key_is_excluded(hip, oracle, fmt, D):
    """A NaN K row at key j: queries that cannot see j (causal, window,
    boolean mask) give the bits of the same call with that row zeroed, and
    queries that can see it give NaN -- the oracle's rule, through the
    masked entry (fa_small at head_dim 16, fa_fwd at 128) and, at 128, the
    plain causal entry's dedicated kernel."""
    say("invisible NaN key", fmt, D)
    rng = np.random.default_rng(170 + D + fmt)
    Sq = Skv = 100
    j = 50
    nan = 0x7E00 if fmt == F16 else 0x7FC0
    q, k, v = inputs(oracle, rng, fmt, 2, 1, Sq, Skv, D)
    kn, kz = k.copy(), k.copy()
    kn[:, :, j] = nan
    kz[:, :, j] = 0
    s = 1.0 / math.sqrt(D)
    isnan = lambda a: np.isnan(tof(oracle, fmt, a).astype(np.float64))  # noqa: E731
    a = run_masked(hip, fmt, q, kn, v, s, causal=True)
    b = run_masked(hip, fmt, q, kz, v, s, causal=True)
    assert np.array_equal(a[:, :, :j], b[:, :, :j]) and isnan(a[:, :, j:]).all()
    ref = oracle.attention_prefill_ex(q, kn, v, s, causal=True, fmt=fmt)
    attention_gate(tof(oracle, fmt, a[:, :, :j]), tof(oracle, fmt, ref[:, :, :j]), what="causal, rows before the NaN key")
    if D == 128:  # the plain entry's dedicated kernel
        o1 = torch.full(q.shape, 0x7E00, dtype=torch.int16, device="cuda")
        o2 = torch.full(q.shape, 0x7E00, dtype=torch.int16, device="cuda")
        hip.attention_prefill(u16(q), u16(kn), u16(v), o1, s, causal=True, fmt=fmt)
        hip.attention_prefill(u16(q), u16(kz), u16(v), o2, s, causal=True, fmt=fmt)
        p1, p2 = back(o1), back(o2)
        assert np.array_equal(p1[:, :, :j], p2[:, :, :j]) and isnan(p1[:, :, j:]).all()
    keep = np.ones((1, 1, 1, Skv), np.uint8)
    keep[..., j] = 0
    assert np.array_equal(run_masked(hip, fmt, q, kn, v, s, keep=keep), run_masked(hip, fmt, q, kz, v, s, keep=keep))
    a = run_masked(hip, fmt, q, kn, v, s, causal=True, window=8)
    b = run_masked(hip, fmt, q, kz, v, s, causal=True, window=8)
    rows = np.r_[0:j, j + 8:Sq]
    assert np.array_equal(a[:, :, rows], b[:, :, rows]) and isnan(a[:, :, j:j + 8]).all()


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("D", [16, 64, 128])
def test_hugely_negative_visible_scores_keep_their_maximum(hip, oracle, fmt, D):
    """Every visible score far below -1e29 (an additive mask of -1e30 -
    1e28 * j): softmax keeps only the maximum, so every output row is the V
    row of its largest visible score, bit for bit, as in the oracle."""
    say("hugely negative scores", fmt, D)
    rng = np.random.default_rng(181 + D + fmt)
    Sq, Skv = 40, 200
    q, k, v = inputs(oracle, rng, fmt, 1, 1, Sq, Skv, D)
    bias = np.ascontiguousarray(np.broadcast_to(
        (-1e30 - 1e28 * rng.permutation(Skv)).astype(np.float32)[None, None, None, :], (1, 1, Sq, Skv)))
    got = run_masked(hip, fmt, q, k, v, 0.125, bias=bias)
    best = int(np.argmax(bias[0, 0, 0]))
    assert np.array_equal(got[0, 0], np.broadcast_to(v[0, 0, best], (Sq, D)))
    assert np.array_equal(got, oracle.attention_prefill_ex(q, k, v, 0.125, bias=bias, fmt=fmt))
