"""Pins the oracle's masked FA prefill (oracle_attention_prefill_ex) before it
checks the HIP kernels.

Checks: the reference's own score-rounding corpus
(test/Board/Support/wafer_target_model_source_runner.py:85-99) bit for bit;
every mask case of the reference's attention board cases
(test/Board/PyTorch/wafer_pytorch_board_cases.py:937-1130, 1478-1516) against
a float64 closed form of SDPA with the same mask (rows with no visible key
give 0, as validate_fully_masked requires) under the reference's attention
policy; and structural identities that hold bit for bit (a boolean mask is an
additive 0/-inf mask, a causal diagonal is a triangular boolean mask, a
window is a band mask, a valid prefix never reads the tail, broadcast
strides equal the expanded mask).
"""
import math
import zlib

import numpy as np
import pytest

from tests.similarity import attention_gate, stats

F16, BF16 = 2, 3


def _store(oracle, fmt, x):
    x = np.asarray(x, np.float32)
    if fmt == BF16:
        return oracle.f32_to_bf16(x).reshape(x.shape)
    return x.astype(np.float16).view(np.uint16)


def _inputs(oracle, rng, fmt, Hq, Hkv, Sq, Skv, D, B=1):
    """The board cases' inputs: q and k are randn * 0.125, v is randn."""
    q = _store(oracle, fmt, rng.standard_normal((B, Hq, Sq, D)) * 0.125)
    k = _store(oracle, fmt, rng.standard_normal((B, Hkv, Skv, D)) * 0.125)
    v = _store(oracle, fmt, rng.standard_normal((B, Hkv, Skv, D)))
    return q, k, v


def sdpa64(q, k, v, scale, visible, bias=None, score_fn=None):
    """float64 SDPA: softmax over visible keys of q.k*scale (+ bias); a row
    with no visible key is 0.  visible / bias broadcast to [B, Hq, Sq, Skv]."""
    qf, kf, vf = (np.asarray(t, np.float64) for t in (q, k, v))
    g = qf.shape[1] // kf.shape[1]
    kf, vf = np.repeat(kf, g, axis=1), np.repeat(vf, g, axis=1)
    s = np.einsum("bhqd,bhkd->bhqk", qf, kf)
    s = score_fn(s) if score_fn else s * scale
    if bias is not None:
        s = s + np.asarray(bias, np.float64)
    vis = np.broadcast_to(visible, s.shape)
    s = np.where(vis, s, -np.inf)
    any_vis = vis.any(-1, keepdims=True)
    m = np.where(any_vis, np.max(np.where(vis, s, -np.inf), -1, keepdims=True), 0.0)
    p = np.where(vis, np.exp(s - m), 0.0)
    den = p.sum(-1, keepdims=True)
    p = np.where(any_vis, p / np.where(den == 0, 1, den), 0.0)
    return np.einsum("bhqk,bhkd->bhqd", p, vf)


def _f(oracle, fmt, a):
    return oracle.to_float(fmt, a).reshape(a.shape)


def test_score_region_rounding_corpus(oracle):
    """The reference's score-rounding program: f32(f16(f16(lhs*0.0883883461) +
    rhs)) over its (2, extent, 64) corpus, with rounding on both boundaries;
    without the flags the region stays in f32."""
    shape = (2, 40, 64)
    values = np.arange(int(np.prod(shape)), dtype=np.int64).reshape(shape)
    lhs = ((values % 37) - 18).astype(np.float16) / np.float16(7)
    rhs = ((values % 17) - 8).astype(np.float16) / np.float16(19)
    scale = np.float32(0.0883883461)
    expected = ((lhs.astype(np.float32) * scale).astype(np.float16) + rhs).astype(np.float32)
    unrounded = lhs.astype(np.float32) * scale + rhs.astype(np.float32)
    assert np.any(expected != unrounded)  # the corpus distinguishes a lost cast
    got = oracle.attention_score(lhs.astype(np.float32), scale, rhs.astype(np.float32), round_scaled=True,
                                 round_biased=True, fmt=F16)
    assert np.array_equal(got.view(np.uint32), expected.ravel().view(np.uint32))
    plain = oracle.attention_score(lhs.astype(np.float32), scale, rhs.astype(np.float32), fmt=F16)
    assert np.array_equal(plain.view(np.uint32), unrounded.ravel().view(np.uint32))
    # BF16 storage narrows to bf16 on the same boundaries
    got_b = oracle.attention_score(lhs.astype(np.float32), scale, rhs.astype(np.float32), round_scaled=True,
                                   round_biased=True, fmt=BF16)
    sb = oracle.bf16_to_f32(oracle.f32_to_bf16((lhs.astype(np.float32) * scale).ravel()))
    exp_b = oracle.bf16_to_f32(oracle.f32_to_bf16(sb + rhs.astype(np.float32).ravel()))
    assert np.array_equal(got_b.view(np.uint32), exp_b.view(np.uint32))


def _band(Sq, Skv, diag, window=None):
    i = np.arange(Sq)[:, None]
    j = np.arange(Skv)[None, :]
    vis = j <= i + diag
    if window is not None:
        vis &= j > i + diag - window
    return vis


# (name, fmt, Hq, Hkv, Sq, Skv, valid, D, mode): the reference's case shapes
# (the GQA case at a CPU-sized extent; the GPU tests run it at 1024)
CASES = [
    ("attention-noncausal", F16, 1, 1, 1024, 33, None, 64, "none"),
    ("attention-noncausal-additive", BF16, 1, 1, 1024, 33, None, 64, "additive"),
    ("attention-padding", F16, 1, 1, 1024, 33, None, 64, "padding"),
    ("attention-valid-kv-prefix", BF16, 1, 1, 1025, 1031, 1024, 64, "causal"),
    ("attention-sliding-window", F16, 1, 1, 1025, 1031, None, 64, "sliding"),
    ("attention-causal-decode-two-tokens", F16, 1, 1, 2, 1026, None, 64, "lower-right"),
    ("attention-probability-rounding-1025", BF16, 2, 2, 1025, 33, None, 16, "none"),
    ("attention-gqa-tail", F16, 32, 8, 130, 130, None, 128, "causal"),
]


def _case(oracle, rng, fmt, Hq, Hkv, Sq, Skv, valid, D, mode):
    q, k, v = _inputs(oracle, rng, fmt, Hq, Hkv, Sq, Skv, D)
    L = Skv if valid is None else valid
    kw = dict(kv_len=L, fmt=fmt)
    bias = keep = None
    vis = np.ones((Sq, L), bool)
    if mode == "additive":
        bias = (rng.standard_normal((1, 1, Sq, L)) * 0.125).astype(np.float32)
        kw["bias"] = bias
    elif mode == "padding":
        keep = np.zeros((1, 1, 1, L), np.uint8)
        keep[..., :L - 7] = 1
        kw["keep"] = keep
        vis = np.broadcast_to(keep[0, 0].astype(bool), (Sq, L))
    elif mode == "causal":
        kw.update(causal=True, diagonal=0)
        vis = _band(Sq, L, 0)
    elif mode == "lower-right":
        kw.update(causal=True, diagonal=L - Sq)
        vis = _band(Sq, L, L - Sq)
    elif mode == "sliding":
        vis = _band(Sq, L, L - Sq, 64)  # key <= qpos and key > qpos - 64, qpos = i + L - Sq
        keep = vis[None, None].astype(np.uint8)
        kw["keep"] = keep
    return q, k, v, kw, vis, bias


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_masked_prefill_vs_float64(oracle, case):
    name, fmt, Hq, Hkv, Sq, Skv, valid, D, mode = case
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    q, k, v, kw, vis, bias = _case(oracle, rng, fmt, Hq, Hkv, Sq, Skv, valid, D, mode)
    scale = 1.0 / math.sqrt(D)
    o = oracle.attention_prefill_ex(q, k, v, scale, **kw)
    L = kw["kv_len"]
    ref = sdpa64(_f(oracle, fmt, q), _f(oracle, fmt, k)[:, :, :L], _f(oracle, fmt, v)[:, :, :L], scale,
                 vis[None, None], bias)
    attention_gate(_f(oracle, fmt, o), ref, what=name)


@pytest.mark.parametrize("fmt", [F16, BF16])
def test_fully_masked_rows_are_exact_zero(oracle, fmt):
    """attention-fully-masked: a boolean mask with no visible key gives +0
    exactly (validate_fully_masked); so does a causal diagonal left of every
    key, and so do exactly the rows of a partial one that see no key."""
    rng = np.random.default_rng(11)
    q, k, v = _inputs(oracle, rng, fmt, 1, 1, 1024, 33, 64)
    keep = np.zeros((1, 1, 1, 33), np.uint8)
    o = oracle.attention_prefill_ex(q, k, v, 0.125, keep=keep, fmt=fmt)
    assert not o.any()
    o = oracle.attention_prefill_ex(q, k, v, 0.125, causal=True, diagonal=-2000, fmt=fmt)
    assert not o.any()
    # partially masked: row i sees keys <= i - 5; rows 0..4 are exactly zero, the rest are not
    o = oracle.attention_prefill_ex(q, k, v, 0.125, causal=True, diagonal=-5, fmt=fmt)
    assert not o[:, :, :5].any() and o[:, :, 5:].any(axis=-1).all()


@pytest.mark.parametrize("fmt", [F16, BF16])
def test_mask_identities(oracle, fmt):
    rng = np.random.default_rng(12)
    B, Hq, Hkv, Sq, Skv, D = 2, 4, 2, 70, 90, 64
    q, k, v = _inputs(oracle, rng, fmt, Hq, Hkv, Sq, Skv, D, B=B)
    s = 0.125
    base = oracle.attention_prefill_ex(q, k, v, s, fmt=fmt)
    # an all-true boolean mask is no mask
    ones = np.ones((1, 1, 1, Skv), np.uint8)
    assert np.array_equal(oracle.attention_prefill_ex(q, k, v, s, keep=ones, fmt=fmt), base)
    # a boolean mask is the additive 0 / -inf mask, per batch / head / query row
    keep = (rng.random((B, Hq, Sq, Skv)) < 0.7).astype(np.uint8)
    add = np.where(keep.astype(bool), 0.0, -np.inf).astype(np.float32)
    assert np.array_equal(oracle.attention_prefill_ex(q, k, v, s, keep=keep, fmt=fmt),
                          oracle.attention_prefill_ex(q, k, v, s, bias=add, fmt=fmt))
    # causal diagonal d is the triangular boolean mask j <= i + d (top-left d = 0, lower-right d = Skv - Sq)
    for d in (-3, 0, 5, Skv - Sq):
        tri = _band(Sq, Skv, d)[None, None].astype(np.uint8)
        assert np.array_equal(oracle.attention_prefill_ex(q, k, v, s, causal=True, diagonal=d, fmt=fmt),
                              oracle.attention_prefill_ex(q, k, v, s, keep=tri, fmt=fmt)), d
    # a window is the band i + d - w < j <= i + d
    for d, w in ((Skv - Sq, 64), (0, 1), (7, 16)):
        band = _band(Sq, Skv, d, w)[None, None].astype(np.uint8)
        assert np.array_equal(oracle.attention_prefill_ex(q, k, v, s, causal=True, diagonal=d, window=w, fmt=fmt),
                              oracle.attention_prefill_ex(q, k, v, s, keep=band, fmt=fmt)), (d, w)
    # broadcast strides equal the expanded mask
    bias = (rng.standard_normal((1, Hq, 1, Skv)) * 0.5).astype(np.float32)
    full = np.ascontiguousarray(np.broadcast_to(bias, (B, Hq, Sq, Skv)))
    assert np.array_equal(oracle.attention_prefill_ex(q, k, v, s, bias=bias, fmt=fmt),
                          oracle.attention_prefill_ex(q, k, v, s, bias=full, fmt=fmt))
    # a valid prefix never reads the tail: NaN there changes nothing
    L = 61
    kt, vt = k.copy(), v.copy()
    kt[:, :, L:] = 0x7E00 if fmt == F16 else 0x7FC0
    vt[:, :, L:] = kt[:, :, L:]
    sliced = oracle.attention_prefill_ex(q, np.ascontiguousarray(k[:, :, :L]), np.ascontiguousarray(v[:, :, :L]), s,
                                         causal=True, diagonal=L - Sq, fmt=fmt)
    assert np.array_equal(oracle.attention_prefill_ex(q, kt, vt, s, kv_len=L, causal=True, diagonal=L - Sq, fmt=fmt),
                          sliced)
    # the legacy causal entry is diagonal 0 on the same kernel walk
    assert np.array_equal(oracle.attention_prefill(q, k[:, :, :Sq], v[:, :, :Sq], s, causal=True, fmt=fmt),
                          oracle.attention_prefill_ex(q, np.ascontiguousarray(k[:, :, :Sq]),
                                                      np.ascontiguousarray(v[:, :, :Sq]), s, causal=True, fmt=fmt))


def test_score_rounding_flags_reach_the_scores(oracle):
    """Scores near 512 (where an f16 ulp is 0.5) make the
    rounding of the scaled score and of the biased score visible in the
    output: with the flags the oracle follows the float64 closed form over
    rounded scores and misses the unrounded one, and the other way round."""
    rng = np.random.default_rng(13)
    Sq, Skv, D = 48, 40, 64
    # scores 512 +- a few units: the common part q[:8].k[:8] = 512, the rest
    # small integers, so an f16 ulp (0.5 at 512) is a sizeable share of the
    # score differences
    qi = rng.integers(-1, 2, (1, 1, Sq, D))
    ki = rng.integers(-1, 2, (1, 1, Skv, D))
    qi[..., :8] = 8
    ki[..., :8] = 8
    q, k = _store(oracle, F16, qi), _store(oracle, F16, ki)
    v = _store(oracle, F16, rng.standard_normal((1, 1, Skv, D)))
    scale = 1.0
    bias = (rng.standard_normal((1, 1, Sq, Skv)) * 0.3).astype(np.float32)
    qf, kf, vf = (_f(oracle, F16, t) for t in (q, k, v))

    def rounded(raw):
        t = (raw.astype(np.float32) * np.float32(scale)).astype(np.float16).astype(np.float32)
        return ((t + bias).astype(np.float16).astype(np.float64)) - bias  # sdpa64 adds bias back

    vis = np.ones((1, 1, Sq, Skv), bool)
    ref_r = sdpa64(qf, kf, vf, scale, vis, bias, score_fn=rounded)
    ref_u = sdpa64(qf, kf, vf, scale, vis, bias)
    o_r = _f(oracle, F16, oracle.attention_prefill_ex(q, k, v, scale, bias=bias, round_scaled=True, round_biased=True,
                                                      fmt=F16))
    o_u = _f(oracle, F16, oracle.attention_prefill_ex(q, k, v, scale, bias=bias, fmt=F16))
    attention_gate(o_r, ref_r, what="rounded")
    attention_gate(o_u, ref_u, what="unrounded")
    # each misses the other closed form by more than the policy allows
    assert stats(o_r, ref_u)[1] > 0.01 and stats(o_u, ref_r)[1] > 0.01


def _nan_bits(fmt):
    return 0x7E00 if fmt == F16 else 0x7FC0


@pytest.mark.parametrize("fmt", [F16, BF16])
@pytest.mark.parametrize("D", [16, 128])
def test_invisible_keys_are_excluded(oracle, fmt, D):
    """One rule for every invisible key (past the causal diagonal, outside a
    window, or masked by a boolean mask): it is excluded, whatever its score.
    A NaN K row therefore changes nothing for the queries that cannot see it
    (bit for bit against the same call with that row zeroed), and makes the
    output NaN exactly for the queries that can."""
    rng = np.random.default_rng(70 + D + fmt)
    Sq = Skv = 100
    j = 50
    q, k, v = _inputs(oracle, rng, fmt, 2, 1, Sq, Skv, D)
    kn, kz = k.copy(), k.copy()
    kn[:, :, j] = _nan_bits(fmt)
    kz[:, :, j] = 0
    s = 1.0 / math.sqrt(D)
    # causal: queries i < j cannot see key j
    a = oracle.attention_prefill_ex(q, kn, v, s, causal=True, fmt=fmt)
    b = oracle.attention_prefill_ex(q, kz, v, s, causal=True, fmt=fmt)
    assert np.array_equal(a[:, :, :j], b[:, :, :j])
    assert np.isnan(oracle.to_float(fmt, a[:, :, j:]).astype(np.float64)).all()
    # the legacy causal entry (the dedicated kernel's oracle) follows the same rule
    c = oracle.attention_prefill(q, kn, v, s, causal=True, block_k=64, fmt=fmt)
    assert np.array_equal(c[:, :, :j], oracle.attention_prefill(q, kz, v, s, causal=True, block_k=64, fmt=fmt)[:, :, :j])
    # a boolean mask hiding key j from every query: nothing changes anywhere
    keep = np.ones((1, 1, 1, Skv), np.uint8)
    keep[..., j] = 0
    assert np.array_equal(oracle.attention_prefill_ex(q, kn, v, s, keep=keep, fmt=fmt),
                          oracle.attention_prefill_ex(q, kz, v, s, keep=keep, fmt=fmt))
    # a window of 8 keys ending at the diagonal: only queries j..j+7 see key j
    a = oracle.attention_prefill_ex(q, kn, v, s, causal=True, window=8, fmt=fmt)
    b = oracle.attention_prefill_ex(q, kz, v, s, causal=True, window=8, fmt=fmt)
    rows = np.r_[0:j, j + 8:Sq]
    assert np.array_equal(a[:, :, rows], b[:, :, rows])
    assert np.isnan(oracle.to_float(fmt, a[:, :, j:j + 8]).astype(np.float64)).all()


@pytest.mark.parametrize("fmt", [F16, BF16])
def test_hugely_negative_visible_scores_keep_their_maximum(oracle, fmt):
    """A row whose every visible score is far below any float a reference
    floor could hold (an additive mask of -1e30 - 1e28 * j) normalises over
    those scores: softmax keeps only the maximum, so each output row is the
    V row of its largest visible score (narrowed), as the closed form says."""
    rng = np.random.default_rng(81 + fmt)
    Sq, Skv, D = 40, 70, 64
    q, k, v = _inputs(oracle, rng, fmt, 1, 1, Sq, Skv, D)
    bias = (-1e30 - 1e28 * rng.permutation(Skv)).astype(np.float32)[None, None, None, :]
    out = oracle.attention_prefill_ex(q, k, v, 0.125, bias=np.ascontiguousarray(np.broadcast_to(bias, (1, 1, Sq, Skv))),
                                      fmt=fmt)
    best = int(np.argmax(bias[0, 0, 0]))
    assert np.array_equal(out[0, 0], np.broadcast_to(v[0, 0, best], (Sq, D)))
