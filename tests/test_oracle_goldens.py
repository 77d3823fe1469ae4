"""Pins the CPU oracle before it is trusted as the parity checker.

Each check is one of: a golden bit pattern from the reference's own unit
tests (tests/golden/reference_goldens.json), an independent closed form
(exact rational rounding, numpy's IEEE conversions, float64 math), an
invariant, or brute force on tiny inputs.
"""
import math
import struct
from fractions import Fraction

import numpy as np
import pytest

from tests.similarity import attention_gate


def h(s):
    return int(s, 16)


def f32(bits):
    return np.array([bits], dtype=np.uint32).view(np.float32)[0]


def bits32(x):
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


# ---------------------------------------------------------------- GEMM goldens
def test_gemm_fma_goldens(oracle, goldens):
    for case in goldens["gemm_fma"]:
        if "a_f32" in case:
            a, b = f32(h(case["a_f32"])), f32(h(case["b_f32"]))
        else:
            a = np.array([h(case["a_f16"])], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
            b = np.array([h(case["b_f16"])], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
        r = oracle.lib().oracle_gemm_fma(a, b, f32(h(case["acc_f32"])))
        assert bits32(r) == h(case["expect_f32"]), case["cite"]


def test_gemm_finalize_f16(oracle, goldens):
    for case in goldens["gemm_finalize_f16"]:
        out = oracle.gemm_formal(oracle.F32, oracle.F16, np.array([f32(h(case["acc_f32"]))], np.float32),
                                 np.array([1.0], np.float32), 1, 1, 1)
        assert int(out[0]) == h(case["expect_f16"]), case["cite"]


def test_gemm_2x2_f16(oracle, goldens):
    g = goldens["gemm_2x2_f16"]
    lhs = np.array([h(x) for x in g["lhs"]], np.uint16)
    rhs = np.array([h(x) for x in g["rhs"]], np.uint16)
    out = oracle.gemm_formal(oracle.F16, oracle.F16, lhs, rhs, 2, 2, 2)
    assert [int(x) for x in out] == [h(x) for x in g["expect"]]


def test_gemm_sub_ulp_partial_and_psum(oracle, goldens):
    g = goldens["gemm_sub_ulp_partial"]
    for case in g["cases"]:
        fmt = oracle.F16 if case["format"] == "f16" else oracle.BF16
        one, eps = h(case["one"]), h(case["epsilon"])
        lhs = np.array([one, eps, one, eps], np.uint16)
        rhs = np.array([one] * 4, np.uint16)
        out = oracle.gemm_formal(fmt, oracle.F32, lhs, rhs, 1, 2, 1, batch=2)
        assert [bits32(x) for x in out] == [h(case["expect_f32"])] * 2
    g = goldens["gemm_psum_cancellation"]
    for case in g["cases"]:
        fmt = oracle.F16 if case["format"] == "f16" else oracle.BF16
        one, eps = h(case["one"]), h(case["epsilon"])
        lhs = np.array([one, eps, one, eps], np.uint16)
        rhs = np.array([one] * 4, np.uint16)
        psum = np.array([f32(h(g["psum_f32"]))] * 2, np.float32)
        out = oracle.gemm_formal(fmt, fmt, lhs, rhs, 1, 2, 1, batch=2, psum=psum)
        assert [int(x) for x in out] == [eps, eps]


def test_gemm_batched_ncx_f32(oracle, goldens):
    g = goldens["gemm_batched_ncx_f32"]
    lhs = np.array([f32(h(x)) for x in g["lhs"]], np.float32)
    rhs = np.array([f32(h(x)) for x in g["rhs"]], np.float32)
    out = oracle.gemm_formal(oracle.F32, oracle.F32, lhs, rhs, 2, 2, 2, batch=2)
    assert [bits32(x) for x in out] == [h(x) for x in g["expect"]]
    # Through the NCx codec: pack, unpack, multiply, pack, unpack.
    shape = g["shape"]
    geo = oracle.geometry(oracle.F32, oracle.NCX, shape)
    st = oracle.pack(oracle.F32, oracle.NCX, shape, lhs, np.zeros(geo["physical_bytes"], np.uint8))
    assert np.array_equal(oracle.unpack(oracle.F32, oracle.NCX, shape, st).ravel(), lhs)


def test_gemm_orientation_and_bruteforce(oracle):
    rng = np.random.default_rng(7)
    for (m, k, n, batch) in [(3, 5, 4, 2), (1, 17, 1, 1), (7, 1, 3, 3)]:
        a = rng.integers(-8, 8, size=(batch, m, k)).astype(np.float32)
        b = rng.integers(-8, 8, size=(batch, k, n)).astype(np.float32)
        ref = np.einsum("bmk,bkn->bmn", a.astype(np.float64), b.astype(np.float64))
        out = oracle.gemm_formal(oracle.F32, oracle.F32, a, b, m, k, n, batch=batch)
        assert np.array_equal(out.reshape(batch, m, n), ref.astype(np.float32))
        at = np.ascontiguousarray(np.swapaxes(a, 1, 2))
        bt = np.ascontiguousarray(np.swapaxes(b, 1, 2))
        out2 = oracle.gemm_formal(oracle.F32, oracle.F32, at, bt, m, k, n, batch=batch, lhs_t=True, rhs_t=True)
        assert np.array_equal(out, out2)


def test_gemm_sequential_fma_order(oracle):
    """A chain where each step's single rounding is visible: the oracle must
    equal a step-by-step exact-rational fma chain."""
    rng = np.random.default_rng(3)
    a = rng.standard_normal(33).astype(np.float32)
    b = rng.standard_normal(33).astype(np.float32)
    acc = np.float32(0.0)
    for x, y in zip(a, b):
        exact = Fraction(float(x)) * Fraction(float(y)) + Fraction(float(acc))
        acc = np.float32(_round_fraction_to_f32(exact))
    out = oracle.gemm_formal(oracle.F32, oracle.F32, a.reshape(1, 33), b.reshape(33, 1), 1, 33, 1)
    assert bits32(out[0]) == bits32(acc)


def _round_fraction_to_f32(x: Fraction) -> float:
    """Correct RNE rounding of an exact rational to binary32."""
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = math.floor(math.log2(x.numerator) - math.log2(x.denominator))
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    q, r = divmod(x, ulp)
    if r > ulp / 2 or (r == ulp / 2 and q % 2 == 1):
        q += 1
    return sign * float(q * ulp)


# ------------------------------------------------------------- conversions
def _rne_bf16_exact(bits):
    x = f32(bits)
    if not np.isfinite(x):
        return None
    v = Fraction(float(x))
    sign = 0x8000 if (bits >> 31) else 0
    if v == 0:
        return sign
    a = abs(v)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 7)
    q, r = divmod(a, ulp)
    if r > ulp / 2 or (r == ulp / 2 and q % 2 == 1):
        q += 1
    out = float(q * ulp)
    return (struct.unpack("<I", struct.pack("<f", out))[0] >> 16) | sign


def test_bf16_samples_closed_form(oracle, goldens):
    for s in goldens["bf16_samples"]["input_f32"]:
        bits = h(s)
        assert int(oracle.lib().oracle_f32_to_bf16(f32(bits))) == _rne_bf16_exact(bits), s
    rng = np.random.default_rng(1)
    samples = rng.integers(0, 2**32, size=2000, dtype=np.uint64).astype(np.uint32)
    samples = samples[np.isfinite(samples.view(np.float32))]
    got = oracle.f32_to_bf16(samples.view(np.float32))
    for b, g in zip(samples[:300], got[:300]):
        assert int(g) == _rne_bf16_exact(int(b))
    for b, g in zip(samples, got):
        assert int(oracle.lib().oracle_f32_to_bf16(f32(int(b)))) == int(g)


def test_f16_exhaustive_and_stratified(oracle):
    # Exhaustive F16 -> F32 against numpy's IEEE widening.
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expect = allh.view(np.float16).astype(np.float32)
    f16_to_f32 = oracle.lib().oracle_f16_to_f32
    got = np.array([f16_to_f32(int(b)) for b in allh], dtype=np.float32)
    finite = ~np.isnan(expect)
    assert np.array_equal(got.view(np.uint32)[finite], expect.view(np.uint32)[finite])
    # F32 -> F16 RNE against numpy over a stratified sample (all exponents).
    rng = np.random.default_rng(2)
    exps = np.repeat(np.arange(0, 255, dtype=np.uint32), 64)
    mant = rng.integers(0, 2**23, size=exps.size, dtype=np.uint64).astype(np.uint32)
    sign = rng.integers(0, 2, size=exps.size, dtype=np.uint64).astype(np.uint32)
    bits = (sign << 31) | (exps << 23) | mant
    vals = bits.view(np.float32)
    out = oracle.convert(166, vals, oracle.F16)
    assert np.array_equal(out, vals.astype(np.float16).view(np.uint16))


def test_convert_goldens_and_int_routes(oracle, goldens):
    g = goldens["convert_f32_f16"]
    out = oracle.convert(166, np.array([f32(h(x)) for x in g["input_f32"]], np.float32), oracle.F16)
    assert [int(x) for x in out] == [h(x) for x in g["expect_f16"]]
    ints = np.array([0, 1, -1, 255, 257, 16777217, -16777219, 2**31 - 1, -2**31, 65519, 65520, 123456789],
                    dtype=np.int64)
    i32 = ints.astype(np.int32)
    # int32 -> f32: one RNE rounding, equal to float64 -> float32 of the exact integer.
    assert np.array_equal(oracle.convert(149, i32, oracle.F32), ints.astype(np.float64).astype(np.float32))
    # int32 -> bf16: one rounding straight from the exact integer.
    bf = oracle.convert(148, i32, oracle.BF16)
    for v, got in zip(ints, bf):
        expect = _rne_bf16_exact(bits32(np.float64(v))) if abs(int(v)) < 2**24 else None
        if expect is not None:
            assert int(got) == expect
        else:
            val = oracle.bf16_to_f32(np.array([got], np.uint16))[0]
            # nearest bf16 to the exact integer
            e = math.floor(math.log2(abs(int(v))))
            ulp = 2 ** (e - 7)
            assert abs(float(val) - int(v)) <= ulp / 2
    f16 = oracle.convert(147, i32[np.abs(ints) < 70000], oracle.F16)
    ref = ints[np.abs(ints) < 70000].astype(np.float64).astype(np.float16).view(np.uint16)
    assert np.array_equal(f16, ref)
    # float -> int nearest-even.
    fl = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 3.49, 1e9], np.float32)
    assert list(oracle.convert(165, fl, oracle.I32)) == [0, 2, 2, 0, -2, 3, 1000000000]


# ---------------------------------------------------------------- ExpLp
def test_explp_bound(oracle, goldens):
    L = oracle.lib()
    assert bits32(L.oracle_explp(float("-inf"))) == 0
    assert bits32(L.oracle_explp(0.0)) == 0x3F800000
    x = np.linspace(-80.0, 80.0, 4001, dtype=np.float32)
    out = oracle.elementwise(26, oracle.F32, x)
    expect = np.exp(x.astype(np.float64))
    assert np.all(np.abs(out - expect) <= expect * goldens["explp"]["relative_bound"])


# ---------------------------------------------------------------- elementwise
def test_elementwise_exact_ops(oracle):
    rng = np.random.default_rng(4)
    a = (rng.standard_normal(1000) * 4).astype(np.float32)
    b = (rng.standard_normal(1000) * 4).astype(np.float32)
    pos = np.abs(a) + np.float32(0.01)
    cases = {0: np.abs(a), 5: -a, 2: a * a, 6: np.fmax(a, b), 7: np.fmin(a, b), 8: a + b, 9: a - b,
             10: a * b, 31: np.where(a < 0, np.float32(0), a)}
    for op, expect in cases.items():
        got = oracle.elementwise(op, oracle.F32, a, b if op in (6, 7, 8, 9, 10) else None)
        assert np.array_equal(got, expect.astype(np.float32)), op
    assert np.array_equal(oracle.elementwise(1, oracle.F32, pos), (np.float32(1) / pos))
    assert np.array_equal(oracle.elementwise(3, oracle.F32, pos), np.sqrt(pos))
    assert np.array_equal(oracle.elementwise(4, oracle.F32, pos), np.float32(1) / np.sqrt(pos))
    # bf16 storage: computed in f32, one RNE narrowing (the Mul-by-one
    # identity of ManagedReferenceTargetModelTest.cpp:98-117).
    bb = oracle.f32_to_bf16(a)
    ones = np.full_like(bb, 0x3F80)
    assert np.array_equal(oracle.elementwise(10, oracle.BF16, bb, ones), bb)


def test_elementwise_transcendental(oracle):
    x = np.linspace(-6, 6, 2001, dtype=np.float32)
    xd = x.astype(np.float64)
    ref = {27: np.sin(xd), 28: np.cos(xd), 29: np.tanh(xd), 25: np.exp(xd), 24: np.exp2(xd),
           30: 1 / (1 + np.exp(-xd)), 34: np.log1p(np.exp(xd))}
    for op, r in ref.items():
        got = oracle.elementwise(op, oracle.F32, x).astype(np.float64)
        assert np.all(np.abs(got - r) <= 4e-7 * np.abs(r) + 1e-37 + 2e-7 * (op in (27, 28))), op
    pos = np.linspace(0.01, 100, 1001, dtype=np.float32)
    assert np.allclose(oracle.elementwise(22, oracle.F32, pos), np.log2(pos.astype(np.float64)), rtol=1e-6, atol=1e-6)
    assert np.allclose(oracle.elementwise(23, oracle.F32, pos), np.log(pos.astype(np.float64)), rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- reduce
def test_reduce_goldens(oracle, goldens):
    g = goldens["reduce_sum_ncx"]
    out = oracle.reduce(0, g["dim"], oracle.F32, g["shape"], np.array([f32(h(x)) for x in g["input"]], np.float32))
    assert [bits32(x) for x in out.ravel()] == [h(x) for x in g["expect"]]
    g = goldens["reduce_axes_tails"]
    for C in g["channels"]:
        hh, ww, cc = np.meshgrid(np.arange(2), np.arange(3), np.arange(C), indexing="ij")
        vals = (1 + hh * 3 + ww + cc % 5).astype(np.float32).reshape(1, 2, 3, C)
        for dim in g["dims"]:
            out = oracle.reduce(0, dim, oracle.F32, [1, 2, 3, C], vals)
            axes = {0: (3,), 1: (2,), 2: (1,), 4: (1, 2)}[dim]
            expect = vals.astype(np.float64).sum(axis=axes, keepdims=True)
            assert np.array_equal(out, expect.astype(np.float32)), (C, dim)
            if dim == 0:
                shape = [1, 2, 3, 1]
                geo = oracle.geometry(oracle.F32, oracle.NCX, shape)
                st = oracle.pack(oracle.F32, oracle.NCX, shape, out.ravel(), np.zeros(geo["physical_bytes"], np.uint8))
                assert bytes(st[4:8]) == b"\0\0\0\0"
                assert st[16:20].view(np.float32)[0] == out.ravel()[1]


def test_reduce_extrema_signed_zero(oracle):
    for fmt in (oracle.F32, oracle.BF16, oracle.F16):
        zero, negz = (np.array([0.0, -0.0], np.float32) if fmt == oracle.F32 else
                      (np.array([0, 0x8000], np.uint16)))
        src = np.array([negz, zero, negz, negz]).reshape(1, 1, 2, 2)
        mx = oracle.reduce(1, 0, fmt, [1, 1, 2, 2], src)
        mn = oracle.reduce(2, 0, fmt, [1, 1, 2, 2], src)
        sb = (lambda v: np.signbit(v)) if fmt == oracle.F32 else (lambda v: (v.astype(np.uint16) & 0x8000) != 0)
        assert list(sb(mx.ravel())) == [False, True]
        assert list(sb(mn.ravel())) == [True, True]


# ---------------------------------------------------------------- codec
def test_cx_tail_codec(oracle, goldens):
    g = goldens["cx_tail_codec"]
    geo = oracle.geometry(oracle.F16, oracle.CX, g["shape"])
    assert geo["physical_bytes"] > 2 * 3 * 2
    values = np.zeros(6, np.uint16)
    st = oracle.pack(oracle.F16, oracle.CX, g["shape"], values, np.full(geo["physical_bytes"], 0xA5, np.uint8))
    assert (st == 0xA5).any()
    assert np.array_equal(oracle.unpack(oracle.F16, oracle.CX, g["shape"], st).ravel(), values)


@pytest.mark.parametrize("fmt", [0, 2, 3, 5, 11])
@pytest.mark.parametrize("layout", [2, 3])
@pytest.mark.parametrize("shape", [[5], [3, 1], [2, 3, 33], [2, 65], [1, 2, 3, 1025], [2, 2, 130], [3, 96],
                                   [2, 1, 129], [1, 200]])
def test_codec_bijection_and_padding(oracle, fmt, layout, shape):
    """The blocked map is injective, stays inside the physical span, keeps
    every padding byte of the template, and round-trips."""
    geo = oracle.geometry(fmt, layout, shape)
    bits = geo["element_bits"]
    idx = np.indices(shape).reshape(len(shape), -1).T
    offs = [oracle.bit_offset(fmt, layout, shape, i) for i in idx]
    assert len(set(offs)) == len(offs)
    assert min(offs) >= 0 and max(offs) + bits <= geo["physical_bytes"] * 8
    assert geo["physical_bytes"] * 8 % 2048 == 0  # bank-line (256 B) aligned span
    rng = np.random.default_rng(len(shape))
    dt = oracle.storage_dtype(fmt) if fmt != 11 else np.int64
    logical = rng.integers(0, 120, size=len(offs)).astype(dt)
    template = rng.integers(0, 256, size=geo["physical_bytes"]).astype(np.uint8)
    st = oracle.pack(fmt, layout, shape, logical, template)
    owned = np.zeros(geo["physical_bytes"], bool)
    for o in offs:
        owned[o // 8: o // 8 + bits // 8] = True
    assert np.array_equal(st[~owned], template[~owned])
    assert np.array_equal(oracle.unpack(fmt, layout, shape, st).ravel(), logical)


def test_codec_block_structure(oracle):
    # f32 [1,2,3,1025] NCx: 16 full blocks of 64 then a tail of 4, outer 6,
    # slice stride aligned to 64 elements (256 B).
    geo = oracle.geometry(oracle.F32, oracle.NCX, [1, 2, 3, 1025])
    assert (geo["cx_blocks"], geo["c0"], geo["aligned_c"]) == (16, 4, 1028)
    assert geo["outer_slice_stride"] == 6208 and geo["physical_elements"] == 6208
    # int8 uses 128-channel blocks and keeps tails up to 64.
    g8 = oracle.geometry(oracle.I8, oracle.CX, [3, 200])
    assert (g8["c_block"], g8["cx_blocks"], g8["c0"]) == (128, 2, 0) and g8["aligned_c"] == 256
    g8b = oracle.geometry(oracle.I8, oracle.CX, [3, 160])
    assert (g8b["cx_blocks"], g8b["c0"]) == (1, 32)
    # channel c of outer row r in block-major order
    assert oracle.bit_offset(oracle.F16, oracle.CX, [3, 130], [1, 65]) == (1 * 3 * 64 + 1 * 64 + 1) * 16
    assert oracle.bit_offset(oracle.F16, oracle.CX, [3, 130], [2, 129]) == (2 * 3 * 64 + 2 * 4 + 1) * 16


# ---------------------------------------------------------------- int8 GEMM
def test_i8_gemm_closed_form(oracle):
    rng = np.random.default_rng(11)
    for (m, k, n) in [(5, 7, 3), (16, 64, 9), (33, 130, 17)]:
        a = rng.integers(-127, 128, size=(m, k), dtype=np.int64)
        b = rng.integers(-127, 128, size=(k, n), dtype=np.int64)
        scale = rng.uniform(0.001, 0.01, size=n).astype(np.float32)
        acc, y = oracle.gemm_i8(a.astype(np.int8), b.astype(np.int8), scale, m, k, n)
        ref = a @ b
        assert np.array_equal(acc, ref.astype(np.int32))
        f = ref.astype(np.float64).astype(np.float32) * scale
        assert np.array_equal(y, oracle.f32_to_bf16(f.astype(np.float32)))
        acc2, y2 = oracle.gemm_i8(a.astype(np.int8), np.ascontiguousarray(b.T).astype(np.int8), scale, m, k, n, rhs_t=True)
        assert np.array_equal(acc2, acc) and np.array_equal(y2, y)
    # extreme magnitude: K=4096 of 127*127 fits int32 and converts exactly
    a = np.full((2, 4096), 127, np.int8)
    b = np.full((4096, 3), -127, np.int8)
    acc, _ = oracle.gemm_i8(a, b, np.ones(3, np.float32), 2, 4096, 3)
    assert int(acc[0, 0]) == -4096 * 127 * 127


# ---------------------------------------------------------------- attention
def _ref_attention(q, k, v, scale, causal):
    qf, kf, vf = (t.astype(np.float64) for t in (q, k, v))
    B, Hq, Sq, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    kf = np.repeat(kf, g, axis=1)
    vf = np.repeat(vf, g, axis=1)
    s = np.einsum("bhqd,bhkd->bhqk", qf, kf) * scale
    if causal:
        mask = np.triu(np.ones((Sq, k.shape[2]), bool), 1)
        s = np.where(mask, -np.inf, s)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p, vf)


def _bf16_randn(rng, shape):
    from oracle.oracle import f32_to_bf16
    return f32_to_bf16(rng.standard_normal(shape).astype(np.float32)).reshape(shape)


def test_attention_prefill_vs_float64(oracle):
    rng = np.random.default_rng(5)
    for (B, Hq, Hkv, S, D, causal) in [(1, 2, 2, 70, 64, True), (2, 4, 2, 33, 128, False), (1, 4, 1, 128, 128, True)]:
        q, k, v = (_bf16_randn(rng, (B, h_, S, D)) for h_ in (Hq, Hkv, Hkv))
        scale = 1.0 / math.sqrt(D)
        o = oracle.attention_prefill(q, k, v, scale, causal=causal, block_k=32)
        ref = _ref_attention(*(oracle.bf16_to_f32(t).reshape(t.shape) for t in (q, k, v)), scale, causal)
        attention_gate(oracle.bf16_to_f32(o).reshape(o.shape), ref, what="oracle FA")


def test_attention_invariants(oracle):
    rng = np.random.default_rng(6)
    B, Hq, Hkv, S, D = 2, 4, 2, 96, 64
    q, k, v = (_bf16_randn(rng, (B, h_, S, D)) for h_ in (Hq, Hkv, Hkv))
    scale = 0.125
    # GQA equals MHA on repeated KV heads, bit for bit.
    o_gqa = oracle.attention_prefill(q, k, v, scale, block_k=32)
    o_mha = oracle.attention_prefill(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1), scale, block_k=32)
    assert np.array_equal(o_gqa, o_mha)
    # Block size changes rounding only.
    o64 = oracle.attention_prefill(q, k, v, scale, block_k=64)
    attention_gate(oracle.bf16_to_f32(o64), oracle.bf16_to_f32(o_gqa), what="block size")
    # FD with one chunk equals the non-causal FA of the same single query.
    qd = q[:, :, -1:, :]
    fd1 = oracle.attention_decode(qd, k, v, scale, chunks=1, block_k=32)
    fa = oracle.attention_prefill(qd, k, v, scale, causal=False, block_k=32)
    assert np.array_equal(fd1, fa)
    # FD with many chunks agrees within tolerance; empty trailing chunks are neutral.
    fd16 = oracle.attention_decode(qd, k, v, scale, chunks=16, block_k=32)
    attention_gate(oracle.bf16_to_f32(fd16), oracle.bf16_to_f32(fa), what="FD chunks")
    fd_many = oracle.attention_decode(qd[:, :, :, :], k[:, :, :3], v[:, :, :3], scale, chunks=8, block_k=32)
    fa3 = oracle.attention_prefill(qd, k[:, :, :3], v[:, :, :3], scale, causal=False, block_k=32)
    attention_gate(oracle.bf16_to_f32(fd_many), oracle.bf16_to_f32(fa3), what="FD empty chunks")


def test_attention_probability_rounding_point(oracle):
    """P is narrowed to bf16 before PV while l sums the unrounded P.
    Two keys, scores (0, x) with V rows (0, 1): out = bf16(p)/(1+p), with
    p = ExpLp(x).  x is chosen so that narrowing p changes the result."""
    L = oracle.lib()
    D = 64
    found = False
    for x in np.linspace(0.001, 0.05, 400, dtype=np.float32):
        p = np.float32(L.oracle_explp(float(x)))
        pb = oracle.bf16_to_f32(oracle.f32_to_bf16(np.array([p], np.float32)))[0]
        with_round = oracle.f32_to_bf16(np.array([np.float32(pb) * (np.float32(1) / (np.float32(1) + p))], np.float32))[0]
        no_round = oracle.f32_to_bf16(np.array([p * (np.float32(1) / (np.float32(1) + p))], np.float32))[0]
        if with_round != no_round:
            found = True
            break
    assert found
    # q = [x, 0...] with scale 1, keys e0*0 and e0*1 give scores 0 and x
    # only if x is bf16-representable; pick q[0] = bf16(x), k1[0] = 1.
    xb = oracle.f32_to_bf16(np.array([x], np.float32))
    xv = oracle.bf16_to_f32(xb)[0]
    p = np.float32(L.oracle_explp(float(xv)))
    pb = oracle.bf16_to_f32(oracle.f32_to_bf16(np.array([p], np.float32)))[0]
    q = np.zeros((1, 1, 1, D), np.uint16)
    q[..., 0] = xb[0]
    k = np.zeros((1, 1, 2, D), np.uint16)
    k[0, 0, 1, 0] = 0x3F80
    v = np.zeros((1, 1, 2, D), np.uint16)
    v[0, 0, 1, :] = 0x3F80
    o = oracle.attention_prefill(q, k, v, 1.0, causal=False, block_k=64)
    # m = xv (> 0), alpha... single block: e = xv; P = (ExpLp(-xv), 1); l = P0 + 1
    p0 = np.float32(L.oracle_explp(float(np.float32(0) - xv)))
    l = np.float32(p0 + np.float32(1))
    acc = oracle.bf16_to_f32(oracle.f32_to_bf16(np.array([np.float32(1)], np.float32)))[0]
    expect = oracle.f32_to_bf16(np.array([acc * (np.float32(1) / l)], np.float32))[0]
    assert int(o[0, 0, 0, 5]) == int(expect)
    # and the P0 narrowing shows up when V row 0 is one as well
    v[0, 0, 0, :] = 0x3F80
    o = oracle.attention_prefill(q, k, v, 1.0, causal=False, block_k=64)
    p0b = oracle.bf16_to_f32(oracle.f32_to_bf16(np.array([p0], np.float32)))[0]
    acc = np.float32(np.float32(0) + p0b * np.float32(1))
    acc = np.float32(acc + np.float32(1))
    expect = oracle.f32_to_bf16(np.array([acc * (np.float32(1) / l)], np.float32))[0]
    assert int(o[0, 0, 0, 7]) == int(expect)


# ---------------------------------------------------------------- fused regions
def test_fused_regions_vs_float64(oracle):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((16, 512)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    xb, wb = oracle.f32_to_bf16(x).reshape(x.shape), oracle.f32_to_bf16(w)
    xf, wf = oracle.bf16_to_f32(xb).reshape(x.shape).astype(np.float64), oracle.bf16_to_f32(wb).astype(np.float64)
    y = oracle.rmsnorm(xb, wb, 1e-5)
    ref = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-5) * wf
    attention_gate(oracle.bf16_to_f32(y).reshape(x.shape), ref, what="rmsnorm")
    y = oracle.softmax(xb)
    e = np.exp(xf - xf.max(-1, keepdims=True))
    attention_gate(oracle.bf16_to_f32(y).reshape(x.shape), e / e.sum(-1, keepdims=True), what="softmax")
    g = x[:, :256].copy()
    u = x[:, 256:].copy()
    y = oracle.silu_mul(g, u, fmt=oracle.F32)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    assert np.allclose(y, gd / (1 + np.exp(-gd)) * ud, rtol=1e-5, atol=1e-6)
    y = oracle.gelu_tanh(x, fmt=oracle.F32)
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-6)
    # RoPE, rotate-half, against a float64 restatement of the HF formula.
    T, H, D = 9, 3, 128
    xr = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = np.arange(T, dtype=np.int32) * 37
    y = oracle.rope(xr, pos, 1e4, fmt=oracle.F32)
    inv = 1.0 / (1e4 ** (np.arange(0, D, 2, dtype=np.float64) / D))
    ang = pos[:, None].astype(np.float64) * inv[None, :]
    ang = np.concatenate([ang, ang], -1)[:, None, :]
    xd = xr.astype(np.float64)
    rot = np.concatenate([-xd[..., D // 2:], xd[..., :D // 2]], -1)
    assert np.allclose(y, xd * np.cos(ang) + rot * np.sin(ang), rtol=1e-4, atol=2e-4)


def test_bias_add_closed_form(oracle):
    """bias_add is one IEEE binary32 Add per element (the managed lane's
    `float` Add, ManagedReferenceTargetModel.cpp:245) followed by the RNE
    narrowing of the output format: numpy's float32 add, then numpy's own
    float16 conversion (IEEE RNE) or a round-half-even bf16 narrowing written
    here from the bit definition.  Edge values cover cancellation to +0,
    signed zeros, infinities and a bf16 tie in both directions."""
    rng = np.random.default_rng(951)
    rows, cols = 7, 193
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 3
    b = (rng.standard_normal(cols) * 0.02).astype(np.float32)
    x[0, :4] = [1.0, -0.0, np.inf, 65504.0]
    b[:4] = [-1.0, -0.0, 1.0, 16.0]
    y = oracle.bias_add(x, b, fmt=oracle.F32)
    ref = (x + b[None, :]).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    assert y[0, 0].view(np.uint32) == 0 and y[0, 1].view(np.uint32) == 0x80000000

    def bf16_rne(f):
        u = f.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    # bf16 storage: x is bf16, the sum is formed in f32 and narrowed RNE
    xb = oracle.f32_to_bf16(x).reshape(x.shape)
    xb[1, :2] = [0x3F80, 0x3F80]          # 1.0
    b2 = b.copy()
    b2[:2] = [f32(0x3B800000), f32(0x3BC00000)]   # 2^-8 (tie, stays even) and 1.5*2^-8 (rounds up)
    yb = oracle.bias_add(xb, b2, fmt=oracle.BF16)
    wide = (oracle.bf16_to_f32(xb).reshape(x.shape) + b2[None, :]).astype(np.float32)
    assert np.array_equal(yb, bf16_rne(wide))
    assert [int(v) for v in yb[1, :2]] == [0x3F80, 0x3F81]
    # f16 storage: numpy's float32 -> float16 cast is IEEE RNE with overflow to inf
    xh = x.astype(np.float16)
    yh = oracle.bias_add(xh.view(np.uint16), b, fmt=oracle.F16)
    wideh = (xh.astype(np.float32) + b[None, :]).astype(np.float32)
    assert np.array_equal(yh, wideh.astype(np.float16).view(np.uint16))
