"""Pins the oracle's formal-lane elementwise and pooling restatement
(oracle_elementwise_formal / oracle_pool) before the GPU tests trust it.

Known answers come from the reference's own kernel tests
(unittests/Simulator/Kernel/TargetModelKernelTest.cpp): the F32 Add case
(:882-918), unit broadcast (:920-979), grouped broadcast (:981-1068),
relations in full / scalar / unit form with Bool and numeric results
(:1070-1160), scalar immediates (:1162-1213) and pooling windows
(:1657-1722).  IEEE rounding is pinned independently of the oracle's own
rounding routine: F32 and F16 against numpy's IEEE arithmetic, every format
against exact rational arithmetic with a brute-force nearest-even search over
the format's representable values.  The formal zero / NaN rules
(FormalNumericElementwise.cpp:93-238) are pinned by special cases.
"""
from __future__ import annotations

import bisect
import fractions
import itertools

import numpy as np
import pytest

from oracle import oracle as o

F16, BF16, F32, BOOL = o.F16, o.BF16, o.F32, o.BOOL
FLOATS = (F16, BF16, F32)
EW = dict(Abs=0, Recip=1, Square=2, Neg=5, Max=6, Min=7, Add=8, Sub=9, Mul=10, Eq=12, Ne=13, Ge=14, Gt=15, Le=16,
          Lt=17, LogicNot=18, LogicAnd=19, LogicOr=20, LogicXor=21, Relu=31)
ONE = {F16: 0x3C00, BF16: 0x3F80, F32: 0x3F800000}
TWO = {F16: 0x4000, BF16: 0x4000, F32: 0x40000000}
NAN = {F16: 0x7E00, BF16: 0x7FC0, F32: 0x7FC00000}
SIGN = {F16: 0x8000, BF16: 0x8000, F32: 0x80000000}


def bits_of(fmt, value: float) -> int:
    """Storage bits of a value exactly representable in fmt."""
    f = np.float32(value)
    if fmt == F32:
        return int(f.view(np.uint32))
    if fmt == F16:
        h = np.float16(value)
        assert float(h) == value
        return int(h.view(np.uint16))
    u = int(f.view(np.uint32))
    assert u & 0xFFFF == 0
    return u >> 16


def test_reference_f32_add():
    lhs = np.array([bits_of(F32, v) for v in (1, 2, 3, 4)], np.uint32)
    rhs = np.array([bits_of(F32, v) for v in (4, 3, 2, 1)], np.uint32)
    assert (o.elementwise_formal(EW["Add"], F32, lhs, rhs) == 0x40A00000).all()


@pytest.mark.parametrize("fmt", FLOATS)
@pytest.mark.parametrize("extent", (1024, 1025, 1031))
@pytest.mark.parametrize("unit", (1, 32, 64))
def test_reference_unit_broadcast(fmt, extent, unit):
    count = 2 * extent * unit
    lhs = np.full(count, ONE[fmt])
    rhs = np.array([ONE[fmt] if i % 2 else 0 for i in range(unit)])
    got = o.elementwise_formal(EW["Add"], fmt, lhs, rhs, unit=unit)
    i = np.arange(count)
    assert (got == np.where((i % unit) % 2 == 1, TWO[fmt], ONE[fmt])).all()


@pytest.mark.parametrize("fmt", FLOATS)
@pytest.mark.parametrize("extent", (1024, 1025, 1031))
@pytest.mark.parametrize("op", ("Add", "Sub", "Mul", "Max", "Min"))
def test_reference_grouped_broadcast(fmt, extent, op):
    count = 2 * extent * 64
    lhs_value = 1 if op == "Mul" else (256 if op == "Min" else 0)
    lhs = np.full(count, bits_of(fmt, lhs_value))
    rhs = np.array([bits_of(fmt, i + 1) for i in range(128)])
    got = o.elementwise_formal(EW[op], fmt, lhs, rhs, unit=64, group=extent * 64).reshape(2, extent, 64)
    for g in range(2):
        want = np.array([bits_of(fmt, (-1 if op == "Sub" else 1) * (g * 64 + lane + 1)) for lane in range(64)])
        assert (got[g] == want[None, :]).all()


@pytest.mark.parametrize("fmt", FLOATS)
@pytest.mark.parametrize("extent", (1024, 1031))
@pytest.mark.parametrize("form", (0, 1, 2))
@pytest.mark.parametrize("numeric", (False, True))
def test_reference_relations(fmt, extent, form, numeric):
    count = 2 * 32 * extent
    rhs_count = 32 if form == 2 else count
    i = np.arange(count)
    lhs = np.where(i % 2 == 1, ONE[fmt], 0)
    rhs = np.where(np.arange(rhs_count) % 3 != 0, ONE[fmt], 0)
    a = i % 2
    b = np.ones(count, int) if form == 1 else ((i % rhs_count) % 3 != 0).astype(int)
    for name, fn in (("Eq", np.equal), ("Ne", np.not_equal), ("Ge", np.greater_equal), ("Gt", np.greater),
                     ("Le", np.less_equal), ("Lt", np.less)):
        if form == 1:
            got = o.elementwise_formal(EW[name], fmt, lhs, scalar=ONE[fmt], numeric=numeric)
        else:
            got = o.elementwise_formal(EW[name], fmt, lhs, rhs, unit=32 if form == 2 else 0, numeric=numeric)
        expect = fn(a, b)
        assert (got == np.where(expect, ONE[fmt] if numeric else 1, 0)).all(), name


@pytest.mark.parametrize("fmt", FLOATS)
@pytest.mark.parametrize("negative_infinity", (False, True))
def test_reference_scalar_immediate(fmt, negative_infinity):
    inf = {F32: 0xFF800000, F16: 0xFC00, BF16: 0xFF80}[fmt]
    lhs = np.full(2 * 1025 * 32, ONE[fmt])
    op = EW["Add"] if negative_infinity else EW["Mul"]
    got = o.elementwise_formal(op, fmt, lhs, scalar=inf if negative_infinity else TWO[fmt])
    assert (got == (inf if negative_infinity else TWO[fmt])).all()


@pytest.mark.parametrize("width", (1024, 1025))
@pytest.mark.parametrize("kind", (117, 119, 116))
def test_reference_pool_windows(width, kind):
    h, w, c = np.meshgrid(np.arange(5), np.arange(width + 2), np.arange(2), indexing="ij")
    src = (h * 8 + w + c).astype(np.float32).view(np.uint32)[None]
    got = o.pool(kind, F32, src, (2, width), (3, 2, 1, 2)).view(np.float32)[0]
    oh, ow, oc = np.meshgrid(np.arange(2), np.arange(width), np.arange(2), indexing="ij")
    first = (oh * 16 + ow + oc).astype(np.float32)
    want = first + 10 if kind == 117 else (first if kind == 119 else first * 6 + 30)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


# ---- IEEE rounding against independent arithmetic ----------------------------
def _special_f32(rng, n):
    vals = rng.standard_normal(n).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 30, n).astype(np.float32)
    extra = np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 1.1754942e-38, 3.4028235e38, -3.4028235e38, 1.0,
                      -1.0, 0.5, 2.0 ** -140, 3.0e38], np.float32)
    return np.concatenate([vals, extra, (rng.random(n // 8) * 1e-38).astype(np.float32)])


def _canon(fmt, bits):
    """Replace NaN encodings with the canonical positive quiet NaN."""
    bits = np.asarray(bits).astype(np.uint64)
    if fmt == F32:
        nan = (bits & 0x7FFFFFFF) > 0x7F800000
    elif fmt == F16:
        nan = (bits & 0x7FFF) > 0x7C00
    else:
        nan = (bits & 0x7FFF) > 0x7F80
    return np.where(nan, NAN[fmt], bits)


@pytest.mark.parametrize("op", ("Add", "Sub", "Mul", "Square", "Recip"))
def test_f32_matches_numpy(op):
    rng = np.random.default_rng(11)
    a = _special_f32(rng, 4000)
    b = rng.permutation(_special_f32(rng, 4000))[: a.size]
    with np.errstate(all="ignore"):
        want = {"Add": a + b, "Sub": a - b, "Mul": a * b, "Square": a * a, "Recip": np.float32(1) / a}[op]
    unary = op in ("Square", "Recip")
    got = o.elementwise_formal(EW[op], F32, a.view(np.uint32), None if unary else b.view(np.uint32))
    assert (got == _canon(F32, want.view(np.uint32))).all()


@pytest.mark.parametrize("op", ("Add", "Sub", "Mul", "Square", "Recip"))
def test_f16_matches_numpy(op):
    rng = np.random.default_rng(12)
    a = rng.integers(0, 1 << 16, 20000).astype(np.uint16)
    b = rng.integers(0, 1 << 16, 20000).astype(np.uint16)
    fa, fb = a.view(np.float16), b.view(np.float16)
    with np.errstate(all="ignore"):
        want = {"Add": fa + fb, "Sub": fa - fb, "Mul": fa * fb, "Square": fa * fa, "Recip": np.float16(1) / fa}[op]
    unary = op in ("Square", "Recip")
    got = o.elementwise_formal(EW[op], F16, a, None if unary else b)
    assert (got == _canon(F16, want.view(np.uint16))).all()


def _finite_values(fmt):
    """All finite non-negative values of fmt as (Fraction, bits), ascending."""
    if fmt == F16:
        bits = np.arange(0, 0x7C00, dtype=np.uint16)
        vals = bits.view(np.float16).astype(np.float64)
    else:
        bits = np.arange(0, 0x7F80, dtype=np.uint32)
        vals = (bits << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    return [fractions.Fraction(float(v)) for v in vals], [int(x) for x in bits]


def _round_exact(table, fmt, x: fractions.Fraction) -> int:
    """Nearest-even rounding of an exact rational by search over the format's
    values; beyond the largest finite value plus half its spacing -> inf."""
    values, bits = table
    sign = SIGN[fmt] if x < 0 else 0
    a = abs(x)
    top = values[-1] + (values[-1] - values[-2]) / 2
    inf = 0x7C00 if fmt == F16 else 0x7F80
    if a >= top:
        return sign | inf
    j = bisect.bisect_left(values, a)
    if j < len(values) and values[j] == a:
        return sign | bits[j]
    lo, hi = j - 1, j
    dl, dh = a - values[lo], values[hi] - a
    pick = lo if dl < dh else hi if dh < dl else (lo if bits[lo] % 2 == 0 else hi)
    return sign | bits[pick]


@pytest.mark.parametrize("fmt", (F16, BF16))
@pytest.mark.parametrize("op", ("Add", "Sub", "Mul", "Square", "Recip"))
def test_narrow_formats_match_exact_rounding(fmt, op):
    table = _finite_values(fmt)
    rng = np.random.default_rng(13 + fmt)
    lim = 0x7C00 if fmt == F16 else 0x7F80
    a = rng.integers(0, lim, 600) | (rng.integers(0, 2, 600) << 15)
    b = rng.integers(0, lim, 600) | (rng.integers(0, 2, 600) << 15)
    # exponents close together so sums and differences round non-trivially
    b[:300] = (a[:300] & 0xFF80) | rng.integers(0, 0x80, 300)
    got = o.elementwise_formal(EW[op], fmt, a, None if op in ("Square", "Recip") else b)

    def val(x):
        x = int(x)
        f = float(np.uint16(x).view(np.float16)) if fmt == F16 else float(np.uint32(x << 16).view(np.float32))
        return fractions.Fraction(f)

    for i in range(a.size):
        x, y = val(a[i]), val(b[i])
        if op == "Recip" and x == 0:
            want = (SIGN[fmt] if a[i] & 0x8000 else 0) | (0x7C00 if fmt == F16 else 0x7F80)
        else:
            r = {"Add": lambda: x + y, "Sub": lambda: x - y, "Mul": lambda: x * y, "Square": lambda: x * x,
                 "Recip": lambda: 1 / x}[op]()
            want = _round_exact(table, fmt, r)
            if r == 0:  # sign of an exact zero: IEEE rules
                if op == "Mul":
                    want = SIGN[fmt] if (a[i] ^ b[i]) & 0x8000 else 0
                elif op == "Square":
                    want = 0
                elif op in ("Add", "Sub"):
                    sa = bool(a[i] & 0x8000)
                    sb = bool(b[i] & 0x8000) != (op == "Sub")
                    want = SIGN[fmt] if (sa and sb) else 0
        assert int(got[i]) == want, (op, hex(int(a[i])), hex(int(b[i])), hex(int(got[i])), hex(want))


# ---- formal zero / NaN rules ---------------------------------------------------
@pytest.mark.parametrize("fmt", FLOATS)
def test_max_min_signed_zero_and_nan(fmt):
    z, nz, one, nan, snan = 0, SIGN[fmt], ONE[fmt], NAN[fmt] | 1, (0x7F800001 if fmt == F32 else
                                                                    (0x7C01 if fmt == F16 else 0x7F81))
    pairs = [(z, nz), (nz, z), (nz, nz), (z, z), (one, z), (nz, one), (nan, one), (one, snan)]
    lhs = np.array([p[0] for p in pairs])
    rhs = np.array([p[1] for p in pairs])
    mx = o.elementwise_formal(EW["Max"], fmt, lhs, rhs)
    mn = o.elementwise_formal(EW["Min"], fmt, lhs, rhs)
    assert list(mx) == [z, z, nz, z, one, one, NAN[fmt], NAN[fmt]]
    assert list(mn) == [nz, nz, nz, z, z, nz, NAN[fmt], NAN[fmt]]


@pytest.mark.parametrize("fmt", FLOATS)
def test_unary_bit_rules(fmt):
    tiny = 1  # smallest subnormal
    vals = np.array([0, SIGN[fmt], ONE[fmt], SIGN[fmt] | ONE[fmt], SIGN[fmt] | tiny, NAN[fmt] | 2 | SIGN[fmt]])
    assert list(o.elementwise_formal(EW["Relu"], fmt, vals)) == [0, SIGN[fmt], ONE[fmt], 0, 0, NAN[fmt]]
    assert list(o.elementwise_formal(EW["Abs"], fmt, vals)) == [0, 0, ONE[fmt], ONE[fmt], tiny, NAN[fmt]]
    assert list(o.elementwise_formal(EW["Neg"], fmt, vals)) == [SIGN[fmt], 0, SIGN[fmt] | ONE[fmt], ONE[fmt], tiny,
                                                                NAN[fmt]]


@pytest.mark.parametrize("fmt", FLOATS)
def test_relations_with_nan_and_zeros(fmt):
    nan = NAN[fmt] | 3
    lhs = np.array([nan, ONE[fmt], nan, 0, SIGN[fmt]])
    rhs = np.array([ONE[fmt], nan, nan, SIGN[fmt], 0])
    out = {k: list(o.elementwise_formal(EW[k], fmt, lhs, rhs)) for k in ("Eq", "Ne", "Ge", "Gt", "Le", "Lt")}
    assert out["Ne"] == [1, 1, 1, 0, 0]
    assert out["Eq"] == [0, 0, 0, 1, 1]
    for k in ("Ge", "Le"):
        assert out[k] == [0, 0, 0, 1, 1]
    for k in ("Gt", "Lt"):
        assert out[k] == [0, 0, 0, 0, 0]


def test_logic_truth_tables_and_noncanonical_bool():
    a = np.array([0, 0, 1, 1], np.uint8)
    b = np.array([0, 1, 0, 1], np.uint8)
    assert list(o.elementwise_formal(EW["LogicAnd"], BOOL, a, b)) == [0, 0, 0, 1]
    assert list(o.elementwise_formal(EW["LogicOr"], BOOL, a, b)) == [0, 1, 1, 1]
    assert list(o.elementwise_formal(EW["LogicXor"], BOOL, a, b)) == [0, 1, 1, 0]
    assert list(o.elementwise_formal(EW["LogicNot"], BOOL, a)) == [1, 1, 0, 0]
    with pytest.raises(RuntimeError):
        o.elementwise_formal(EW["LogicAnd"], BOOL, np.array([2], np.uint8), np.array([1], np.uint8))


def test_outside_subset_refused():
    for op in (3, 4, 25, 32, 33):  # Sqrt Rsqrt Exp SatRelu LeakyRelu
        with pytest.raises(RuntimeError):
            o.elementwise_formal(op, F32, np.zeros(4, np.uint32))


# ---- pooling against a direct window evaluation -----------------------------
@pytest.mark.parametrize("fmt", FLOATS)
@pytest.mark.parametrize("kind", (117, 119))
def test_pool_maxmin_matches_numpy_windows(fmt, kind):
    rng = np.random.default_rng(5 + fmt + kind)
    n, h, w, c, kw, kh, sw, sh = 2, 9, 11, 3, 3, 2, 2, 3
    vals = rng.integers(-100, 101, n * h * w * c).astype(np.float32)  # exact in every format
    src = np.array([bits_of(fmt, float(v)) for v in vals]).reshape(n, h, w, c)
    oh, ow = (h - kh) // sh + 1, (w - kw) // sw + 1
    got = o.pool(kind, fmt, src, (oh, ow), (kw, kh, sw, sh))
    x = vals.reshape(n, h, w, c)
    red = np.max if kind == 117 else np.min
    want = np.empty((n, oh, ow, c), np.float32)
    for y, z in itertools.product(range(oh), range(ow)):
        want[:, y, z] = red(x[:, y * sh:y * sh + kh, z * sw:z * sw + kw], axis=(1, 2))
    assert (got == np.vectorize(lambda v: bits_of(fmt, float(v)))(want)).all()


def test_pool_sum_order_and_nan():
    rng = np.random.default_rng(21)
    n, h, w, c, kw, kh, sw, sh = 1, 7, 8, 4, 2, 3, 1, 2
    x = (rng.standard_normal((n, h, w, c)) * 10.0 ** rng.integers(-3, 4, (n, h, w, c))).astype(np.float32)
    x[0, 0, 0, 0] = np.nan
    oh, ow = (h - kh) // sh + 1, (w - kw) // sw + 1
    got = o.pool(116, F32, x.view(np.uint32), (oh, ow), (kw, kh, sw, sh))
    want = np.zeros((n, oh, ow, c), np.float32)
    for ky in range(kh):  # sequential F32 adds from +0, kernel row outer
        for kx in range(kw):
            want = want + x[:, ky:ky + sh * (oh - 1) + 1:sh, kx:kx + sw * (ow - 1) + 1:sw]
    assert (got == _canon(F32, want.view(np.uint32))).all()
    assert got[0, 0, 0, 0] == NAN[F32]


def test_pool_single_element_window_copies_bits():
    src = np.array([NAN[F32] | 5, SIGN[F32], 0x3F800000, 0x7F800001], np.uint32).reshape(1, 2, 2, 1)
    got = o.pool(117, F32, src, (2, 2), (1, 1, 1, 1))
    assert list(got.ravel()) == list(src.ravel())  # no combine: raw NaN payloads survive
    got = o.pool(116, F32, src, (2, 2), (1, 1, 1, 1))
    assert list(got.ravel()) == [NAN[F32], 0, 0x3F800000, NAN[F32]]  # +0 + -0 = +0


def test_f32_to_f16_matches_ieee_rne():
    """oracle.f32_to_f16 (the narrowing of every F16 store) against numpy's
    IEEE round-to-nearest-even cast on the values that decide it: ties with
    even and odd mantissas, just off a tie, carries into the exponent, the
    overflow edge 65504 + 16 (ties to inf) and 65504 + 8 (stays finite),
    subnormal ties and underflow, plus random bit patterns over the range."""
    rng = np.random.default_rng(7)
    h = rng.integers(0, 0x7C00, 4096).astype(np.uint16)      # finite f16, both signs below
    base = h.view(np.float16).astype(np.float32)
    ulp = np.spacing(h.view(np.float16)).astype(np.float32)
    frac = rng.choice(np.array([0.5, 0.5 - 2.0 ** -12, 0.5 + 2.0 ** -12, 0.25, 0.75], np.float32), h.size)
    x = np.concatenate([base + frac * ulp, -(base + frac * ulp),
                        rng.integers(0, 2 ** 32, 4096, dtype=np.uint64).astype(np.uint32).view(np.float32),
                        np.array([65504 + 16, 65504 + 8, 65504 + 15.99, -65520, 2.0 ** -25, 1.5 * 2.0 ** -25,
                                  2.0 ** -26, 1023 * 2.0 ** -24 + 2.0 ** -25, 3 * 2.0 ** -25, np.inf, -np.inf,
                                  0.0, -0.0, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11], np.float32)])
    got = o.f32_to_f16(x)
    nan = np.isnan(x)
    assert (got[nan] == NAN[F16]).all()
    with np.errstate(over="ignore"):
        want = x[~nan].astype(np.float16).view(np.uint16)
    assert np.array_equal(got[~nan], want), np.nonzero(got[~nan] != want)[0][:8]
    assert list(got[-15:-10]) == [0x7C00, 0x7BFF, 0x7BFF, 0xFC00, 0x0000]
    assert list(got[-10:-4]) == [0x0001, 0x0000, 0x0400, 0x0002, 0x7C00, 0xFC00]
    assert list(got[-2:]) == [0x3C00, 0x3C02]
