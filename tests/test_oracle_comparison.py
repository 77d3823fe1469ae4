"""The comparator oracle (output gate and error statistics) pinned against
the reference's own unit tests
(unittests/Simulator/Invocation/ProgramTensorComparisonTest.cpp, vectors in
tests/golden/reference_goldens.json "comparison"), and against independent
numpy formulations: numpy's IEEE decoding, np.longdouble similarity sums,
np.sort nearest-rank quantiles and ULP distances from the integer views."""
import math

import numpy as np
import pytest

DT = dict(bool=0, i8=1, u8=2, i16=3, u16=4, i32=5, u32=6, i64=7, u64=8, f16=9, bf16=10, f32=11, tf32=12, f64=13)
ACC, INVALID_TOL, DTYPE, SHAPE, BYTES, UNSUP_FLOAT, UNSUP_STATS, ACT_NF, EXP_NF, NUMERIC, RAW = range(11)


def tensor(dtype, shape, words):
    width = np.uint32 if dtype == DT["f32"] else np.uint16
    if dtype in (DT["i16"],):
        width = np.uint16
    arr = np.array([int(w, 16) if isinstance(w, str) else w for w in words], dtype=width)
    return (dtype, tuple(shape), arr.view(np.uint8))


def fill(dtype, shape, word, last=None):
    n = int(np.prod(shape))
    words = [word] * n
    if last is not None:
        words[-1] = last
    return tensor(dtype, shape, words)


def test_similarity_uses_all_elements(oracle, goldens):
    g = goldens["comparison"]["similarity_all_elements"]
    pol = g["policy"]
    sim = (pol["minimum_cosine"], pol["maximum_relative_l2"])
    for name, (one, pert, two) in g["formats"].items():
        for extent in g["extents"]:
            count = 4 * extent
            exp = fill(DT[name], (2, 2, extent), one)
            act = fill(DT[name], (2, 2, extent), one, pert)
            assert oracle.compare_expected(act, exp, pol["atol"], pol["rtol"])[0] == NUMERIC
            assert oracle.compare_expected(act, exp, pol["atol"], pol["rtol"], sim)[0] == ACC
            v, st = oracle.compare_statistics(act, exp, pol["atol"], pol["rtol"])
            assert v == ACC
            assert st["elementwise_mismatch_count"] == 1
            assert st["maximum_absolute_error"] == 0.125
            assert abs(st["relative_l2_error"] - 0.125 / math.sqrt(count)) <= 1e-15
            assert abs(st["cosine_similarity"] - (count + 0.125) / math.sqrt(count) / math.sqrt(count + 0.265625)) <= 1e-14
            scaled = fill(DT[name], (2, 2, extent), two)
            v, st = oracle.compare_statistics(scaled, exp, pol["atol"], pol["rtol"])
            assert st["cosine_similarity"] == 1.0 and st["relative_l2_error"] == 1.0
            assert oracle.compare_expected(scaled, exp, pol["atol"], pol["rtol"], sim)[0] == NUMERIC


def test_similarity_zero_and_failure_contracts(oracle, goldens):
    g = goldens["comparison"]["similarity_zero_and_failure"]
    pol = g["policy"]
    at, rt = pol["atol"], pol["rtol"]
    sim = (pol["minimum_cosine"], pol["maximum_relative_l2"])
    f = {k: tensor(DT["f16"], (1,), [v]) for k, v in g["f16"].items()}
    p = g["permuted"]
    perm, ordered = tensor(DT["f16"], (2,), p["actual"]), tensor(DT["f16"], (2,), p["expected"])
    v, st = oracle.compare_statistics(perm, ordered, at, rt)
    assert st["cosine_similarity"] == pytest.approx(p["cosine"], rel=4e-16)
    assert st["relative_l2_error"] == pytest.approx(math.sqrt(p["relative_l2_squared"]), rel=4e-16)
    assert oracle.compare_expected(perm, ordered, at, rt, sim)[0] == NUMERIC
    assert oracle.compare_expected(ordered, f["one"], at, rt, sim)[0] == SHAPE
    assert oracle.compare_expected(f["zero"], f["zero"], at, rt, sim)[0] == ACC
    v, st = oracle.compare_statistics(f["zero"], f["zero"], at, rt)
    assert st["cosine_similarity"] == 1.0 and st["relative_l2_error"] == 0.0
    for a in ("zero", "negative"):
        assert oracle.compare_expected(f[a], f["one"], at, rt, sim)[0] == NUMERIC
    v, st = oracle.compare_statistics(f["one"], f["zero"], at, rt)
    assert math.isinf(st["relative_l2_error"])
    assert oracle.compare_expected(f["one"], f["zero"], at, rt, sim)[0] == NUMERIC
    for bad in ("infinity", "nan"):
        assert oracle.compare_expected(f[bad], f["one"], at, rt, sim)[0] == ACT_NF
        assert oracle.compare_expected(f["one"], f[bad], at, rt, sim)[0] == EXP_NF
    empty = (DT["f16"], (0,), np.zeros(0, np.uint8))
    assert oracle.compare_expected(empty, empty, at, rt, sim)[0] == UNSUP_STATS
    integer = (DT["i16"], (1,), np.zeros(2, np.uint8))
    assert oracle.compare_expected(integer, f["zero"], at, rt, sim)[0] == DTYPE
    wrong = (DT["i16"], (1,), np.array([1, 0], np.uint8))
    assert oracle.compare_expected(integer, wrong, at, rt, sim)[0] == RAW
    for bad in g["invalid_minimum_cosine"]:
        assert oracle.compare_expected(f["one"], f["one"], at, rt, (float(bad), sim[1]))[0] == INVALID_TOL
    for bad in g["invalid_maximum_relative_l2"]:
        assert oracle.compare_expected(f["one"], f["one"], at, rt, (sim[0], float(bad)))[0] == INVALID_TOL


@pytest.mark.parametrize("key,dt", [("f16_tolerance", "f16"), ("bf16_tolerance", "bf16"), ("f32_tolerance", "f32")])
def test_format_tolerances(oracle, goldens, key, dt):
    g = goldens["comparison"][key]
    exp, act = tensor(DT[dt], (1,), [g["expected"]]), tensor(DT[dt], (1,), [g["actual"]])
    assert oracle.compare_expected(act, exp, *g["pass"])[0] == ACC
    assert oracle.compare_expected(act, exp, *g["fail"])[0] == NUMERIC


def test_summary_zero_subnormal_nonfinite_raw(oracle, goldens):
    c = goldens["comparison"]
    g = c["mismatch_summary"]
    v, info = oracle.compare_expected(tensor(9, (3,), g["actual"]), tensor(9, (3,), g["expected"]), 0.0, 0.0)
    assert v == NUMERIC and info["mismatches"] == 2 and info["first"] == 1 and info["max_abs"] == 2
    g = c["signed_zero"]
    assert oracle.compare_expected(tensor(9, (1,), [g["actual"]]), tensor(9, (1,), [g["expected"]]), 0, 0)[0] == ACC
    g = c["subnormal"]
    a, e = tensor(9, (1,), [g["actual"]]), tensor(9, (1,), [g["expected"]])
    assert oracle.compare_expected(a, e, g["pass_atol"], 0.0)[0] == ACC
    assert oracle.compare_expected(a, e, g["fail_atol"], 0.0)[0] == NUMERIC
    g = c["nonfinite"]
    one16 = tensor(9, (1,), ["0x3c00"])
    assert oracle.compare_expected(tensor(9, (1,), [g["f16_actual_inf"]]), one16, *g["tolerances"])[0] == ACT_NF
    assert oracle.compare_expected(tensor(10, (1,), [g["bf16_finite"]]), tensor(10, (1,), [g["bf16_expected_nan"]]),
                                   *g["tolerances"])[0] == EXP_NF
    g = c["raw"]
    e = (DT["i16"], (2,), np.array(g["expected"], np.uint8))
    assert oracle.compare_expected((DT["i16"], (2,), np.array(g["same"], np.uint8)), e, 100.0, 100.0)[0] == ACC
    v, first = oracle.compare_expected((DT["i16"], (2,), np.array(g["different"], np.uint8)), e, 100.0, 100.0)
    assert v == RAW and first == g["first_byte"]
    # dtype, shape and unsupported floating dtypes
    assert oracle.compare_expected(one16, (DT["i16"], (1,), one16[2]), 0, 0)[0] == DTYPE
    flat = tensor(9, (2,), ["0x3c00", "0x4000"])
    assert oracle.compare_expected(flat, (9, (1, 2), flat[2]), 0, 0)[0] == SHAPE
    f64 = (DT["f64"], (1,), np.array([1.0]).view(np.uint8))
    assert oracle.compare_expected(f64, f64, 0, 0)[0] == UNSUP_FLOAT


def test_statistics_nearest_rank_and_ulp_domains(oracle, goldens):
    g = goldens["comparison"]["nearest_rank"]
    n = g["count"]
    exp = np.full(n, int(g["expected"], 16), np.uint16)
    act = exp.copy()
    act[g["plus_one_from"]:] += 1
    act[g["plus_two_at"]] = exp[0] + 2
    v, st = oracle.compare_statistics((9, (n,), act.view(np.uint8)), (9, (n,), exp.view(np.uint8)))
    assert v == ACC and st["element_count"] == n
    for k, want in g["expect"].items():
        if k == "mean_absolute_error":
            assert st[k] == 12.0 / 1024.0 / 1000.0
        elif k == "mean_ulp_distance":
            assert st[k] == 12.0 / 1000.0
        else:
            assert st[k] == want, k
    v, st = oracle.compare_statistics(tensor(9, (1,), ["0x8000"]), tensor(9, (1,), ["0x0000"]))
    assert st["exact_element_count"] == 1 and st["maximum_ulp_distance"] == 0
    u = goldens["comparison"]["ulp_domains"]
    for dt, name in ((10, "bf16"), (11, "f32")):
        v, st = oracle.compare_statistics(tensor(dt, (1,), [u[name]["actual"]]), tensor(dt, (1,), [u[name]["expected"]]))
        assert st["maximum_absolute_error"] == u[name]["maximum_absolute_error"]
        assert st["maximum_ulp_distance"] == u[name]["ulp"]
    assert oracle.compare_statistics((DT["i16"], (1,), np.zeros(2, np.uint8)),
                                     (DT["i16"], (1,), np.zeros(2, np.uint8)))[0] == UNSUP_STATS
    assert oracle.compare_statistics(tensor(9, (1,), ["0x7c00"]), tensor(9, (1,), ["0x3c00"]))[0] == ACT_NF


def numpy_statistics(a_bits, e_bits, dt, atol, rtol):
    """The statistics from numpy's own decoding: values through astype
    (f16: numpy half; bf16: bits << 16 as f32; f32: view), sums in
    np.longdouble, quantiles from np.sort, ULP distance from the sign-aware
    integer keys."""
    if dt == 11:
        av, ev = a_bits.view(np.float32).astype(np.float64), e_bits.view(np.float32).astype(np.float64)
        w = 32
    elif dt == 9:
        av, ev = a_bits.view(np.float16).astype(np.float64), e_bits.view(np.float16).astype(np.float64)
        w = 16
    else:
        av = (a_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        ev = (e_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        w = 16
    ad = np.abs(av - ev)
    tol = atol + rtol * np.abs(ev)
    sign = np.uint64(1) << np.uint64(w - 1)

    def key(b):
        b = b.astype(np.uint64)
        mag = b & (sign - np.uint64(1))
        return np.where(b & sign, sign - mag, sign + mag)
    ka, ke = key(a_bits), key(e_bits)
    ulp = np.where(av == ev, np.uint64(0), np.where(ka >= ke, ka - ke, ke - ka))
    la, le = av.astype(np.longdouble), ev.astype(np.longdouble)
    dot, aa, bb, ee = (la * le).sum(), (la * la).sum(), (le * le).sum(), ((la - le) ** 2).sum()
    n = ad.size
    r99 = max(1, min(n, math.ceil(0.99 * n))) - 1
    r999 = max(1, min(n, math.ceil(0.999 * n))) - 1
    sa, su = np.sort(ad), np.sort(ulp)
    return dict(element_count=n, exact_element_count=int((ad == 0).sum()), mean_absolute_error=float(ad.mean()),
                p99_absolute_error=sa[r99], p999_absolute_error=sa[r999], maximum_absolute_error=sa[-1],
                elementwise_mismatch_count=int((ad > tol).sum()),
                cosine_similarity=float(dot / np.sqrt(aa) / np.sqrt(bb)), relative_l2_error=float(np.sqrt(ee / bb)),
                mean_ulp_distance=float(ulp.astype(np.float64).mean()), p99_ulp_distance=int(su[r99]),
                p999_ulp_distance=int(su[r999]), maximum_ulp_distance=int(su[-1]))


@pytest.mark.parametrize("dt", [9, 10, 11])
def test_statistics_match_numpy(oracle, dt):
    rng = np.random.default_rng(dt)
    n = 30011
    x = rng.standard_normal(n).astype(np.float32)
    y = x + (rng.standard_normal(n) * 1e-2).astype(np.float32) * (rng.random(n) < 0.3)
    if dt == 11:
        ab, eb = y.view(np.uint32), x.view(np.uint32)
    elif dt == 9:
        ab, eb = y.astype(np.float16).view(np.uint16), x.astype(np.float16).view(np.uint16)
    else:
        ab, eb = (y.view(np.uint32) >> 16).astype(np.uint16), (x.view(np.uint32) >> 16).astype(np.uint16)
    v, st = oracle.compare_statistics((dt, (n,), ab.view(np.uint8)), (dt, (n,), eb.view(np.uint8)), 1e-3, 1e-3)
    assert v == ACC
    want = numpy_statistics(ab, eb, dt, 1e-3, 1e-3)
    for k, w in want.items():
        if isinstance(w, float) and k in ("mean_absolute_error", "mean_ulp_distance", "cosine_similarity",
                                          "relative_l2_error"):
            assert st[k] == pytest.approx(w, rel=1e-12), k
        else:
            assert st[k] == w, k
