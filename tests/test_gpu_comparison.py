"""GPU comparator (output gate and error statistics) through the C ABI,
against the reference's own comparator unit tests (goldens), the CPU oracle
on seeded random tensors, and at large sizes against torch float64 on the
GPU (kthvalue for the nearest-rank quantiles).

Tolerances stated here: verdicts, counts, maxima, quantiles and ULP figures
are exact; the similarity figures and the means (sums accumulated in
double-double on the GPU, long double in order on the CPU) agree to a
relative 1e-12."""
import math
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

DT = dict(bool=0, i8=1, u8=2, i16=3, u16=4, i32=5, u32=6, i64=7, u64=8, f16=9, bf16=10, f32=11, tf32=12, f64=13)
ACC, INVALID_TOL, DTYPE, SHAPE, BYTES, UNSUP_FLOAT, UNSUP_STATS, ACT_NF, EXP_NF, NUMERIC, RAW = range(11)
FLOATS_REL = ("mean_absolute_error", "mean_ulp_distance", "cosine_similarity", "relative_l2_error", "exact_fraction")


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def hip():
    from vibe_compiler_amd import backend

    ctx = backend.Context(0)
    yield ctx
    ctx.close()


def host_tensor(dtype, shape, words):
    width = np.uint32 if dtype == DT["f32"] else np.uint16
    arr = np.array([int(w, 16) if isinstance(w, str) else w for w in words], dtype=width)
    return (dtype, tuple(shape), arr.view(np.uint8))


def on_gpu(t):
    dtype, shape, data = t
    return (dtype, torch.from_numpy(np.ascontiguousarray(data)).cuda(), shape)


def check_stats(got, want):
    for k, w in want.items():
        if k in FLOATS_REL:
            if math.isinf(w):
                assert math.isinf(got[k]), k
            else:
                assert got[k] == pytest.approx(w, rel=1e-12, abs=0.0), k
        else:
            assert got[k] == w, k


def both(hip, oracle, a, e, atol, rtol, sim=None):
    """Gate verdict on the GPU, checked against the oracle's."""
    v, detail = hip.compare_expected(on_gpu(a), on_gpu(e), atol, rtol, sim)
    want, info = oracle.compare_expected(a, e, atol, rtol, sim)
    assert v == want, (v, want, detail)
    return v, detail, info


def test_goldens_similarity(hip, oracle, goldens):
    g = goldens["comparison"]["similarity_all_elements"]
    pol = g["policy"]
    sim = (pol["minimum_cosine"], pol["maximum_relative_l2"])
    for name, (one, pert, two) in g["formats"].items():
        for extent in g["extents"]:
            say("similarity golden", name, extent)
            n = 4 * extent
            words = [one] * n
            exp = host_tensor(DT[name], (2, 2, extent), words)
            act = host_tensor(DT[name], (2, 2, extent), words[:-1] + [pert])
            assert both(hip, oracle, act, exp, pol["atol"], pol["rtol"])[0] == NUMERIC
            assert both(hip, oracle, act, exp, pol["atol"], pol["rtol"], sim)[0] == ACC
            v, st, _ = hip.compare_statistics(on_gpu(act), on_gpu(exp), pol["atol"], pol["rtol"])
            assert v == ACC and st["elementwise_mismatch_count"] == 1 and st["maximum_absolute_error"] == 0.125
            assert abs(st["relative_l2_error"] - 0.125 / math.sqrt(n)) <= 1e-15
            assert abs(st["cosine_similarity"] - (n + 0.125) / math.sqrt(n) / math.sqrt(n + 0.265625)) <= 1e-14
            check_stats(st, oracle.compare_statistics(act, exp, pol["atol"], pol["rtol"])[1])
            scaled = host_tensor(DT[name], (2, 2, extent), [two] * n)
            v, st, _ = hip.compare_statistics(on_gpu(scaled), on_gpu(exp), pol["atol"], pol["rtol"])
            assert st["cosine_similarity"] == 1.0 and st["relative_l2_error"] == 1.0
            assert both(hip, oracle, scaled, exp, pol["atol"], pol["rtol"], sim)[0] == NUMERIC


def test_goldens_contracts(hip, oracle, goldens):
    c = goldens["comparison"]
    g = c["similarity_zero_and_failure"]
    pol = g["policy"]
    at, rt = pol["atol"], pol["rtol"]
    sim = (pol["minimum_cosine"], pol["maximum_relative_l2"])
    say("contract goldens")
    f = {k: host_tensor(DT["f16"], (1,), [v]) for k, v in g["f16"].items()}
    p = g["permuted"]
    perm, ordered = host_tensor(DT["f16"], (2,), p["actual"]), host_tensor(DT["f16"], (2,), p["expected"])
    v, st, _ = hip.compare_statistics(on_gpu(perm), on_gpu(ordered), at, rt)
    assert st["cosine_similarity"] == pytest.approx(p["cosine"], rel=4e-16)
    assert st["relative_l2_error"] == pytest.approx(math.sqrt(p["relative_l2_squared"]), rel=4e-16)
    assert both(hip, oracle, perm, ordered, at, rt, sim)[0] == NUMERIC
    assert both(hip, oracle, ordered, f["one"], at, rt, sim)[0] == SHAPE
    assert both(hip, oracle, f["zero"], f["zero"], at, rt, sim)[0] == ACC
    v, st, _ = hip.compare_statistics(on_gpu(f["zero"]), on_gpu(f["zero"]), at, rt)
    assert st["cosine_similarity"] == 1.0 and st["relative_l2_error"] == 0.0
    for a in ("zero", "negative"):
        assert both(hip, oracle, f[a], f["one"], at, rt, sim)[0] == NUMERIC
    v, st, _ = hip.compare_statistics(on_gpu(f["one"]), on_gpu(f["zero"]), at, rt)
    assert math.isinf(st["relative_l2_error"])
    for bad in ("infinity", "nan"):
        assert both(hip, oracle, f[bad], f["one"], at, rt, sim)[0] == ACT_NF
        assert both(hip, oracle, f["one"], f[bad], at, rt, sim)[0] == EXP_NF
    empty = (DT["f16"], (0,), np.zeros(0, np.uint8))
    assert both(hip, oracle, empty, empty, at, rt, sim)[0] == UNSUP_STATS
    integer = (DT["i16"], (1,), np.zeros(2, np.uint8))
    assert both(hip, oracle, integer, f["zero"], at, rt, sim)[0] == DTYPE
    wrong = (DT["i16"], (1,), np.array([1, 0], np.uint8))
    v, detail, _ = both(hip, oracle, integer, wrong, at, rt, sim)
    assert v == RAW and detail == "byte=0 actual=0 expected=1"
    for bad in g["invalid_minimum_cosine"]:
        assert both(hip, oracle, f["one"], f["one"], at, rt, (float(bad), sim[1]))[0] == INVALID_TOL
    for bad in g["invalid_maximum_relative_l2"]:
        assert both(hip, oracle, f["one"], f["one"], at, rt, (sim[0], float(bad)))[0] == INVALID_TOL
    for key, dt in (("f16_tolerance", 9), ("bf16_tolerance", 10), ("f32_tolerance", 11)):
        t = c[key]
        a, e = host_tensor(dt, (1,), [t["actual"]]), host_tensor(dt, (1,), [t["expected"]])
        assert both(hip, oracle, a, e, *t["pass"])[0] == ACC
        assert both(hip, oracle, a, e, *t["fail"])[0] == NUMERIC
    t = c["mismatch_summary"]
    v, detail, info = both(hip, oracle, host_tensor(9, (3,), t["actual"]), host_tensor(9, (3,), t["expected"]), 0, 0)
    for s in t["contains"]:
        assert s in detail, detail
    t = c["signed_zero"]
    assert both(hip, oracle, host_tensor(9, (1,), [t["actual"]]), host_tensor(9, (1,), [t["expected"]]), 0, 0)[0] == ACC
    t = c["subnormal"]
    a, e = host_tensor(9, (1,), [t["actual"]]), host_tensor(9, (1,), [t["expected"]])
    assert both(hip, oracle, a, e, t["pass_atol"], 0.0)[0] == ACC
    assert both(hip, oracle, a, e, t["fail_atol"], 0.0)[0] == NUMERIC
    t = c["raw"]
    e = (DT["i16"], (2,), np.array(t["expected"], np.uint8))
    assert both(hip, oracle, (DT["i16"], (2,), np.array(t["same"], np.uint8)), e, 100.0, 100.0)[0] == ACC
    v, detail, _ = both(hip, oracle, (DT["i16"], (2,), np.array(t["different"], np.uint8)), e, 100.0, 100.0)
    assert detail.startswith("byte=%d " % t["first_byte"])
    f64 = (DT["f64"], (1,), np.array([1.0]).view(np.uint8))
    assert both(hip, oracle, f64, f64, 0, 0)[0] == UNSUP_FLOAT


def test_goldens_statistics(hip, oracle, goldens):
    g = goldens["comparison"]["nearest_rank"]
    say("nearest-rank golden")
    n = g["count"]
    exp = np.full(n, int(g["expected"], 16), np.uint16)
    act = exp.copy()
    act[g["plus_one_from"]:] += 1
    act[g["plus_two_at"]] = exp[0] + 2
    a, e = (9, (n,), act.view(np.uint8)), (9, (n,), exp.view(np.uint8))
    v, st, _ = hip.compare_statistics(on_gpu(a), on_gpu(e))
    assert v == ACC
    check_stats(st, oracle.compare_statistics(a, e)[1])
    for k, want in g["expect"].items():
        if k not in ("mean_absolute_error", "mean_ulp_distance"):
            assert st[k] == want, k
    u = goldens["comparison"]["ulp_domains"]
    for dt, name in ((10, "bf16"), (11, "f32")):
        v, st, _ = hip.compare_statistics(on_gpu(host_tensor(dt, (1,), [u[name]["actual"]])),
                                          on_gpu(host_tensor(dt, (1,), [u[name]["expected"]])))
        assert st["maximum_absolute_error"] == u[name]["maximum_absolute_error"]
        assert st["maximum_ulp_distance"] == u[name]["ulp"]
    i16 = (DT["i16"], (1,), np.zeros(2, np.uint8))
    assert hip.compare_statistics(on_gpu(i16), on_gpu(i16))[0] == UNSUP_STATS
    v, _, detail = hip.compare_statistics(on_gpu(host_tensor(9, (1,), ["0x7c00"])),
                                          on_gpu(host_tensor(9, (1,), ["0x3c00"])))
    assert v == ACT_NF and detail == "element=0"


def bits_pair(rng, dt, n, mode):
    x = rng.standard_normal(n).astype(np.float32)
    if mode == "sparse":
        y = x + (rng.standard_normal(n) * 1e-2).astype(np.float32) * (rng.random(n) < 0.01)
    elif mode == "dense":
        y = x * (1 + (rng.standard_normal(n) * 1e-3).astype(np.float32))
    elif mode == "equal":
        y = x.copy()
    else:  # a constant offset: every key equal in the f32 domain
        y = x + np.float32(0.25)
    if dt == 11:
        return y.view(np.uint32), x.view(np.uint32)
    if dt == 9:
        return y.astype(np.float16).view(np.uint16), x.astype(np.float16).view(np.uint16)
    return (y.view(np.uint32) >> 16).astype(np.uint16), (x.view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("dt", [9, 10, 11])
@pytest.mark.parametrize("mode", ["sparse", "dense", "equal", "offset"])
def test_statistics_random_vs_oracle(hip, oracle, dt, mode):
    rng = np.random.default_rng(dt * 7 + len(mode))
    for n in (1, 7, 1000, 262147):
        say("statistics", dt, mode, n)
        ab, eb = bits_pair(rng, dt, n, mode)
        a, e = (dt, (n,), ab.view(np.uint8)), (dt, (n,), eb.view(np.uint8))
        v, st, _ = hip.compare_statistics(on_gpu(a), on_gpu(e), 1e-3, 2e-3)
        wv, want = oracle.compare_statistics(a, e, 1e-3, 2e-3)
        assert v == wv == ACC
        check_stats(st, want)
        for sim in (None, (0.9999, 0.01)):
            gv, detail = hip.compare_expected(on_gpu(a), on_gpu(e), 1e-3, 2e-3, sim)
            ov, info = oracle.compare_expected(a, e, 1e-3, 2e-3, sim)
            assert gv == ov
            if ov == NUMERIC and sim is None:
                assert detail.startswith("mismatches=%d/%d first={element=%d " % (info["mismatches"], n, info["first"]))
                assert "max_abs={element=%d " % info["max_abs"] in detail
                assert detail.endswith("at_element=%d" % info["max_ratio"])


def test_unaligned_views_and_first_nonfinite(hip, oracle):
    # element offsets that break 16-byte alignment take the scalar path;
    # the first non-finite element (lowest index) decides the verdict
    rng = np.random.default_rng(2)
    n = 100003
    ab, eb = bits_pair(rng, 10, n + 3, "dense")
    ga, ge = torch.from_numpy(ab.view(np.int16)).cuda(), torch.from_numpy(eb.view(np.int16)).cuda()
    for off in (1, 3):
        say("unaligned", off)
        a = (10, ga[off:off + n].view(torch.uint8), (n,))
        e = (10, ge[off:off + n].view(torch.uint8), (n,))
        v, st, _ = hip.compare_statistics(a, e)
        check_stats(st, oracle.compare_statistics((10, (n,), ab[off:off + n].view(np.uint8)),
                                                  (10, (n,), eb[off:off + n].view(np.uint8)))[1])
    a2, e2 = ab[:n].copy(), eb[:n].copy()
    a2[70001] = 0x7F80  # +inf actual
    e2[50007] = 0x7FC1  # NaN expected, earlier
    a, e = (10, (n,), a2.view(np.uint8)), (10, (n,), e2.view(np.uint8))
    v, detail = hip.compare_expected(on_gpu(a), on_gpu(e), 1.0, 1.0)
    assert v == EXP_NF and detail == "element=50007"
    assert oracle.compare_expected(a, e, 1.0, 1.0)[0] == EXP_NF
    v, _, detail = hip.compare_statistics(on_gpu(a), on_gpu(e))
    assert v == EXP_NF and detail == "element=50007"


def test_statistics_large_vs_torch(hip):
    # 64M bf16 pairs (128 MiB each): counts, maxima and nearest-rank
    # quantiles from torch float64 (kthvalue) on the GPU
    n = 64 << 20
    say("large statistics", n)
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(n, device="cuda", generator=g)
    y = x * (1 + 1e-3 * torch.randn(n, device="cuda", generator=g))
    xb, yb = x.to(torch.bfloat16), y.to(torch.bfloat16)
    v, st, _ = hip.compare_statistics((10, yb.view(torch.uint8), (n,)), (10, xb.view(torch.uint8), (n,)), 1e-3, 1e-3)
    assert v == ACC
    av, ev = yb.double(), xb.double()
    ad = (av - ev).abs()
    r99, r999 = math.ceil(0.99 * n), math.ceil(0.999 * n)
    assert st["p99_absolute_error"] == torch.kthvalue(ad, r99).values.item()
    assert st["p999_absolute_error"] == torch.kthvalue(ad, r999).values.item()
    assert st["maximum_absolute_error"] == ad.max().item()
    assert st["exact_element_count"] == int((ad == 0).sum().item())
    assert st["elementwise_mismatch_count"] == int((ad > 1e-3 + 1e-3 * ev.abs()).sum().item())

    def key(b):
        b = b.view(torch.int16).to(torch.int64) & 0xFFFF
        mag = b & 0x7FFF
        return torch.where(b >= 0x8000, 0x8000 - mag, 0x8000 + mag)
    ulp = torch.where(av == ev, torch.zeros_like(ad, dtype=torch.int64), (key(yb) - key(xb)).abs())
    assert st["p99_ulp_distance"] == torch.kthvalue(ulp, r99).values.item()
    assert st["p999_ulp_distance"] == torch.kthvalue(ulp, r999).values.item()
    assert st["maximum_ulp_distance"] == ulp.max().item()
    assert st["mean_ulp_distance"] == pytest.approx(ulp.double().mean().item(), rel=1e-12)
    cos = (av * ev).sum() / av.square().sum().sqrt() / ev.square().sum().sqrt()
    assert st["cosine_similarity"] == pytest.approx(cos.item(), rel=1e-10)
    rel = ((av - ev).square().sum() / ev.square().sum()).sqrt()
    assert st["relative_l2_error"] == pytest.approx(rel.item(), rel=1e-10)
    del x, y, av, ev, ad, ulp
    torch.cuda.empty_cache()


def test_program_boundary_npy_gate(hip, tmp_path):
    # the reference's board flow at the program boundary: the FA output and a
    # torch float32 reference written as .npy (bf16 as '|V2'), loaded by the
    # C++ loader, gated on the GPU with the attention policy
    # (test/Board/PyTorch/wafer_pytorch_board_cases.py:31-33)
    from vibe_compiler_amd import program_io

    say("npy gate")
    g = torch.Generator(device="cuda").manual_seed(3)
    q, k, v = (torch.randn((1, 4, 256, 128), device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    o = torch.empty_like(q)
    scale = 1 / math.sqrt(128)
    hip.attention_prefill(q, k, v, o, scale, causal=True)
    s = (q.float() @ k.float().transpose(-1, -2).contiguous()) * scale
    mask = torch.ones(256, 256, device="cuda", dtype=torch.bool).tril()
    ref = torch.softmax(s.masked_fill(~mask, float("-inf")), dim=-1) @ v.float()

    def save(t, path):
        bits = t.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.dtype("|V2"))
        np.save(path, bits)
    save(o, tmp_path / "actual.npy")
    save(ref, tmp_path / "expected.npy")
    policy = (0.008, 0.006)
    v_, detail = program_io.compare_npy(hip, torch, tmp_path / "actual.npy", tmp_path / "expected.npy", *policy,
                                        similarity=(0.9999, 0.01))
    assert v_ == ACC, detail
    v_, st, _ = program_io.compare_npy(hip, torch, tmp_path / "actual.npy", tmp_path / "expected.npy", *policy,
                                       statistics=True)
    assert v_ == ACC and st["cosine_similarity"] >= 0.9999 and st["relative_l2_error"] <= 0.01
    bad = o.clone()
    bad[0, 1, 7, :] += 1.0
    save(bad, tmp_path / "bad.npy")
    v_, detail = program_io.compare_npy(hip, torch, tmp_path / "bad.npy", tmp_path / "expected.npy", *policy)
    assert v_ == NUMERIC and "first={element=%d " % (1 * 256 * 128 + 7 * 128) in detail
