"""GPU parity: the HIP kernels, called through the C ABI, against the CPU
oracle on identical seeded inputs (bit-exact where the semantics are
order-free or order-preserving, the reference's attention gate otherwise),
and at BASELINE sizes through size-independent properties.

Tolerances stated here:
  * formal GEMM, int8 GEMM, exact elementwise ops, convert, ordered reduce,
    codec: bit-exact;
  * FA / FD / RMSNorm / softmax (bf16): rtol 0.006, atol 0.008,
    cosine >= 0.9999, relative L2 <= 0.01
    (test/Board/PyTorch/wafer_pytorch_board_cases.py:31-33);
  * MFMA bf16 GEMM vs the formal lane: relative L2 <= 2e-3 (bf16 output
    rounding), max |d| <= 2e-2 * max|ref|;
  * transcendental elementwise ops (device math library vs host libm):
    relative 2e-6 + 1e-30 absolute;
  * fp32 MLP block: |gpu - ref| <= 1e-4 * |ref| + 1e-6.
"""
import math
import sys

import numpy as np
import pytest

from tests.similarity import attention_gate

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def h(s):
    return int(s, 16)


def f32(bits):
    return np.array([bits], dtype=np.uint32).view(np.float32)[0]


def u16(a):
    """numpy uint16 -> torch int16 device tensor with the same bits."""
    return dev(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16))


def from_u16(t):
    return host(t).view(np.uint16)


# ------------------------------------------------------------------ formal GEMM
def test_formal_gemm_reference_goldens(hip, B, oracle, goldens):
    say("formal gemm goldens")
    for case in goldens["gemm_fma"]:
        # k = 2 with lhs [acc, a] and rhs [1, b]: the first step widens acc
        # exactly, the second is the single fused multiply-add under test.
        if "a_f32" in case:
            lhs = np.array([h(case["acc_f32"]), h(case["a_f32"])], np.uint32).view(np.float32)
            rhs = np.array([0x3F800000, h(case["b_f32"])], np.uint32).view(np.float32)
            fmt, ld, rd = B.F32, dev(lhs), dev(rhs)
        else:
            acc16 = np.array([h(case["acc_f32"])], np.uint32).view(np.float32).astype(np.float16).view(np.uint16)[0]
            lhs = np.array([acc16, h(case["a_f16"])], np.uint16)
            rhs = np.array([0x3C00, h(case["b_f16"])], np.uint16)
            fmt, ld, rd = B.F16, u16(lhs), u16(rhs)
        out = torch.zeros(1, dtype=torch.float32, device="cuda")
        hip.gemm(ld, rd, out, 1, 2, 1, in_fmt=fmt, out_fmt=B.F32)
        assert int(host(out).view(np.uint32)[0]) == h(case["expect_f32"]), case["cite"]
    for case in goldens["gemm_finalize_f16"]:
        out = torch.zeros(1, dtype=torch.int16, device="cuda")
        hip.gemm(dev(np.array([f32(h(case["acc_f32"]))], np.float32)), dev(np.array([1.0], np.float32)), out,
                 1, 1, 1, in_fmt=B.F32, out_fmt=B.F16)
        assert int(from_u16(out)[0]) == h(case["expect_f16"]), case["cite"]
    g = goldens["gemm_2x2_f16"]
    out = torch.zeros(4, dtype=torch.int16, device="cuda")
    hip.gemm(u16([h(x) for x in g["lhs"]]), u16([h(x) for x in g["rhs"]]), out, 2, 2, 2, in_fmt=B.F16, out_fmt=B.F16)
    assert [int(x) for x in from_u16(out)] == [h(x) for x in g["expect"]]
    for case in goldens["gemm_sub_ulp_partial"]["cases"]:
        fmt = B.F16 if case["format"] == "f16" else B.BF16
        one, eps = h(case["one"]), h(case["epsilon"])
        out = torch.zeros(2, dtype=torch.float32, device="cuda")
        hip.gemm(u16([one, eps, one, eps]), u16([one] * 4), out, 1, 2, 1, batch=2, in_fmt=fmt, out_fmt=B.F32)
        assert [int(x) for x in host(out).view(np.uint32)] == [h(case["expect_f32"])] * 2
    gp = goldens["gemm_psum_cancellation"]
    for case in gp["cases"]:
        fmt = B.F16 if case["format"] == "f16" else B.BF16
        one, eps = h(case["one"]), h(case["epsilon"])
        out = torch.zeros(2, dtype=torch.int16, device="cuda")
        psum = dev(np.array([f32(h(gp["psum_f32"]))] * 2, np.float32))
        hip.gemm(u16([one, eps, one, eps]), u16([one] * 4), out, 1, 2, 1, batch=2, in_fmt=fmt, out_fmt=fmt, psum=psum)
        assert [int(x) for x in from_u16(out)] == [eps, eps]
    g = goldens["gemm_batched_ncx_f32"]
    out = torch.zeros(8, dtype=torch.float32, device="cuda")
    lhs = np.array([h(x) for x in g["lhs"]], np.uint32).view(np.float32)
    rhs = np.array([h(x) for x in g["rhs"]], np.uint32).view(np.float32)
    hip.gemm(dev(lhs), dev(rhs), out, 2, 2, 2, batch=2)
    assert [int(x) for x in host(out).view(np.uint32)] == [h(x) for x in g["expect"]]


@pytest.mark.parametrize("fmt_in,fmt_out", [(5, 5), (3, 3), (2, 2), (3, 5), (2, 5), (5, 3)])
@pytest.mark.parametrize("lt,rt", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_formal_gemm_bit_exact_random(hip, B, oracle, fmt_in, fmt_out, lt, rt):
    say("formal gemm random", fmt_in, fmt_out, lt, rt)
    rng = np.random.default_rng(100 + fmt_in * 10 + fmt_out + 4 * lt + 2 * rt)
    for (m, k, n, batch, with_psum) in [(37, 70, 65, 2, True), (128, 129, 3, 1, False), (1, 300, 1, 3, True)]:
        a = rng.standard_normal((batch, m, k)).astype(np.float32)
        b = rng.standard_normal((batch, k, n)).astype(np.float32)
        if lt:
            a = np.ascontiguousarray(np.swapaxes(a, 1, 2))
        if rt:
            b = np.ascontiguousarray(np.swapaxes(b, 1, 2))
        if fmt_in == B.F32:
            ah, bh = a, b
            ad, bd = dev(a), dev(b)
        elif fmt_in == B.BF16:
            ah, bh = oracle.f32_to_bf16(a).reshape(a.shape), oracle.f32_to_bf16(b).reshape(b.shape)
            ad, bd = u16(ah), u16(bh)
        else:
            ah, bh = a.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
            ad, bd = u16(ah), u16(bh)
        ps = rng.standard_normal((batch, m, n)).astype(np.float32) if with_psum else None
        ref = oracle.gemm_formal(fmt_in, fmt_out, ah, bh, m, k, n, batch=batch, psum=ps, lhs_t=bool(lt), rhs_t=bool(rt))
        if fmt_out == B.F32:
            out = torch.zeros(batch * m * n, dtype=torch.float32, device="cuda")
        else:
            out = torch.zeros(batch * m * n, dtype=torch.int16, device="cuda")
        hip.gemm(ad, bd, out, m, k, n, batch=batch, in_fmt=fmt_in, out_fmt=fmt_out,
                 psum=None if ps is None else dev(ps), lhs_t=bool(lt), rhs_t=bool(rt))
        got = host(out)
        assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), (m, k, n, batch)


@pytest.mark.parametrize("m,k,n", [(128, 512, 2048), (128, 2048, 512), (256, 96, 1024)])
def test_formal_gemm_bit_exact_config0_shapes(hip, B, oracle, m, k, n):
    """The formal GEMM at the MLP's shapes (each picks a different per-thread
    chain count): every output bit-identical to the CPU formal lane."""
    say("formal gemm config0 shape", m, k, n)
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((k, n)) / math.sqrt(k)).astype(np.float32)
    ref = oracle.gemm_formal(oracle.F32, oracle.F32, a, b, m, k, n)
    out = torch.zeros(m * n, dtype=torch.float32, device="cuda")
    hip.gemm(dev(a), dev(b), out, m, k, n)
    assert np.array_equal(host(out).view(np.uint32), ref.view(np.uint32))


def test_fp32_mlp_block_config0(hip, B, oracle):
    """x[128,512] @ W1 + b1, tanh-GELU, @ W2 + b2 (f32)."""
    say("fp32 mlp block")
    rng = np.random.default_rng(20260803)
    x = rng.standard_normal((128, 512)).astype(np.float32)
    w1 = (rng.standard_normal((512, 2048)) / math.sqrt(512)).astype(np.float32)
    b1 = (rng.standard_normal(2048) * 0.02).astype(np.float32)
    w2 = (rng.standard_normal((2048, 512)) / math.sqrt(2048)).astype(np.float32)
    b2 = (rng.standard_normal(512) * 0.02).astype(np.float32)
    # CPU lane: formal GEMM, bias add, GELU region, formal GEMM, bias add
    h1 = oracle.gemm_formal(oracle.F32, oracle.F32, x, w1, 128, 512, 2048).reshape(128, 2048)
    h1 = oracle.bias_add(h1, b1)
    h1 = oracle.gelu_tanh(h1, fmt=oracle.F32)
    y = oracle.gemm_formal(oracle.F32, oracle.F32, h1, w2, 128, 2048, 512).reshape(128, 512)
    y = oracle.bias_add(y, b2)
    xd, w1d, w2d = dev(x), dev(w1), dev(w2)
    hd = torch.empty((128, 2048), dtype=torch.float32, device="cuda")
    yd = torch.empty((128, 512), dtype=torch.float32, device="cuda")
    hip.gemm(xd, w1d, hd, 128, 512, 2048)
    hip.bias_add(hd, dev(b1), hd, fmt=B.F32)
    hip.gelu_tanh(hd, hd, fmt=B.F32)
    hip.gemm(hd, w2d, yd, 128, 2048, 512)
    hip.bias_add(yd, dev(b2), yd, fmt=B.F32)
    got = host(yd)
    # GEMMs and bias adds are bit-exact; only tanh differs by device ulps.
    assert np.all(np.abs(got - y) <= 1e-4 * np.abs(y) + 1e-6)
    gh = host(hd)
    assert np.abs(gh - h1).max() <= 1e-5


def test_fp32_mlp_block_config0_mfma(hip, B, oracle):
    """BASELINE config 0 on the f32 MFMA lane: two wafer_hip_gemm_f32_mfma
    calls (bias + tanh-GELU fused into the first, bias into the second)
    against the formal CPU composition, to C1's 1e-4 relative bound: relative
    L2 <= 1e-5, and per element rtol 1e-4 with atol 1e-5 * max|ref| (the f32
    sums run in another order: about 1e-6 absolute on outputs of order 1,
    which a pure per-element rtol cannot hold near zero)."""
    say("fp32 mlp block, f32 mfma")
    rng = np.random.default_rng(20260803)
    x = rng.standard_normal((128, 512)).astype(np.float32)
    w1 = (rng.standard_normal((512, 2048)) / math.sqrt(512)).astype(np.float32)
    b1 = (rng.standard_normal(2048) * 0.02).astype(np.float32)
    w2 = (rng.standard_normal((2048, 512)) / math.sqrt(2048)).astype(np.float32)
    b2 = (rng.standard_normal(512) * 0.02).astype(np.float32)
    h1 = oracle.gemm_formal(oracle.F32, oracle.F32, x, w1, 128, 512, 2048).reshape(128, 2048)
    h1 = oracle.gelu_tanh(oracle.bias_add(h1, b1), fmt=oracle.F32)
    y = oracle.gemm_formal(oracle.F32, oracle.F32, h1, w2, 128, 2048, 512).reshape(128, 512)
    y = oracle.bias_add(y, b2)
    hd = torch.empty((128, 2048), dtype=torch.float32, device="cuda")
    yd = torch.empty((128, 512), dtype=torch.float32, device="cuda")
    hip.gemm_f32_mfma(dev(x), dev(w1), hd, 128, 512, 2048, bias=dev(b1), epilogue=B.EPILOGUE_BIAS_GELU_TANH)
    hip.gemm_f32_mfma(hd, dev(w2), yd, 128, 2048, 512, bias=dev(b2), epilogue=B.EPILOGUE_BIAS)
    got = host(yd)
    assert np.linalg.norm(got - y) / np.linalg.norm(y) <= 1e-5
    assert np.all(np.abs(got - y) <= 1e-4 * np.abs(y) + 1e-5 * np.abs(y).max())
    assert np.abs(host(hd) - h1).max() <= 1e-5


@pytest.mark.parametrize("m,k,n,rt", [(128, 512, 2048, False), (128, 2048, 512, False), (128, 2048, 512, True),
                                      (77, 72, 130, False), (300, 1000, 257, True), (1024, 256, 1024, False),
                                      (33, 4096, 40, False), (8, 8, 8, True), (200, 512, 330, True),
                                      (200, 512, 330, False)])
def test_gemm_f32_mfma_vs_formal_and_unfused(hip, B, oracle, m, k, n, rt):
    """wafer_hip_gemm_f32_mfma: the product against the formal lane (f32
    accumulation in another order: relative L2 <= 1e-5, max |d| <= 5e-5 *
    max |ref|); the bias and bias + tanh-GELU epilogues bit-identical to the
    plain product followed by the bias_add and gelu_tanh regions; a repeated
    call bit-identical.  Shapes cover 32x32 tiles with one split (n 2048,
    1024 tiles), 16x16 tiles (n 512 and the ragged 200 x 330), k split over
    workgroups with a fold launch (n 40, the ragged 300 x 257 with k 1000),
    ragged m, n and k."""
    say("gemm f32 mfma", m, k, n, rt)
    rng = np.random.default_rng(m * 7 + k * 3 + n + rt)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((k, n)) / math.sqrt(k)).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.02).astype(np.float32)
    ref = oracle.gemm_formal(oracle.F32, oracle.F32, a, b, m, k, n).reshape(m, n)
    ad, bd, biasd = dev(a), dev(np.ascontiguousarray(b.T) if rt else b), dev(bias)
    plain = torch.full((m, n), 7.5, dtype=torch.float32, device="cuda")
    hip.gemm_f32_mfma(ad, bd, plain, m, k, n, rhs_t=rt)
    got = host(plain)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5
    assert np.abs(got - ref).max() <= 5e-5 * np.abs(ref).max()
    again = torch.empty_like(plain)
    hip.gemm_f32_mfma(ad, bd, again, m, k, n, rhs_t=rt)
    assert torch.equal(again.view(torch.int32), plain.view(torch.int32))
    # fused epilogues against the unfused regions on the same product
    want_b = torch.empty_like(plain)
    hip.bias_add(plain, biasd, want_b, fmt=B.F32)
    want_g = torch.empty_like(plain)
    hip.gelu_tanh(want_b, want_g, fmt=B.F32)
    got_b = torch.empty_like(plain)
    hip.gemm_f32_mfma(ad, bd, got_b, m, k, n, bias=biasd, epilogue=B.EPILOGUE_BIAS, rhs_t=rt)
    got_g = torch.empty_like(plain)
    hip.gemm_f32_mfma(ad, bd, got_g, m, k, n, bias=biasd, epilogue=B.EPILOGUE_BIAS_GELU_TANH, rhs_t=rt)
    torch.cuda.synchronize()
    assert torch.equal(got_b.view(torch.int32), want_b.view(torch.int32))
    assert torch.equal(got_g.view(torch.int32), want_g.view(torch.int32))


def test_gemm_f32_mfma_rejections(hip, B):
    """k not a multiple of 8, a missing bias for a bias epilogue, an unknown
    epilogue and a misaligned lhs are refused before any launch."""
    say("gemm f32 mfma rejections")
    a = torch.zeros(64 * 64 + 4, dtype=torch.float32, device="cuda")
    b = torch.zeros(64 * 64, dtype=torch.float32, device="cuda")
    y = torch.zeros(64 * 64, dtype=torch.float32, device="cuda")
    with pytest.raises(B.WaferHipError) as e:
        hip.gemm_f32_mfma(a, b, y, 64, 60, 64)
    assert e.value.status == -3  # UnsupportedCommand
    for bad in (dict(epilogue=B.EPILOGUE_BIAS), dict(epilogue=3, bias=b)):
        with pytest.raises((B.WaferHipError, ValueError)):
            hip.gemm_f32_mfma(a, b, y, 64, 64, 64, **bad)
    with pytest.raises(B.WaferHipError) as e:
        hip.gemm_f32_mfma(a[1:], b, y, 64, 64, 64)
    assert e.value.status == -3  # UnsupportedCommand


# ------------------------------------------------------------------ int8 GEMM
@pytest.mark.parametrize("m,k,n", [(256, 256, 256), (128, 640, 384), (512, 4096, 256)])
@pytest.mark.parametrize("rt", [0, 1])
def test_i8_gemm_bit_exact(hip, B, oracle, m, k, n, rt):
    say("i8 gemm", m, k, n, rt)
    rng = np.random.default_rng(m + k + n + rt)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int64).astype(np.int8)
    b = rng.integers(-127, 128, size=(k, n), dtype=np.int64).astype(np.int8)
    bb = np.ascontiguousarray(b.T) if rt else b
    scale = rng.uniform(0.001, 0.01, size=n).astype(np.float32)
    acc_ref, y_ref = oracle.gemm_i8(a, bb, scale, m, k, n, rhs_t=bool(rt))
    acc = torch.zeros((m, n), dtype=torch.int32, device="cuda")
    y = torch.zeros((m, n), dtype=torch.int16, device="cuda")
    hip.gemm_i8(dev(a), dev(bb), dev(scale), y, m, k, n, acc_out=acc, rhs_t=bool(rt))
    assert np.array_equal(host(acc), acc_ref)
    assert np.array_equal(host(y).view(np.uint16), y_ref)


def test_i8_gemm_extremes(hip, B, oracle):
    """|acc| at its maximum (k * 127 * 127 and k * 127 * -128) stays exact."""
    say("i8 gemm extremes")
    m = n = 128
    k = 4096
    a = np.full((m, k), 127, np.int8)
    a[1::2] = -128
    b = np.full((k, n), -127, np.int8)
    b[:, ::3] = -128
    scale = np.full(n, 0.0078125, np.float32)
    acc_ref, y_ref = oracle.gemm_i8(a, b, scale, m, k, n)
    acc = torch.zeros((m, n), dtype=torch.int32, device="cuda")
    y = torch.zeros((m, n), dtype=torch.int16, device="cuda")
    hip.gemm_i8(dev(a), dev(b), dev(scale), y, m, k, n, acc_out=acc)
    assert np.array_equal(host(acc), acc_ref)
    assert np.array_equal(host(y).view(np.uint16), y_ref)
    assert int(host(acc)[1, 0]) == 4096 * 128 * 128


def test_i8_gemm_baseline_size_rows(hip, B, oracle):
    """BASELINE config 3 (4096^3, Normal rhs): exact int64 closed form on a
    sample of 24 full rows and the dequant chain bit-exact on them."""
    say("i8 gemm 4096^3")
    rng = np.random.default_rng(20260803)
    M = N = K = 4096
    a = rng.integers(-127, 128, size=(M, K), dtype=np.int64).astype(np.int8)
    b = rng.integers(-127, 128, size=(K, N), dtype=np.int64).astype(np.int8)
    scale = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
    acc = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    y = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    hip.gemm_i8(dev(a), dev(b), dev(scale), y, M, K, N, acc_out=acc)
    accg, yg = host(acc), host(y).view(np.uint16)
    rows = np.concatenate([[0, 1, 255, 256, 2047, 4095], rng.choice(M, 18, replace=False)])
    exact = a[rows].astype(np.int64) @ b.astype(np.int64)
    assert np.array_equal(accg[rows], exact.astype(np.int32))
    yr = oracle.f32_to_bf16((exact.astype(np.float32) * scale).astype(np.float32)).reshape(exact.shape)
    assert np.array_equal(yg[rows], yr)
    # checksum of checksums over the whole output: column sums of the
    # accumulator equal (colsum of A) @ B exactly.
    colsum = a.astype(np.int64).sum(0) @ b.astype(np.int64)
    assert np.array_equal(accg.astype(np.int64).sum(0), colsum)


@pytest.mark.parametrize("rt", [0, 1])
def test_i8_gemm_baseline_size_y_only(hip, B, oracle, rt):
    """BASELINE config 3 exactly as the bench runs it: 4096^3 with no
    accumulator output, which takes the 256x256 tiles with the LDS-staged
    dequant epilogue (passing acc_out switches the staging off).  y must be
    bit-identical to the acc_out run's y, and to the int64 closed form plus
    the dequant chain bf16(f32(f32(acc) * scale)) on sampled rows."""
    say("i8 gemm 4096^3 y-only", rt)
    rng = np.random.default_rng(20260804 + rt)
    M = N = K = 4096
    a = rng.integers(-127, 128, size=(M, K), dtype=np.int64).astype(np.int8)
    b = rng.integers(-127, 128, size=(K, N), dtype=np.int64).astype(np.int8)
    bb = np.ascontiguousarray(b.T) if rt else b
    scale = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
    ad, bd, sd = dev(a), dev(bb), dev(scale)
    y_only = torch.full((M, N), 0x1234, dtype=torch.int16, device="cuda")
    hip.gemm_i8(ad, bd, sd, y_only, M, K, N, rhs_t=bool(rt))
    acc = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    y_acc = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    hip.gemm_i8(ad, bd, sd, y_acc, M, K, N, acc_out=acc, rhs_t=bool(rt))
    yo, ya = host(y_only).view(np.uint16), host(y_acc).view(np.uint16)
    assert np.array_equal(yo, ya)
    rows = np.concatenate([[0, 1, 127, 128, 255, 256, 2047, 4095], rng.choice(M, 16, replace=False)])
    exact = a[rows].astype(np.int64) @ b.astype(np.int64)
    yr = oracle.f32_to_bf16((exact.astype(np.float32) * scale).astype(np.float32)).reshape(exact.shape)
    assert np.array_equal(yo[rows], yr)
    # every column of every 256-wide tile: the accumulator's column sums
    # (checked exactly against (colsum A) @ B) feed the same y
    colsum = a.astype(np.int64).sum(0) @ b.astype(np.int64)
    assert np.array_equal(host(acc).astype(np.int64).sum(0), colsum)


@pytest.mark.parametrize("m,k,n", [(3072, 128, 4096), (4096, 256, 3072), (4096, 384, 3072), (4096, 1152, 4096)])
def test_i8_gemm_kn_rhs_in_place(hip, B, oracle, m, k, n):
    """A [K, N] rhs on >= 192 whole 256x256 tiles is read in place (the
    transposing LDS reads, no re-layout pass): y and the accumulator over
    the whole output equal the run on the same rhs stored [N, K], and the
    int64 closed form on sampled rows; one, two, three and nine 128-byte K
    stages (the two-slot ring's first, even and odd stage counts)."""
    say("i8 gemm [K,N] in place", m, k, n)
    rng = np.random.default_rng(m * 7 + k + n)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int64).astype(np.int8)
    b = rng.integers(-128, 128, size=(k, n), dtype=np.int64).astype(np.int8)
    scale = rng.uniform(0.001, 0.01, size=n).astype(np.float32)
    ad, sd = dev(a), dev(scale)
    outs = []
    for rt, bb in ((0, b), (1, np.ascontiguousarray(b.T))):
        acc = torch.full((m, n), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
        y = torch.full((m, n), 0x1234, dtype=torch.int16, device="cuda")
        hip.gemm_i8(ad, dev(bb), sd, y, m, k, n, acc_out=acc, rhs_t=bool(rt))
        y_only = torch.full((m, n), 0x1234, dtype=torch.int16, device="cuda")
        hip.gemm_i8(ad, dev(bb), sd, y_only, m, k, n, rhs_t=bool(rt))
        outs.append((host(acc), host(y).view(np.uint16), host(y_only).view(np.uint16)))
    (acc0, y0, yo0), (acc1, y1, yo1) = outs
    assert np.array_equal(acc0, acc1)
    assert np.array_equal(y0, y1) and np.array_equal(yo0, yo1) and np.array_equal(y0, yo0)
    rows = np.concatenate([[0, 1, 255, 256, m - 1], rng.choice(m, 11, replace=False)])
    exact = a[rows].astype(np.int64) @ b.astype(np.int64)
    assert np.array_equal(acc0[rows], exact.astype(np.int32))
    yr = oracle.f32_to_bf16((exact.astype(np.float32) * scale).astype(np.float32)).reshape(exact.shape)
    assert np.array_equal(y0[rows], yr)


@pytest.mark.parametrize("m,k,n,rt", [(100, 192, 130, 0), (1, 64, 1, 1), (300, 128, 257, 0), (129, 256, 200, 1),
                                      (257, 64, 128, 0), (130, 320, 384, 1), (64, 128, 1000, 0)])
def test_i8_gemm_ragged_bit_exact(hip, B, oracle, m, k, n, rt):
    """m, n that the 128x128 tiles do not divide (the last tile row / column
    re-reads its last real operand row and stores only real outputs), and the
    bounds-checked re-layout for n that the tiled transpose does not divide.
    Outputs live in flat buffers with a canary tail that must stay intact."""
    say("i8 gemm ragged", m, k, n, rt)
    rng = np.random.default_rng(3 * m + 5 * k + 7 * n + rt)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int64).astype(np.int8)
    b = rng.integers(-128, 128, size=(k, n), dtype=np.int64).astype(np.int8)
    bb = np.ascontiguousarray(b.T) if rt else b
    scale = rng.uniform(0.001, 0.01, size=n).astype(np.float32)
    acc_ref, y_ref = oracle.gemm_i8(a, bb, scale, m, k, n, rhs_t=bool(rt))
    pad = 4096
    acc = torch.full((m * n + pad,), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
    y = torch.full((m * n + pad,), 0x1234, dtype=torch.int16, device="cuda")
    hip.gemm_i8(dev(a), dev(bb), dev(scale), y, m, k, n, acc_out=acc, rhs_t=bool(rt))
    ga, gy = host(acc), host(y).view(np.uint16)
    assert np.array_equal(ga[:m * n].reshape(m, n), acc_ref)
    assert np.array_equal(gy[:m * n].reshape(m, n), y_ref)
    assert np.all(ga[m * n:] == 0x5A5A5A5A) and np.all(gy[m * n:] == 0x1234)


# ------------------------------------------------------------------ MFMA bf16 GEMM
@pytest.mark.parametrize("m,k,n,rt,fmt", [(256, 512, 256, 0, 3), (128, 256, 384, 1, 3), (512, 1024, 512, 0, 2),
                                          (1024, 4096, 1024, 1, 3), (256, 8192, 1024, 1, 3), (256, 8192, 1024, 0, 2)])
def test_mfma_gemm_vs_formal(hip, B, oracle, m, k, n, rt, fmt):
    """The MFMA GEMM against the formal lane (f32 and narrowed outputs);
    k 8192 at 256 x 1024 takes the split-K path (256x256 tiles, K over 4
    workgroups, fold launch)."""
    say("mfma gemm", m, k, n, rt, fmt)
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((k, n)) / math.sqrt(k)).astype(np.float32)
    if fmt == B.BF16:
        ah, bh = oracle.f32_to_bf16(a).reshape(a.shape), oracle.f32_to_bf16(b).reshape(b.shape)
    else:
        ah, bh = a.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    bt = np.ascontiguousarray(bh.T) if rt else bh
    ref = oracle.gemm_formal(fmt, oracle.F32, ah, bt, m, k, n, rhs_t=bool(rt)).reshape(m, n)
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    hip.gemm_mfma(u16(ah), u16(bt), out, m, k, n, in_fmt=fmt, out_fmt=B.F32, rhs_t=bool(rt))
    got = host(out)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= 1e-5 and np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
    outn = torch.zeros((m, n), dtype=torch.int16, device="cuda")
    hip.gemm_mfma(u16(ah), u16(bt), outn, m, k, n, in_fmt=fmt, out_fmt=fmt, rhs_t=bool(rt))
    gn = from_u16(outn)
    gf = oracle.to_float(fmt, gn).reshape(m, n)
    rel = np.linalg.norm(gf - ref) / np.linalg.norm(ref)
    assert rel <= 2e-3 and np.abs(gf - ref).max() <= 2e-2 * np.abs(ref).max()


@pytest.mark.parametrize("rt,fmt,out,K", [(1, 3, 3, 1024), (0, 3, 5, 1024), (1, 2, 2, 1024), (1, 3, 3, 192),
                                          (1, 2, 2, 64)])
def test_mfma_gemm_256_tiles_vs_formal(hip, B, oracle, rt, fmt, out, K):
    """m = n = 4096: 256 tiles of 256x256, which takes the 256x256
    instantiation (used only from 192 such tiles on); k = 192 and 64 give an
    odd number of 128-byte K stages and a single one.  Sampled rows against
    the formal lane run on the GPU (bit-exact k-order fma chains; itself
    pinned against the CPU oracle on two rows here), held to the MFMA GEMM
    tolerances: f32 out relL2 <= 1e-5, narrowed out relL2 <= 2e-3."""
    say("mfma gemm 256x256 tiles", rt, fmt, out, K)
    rng = np.random.default_rng(4096 + 10 * rt + fmt + K)
    M, N = 4096, 4096
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = (rng.standard_normal((K, N)) / math.sqrt(K)).astype(np.float32)
    if fmt == B.BF16:
        ah, bh = oracle.f32_to_bf16(a).reshape(a.shape), oracle.f32_to_bf16(b).reshape(b.shape)
    else:
        ah, bh = a.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    bt = np.ascontiguousarray(bh.T) if rt else bh
    ad, bd = u16(ah), u16(bt)
    if out == B.F32:
        dst = torch.full((M, N), 7.5, dtype=torch.float32, device="cuda")
    else:
        dst = torch.full((M, N), 0x1234, dtype=torch.int16, device="cuda")
    hip.gemm_mfma(ad, bd, dst, M, K, N, in_fmt=fmt, out_fmt=out, rhs_t=bool(rt))
    got_all = host(dst)
    rows = np.concatenate([[0, 1, 255, 256, 2047, 4095], rng.choice(M, 26, replace=False)])
    sub = np.ascontiguousarray(ah[rows])
    ref_d = torch.zeros((len(rows), N), dtype=torch.float32, device="cuda")
    hip.gemm(u16(sub), bd, ref_d, len(rows), K, N, in_fmt=fmt, out_fmt=B.F32, rhs_t=bool(rt))
    ref = host(ref_d)
    cpu = oracle.gemm_formal(fmt, oracle.F32, np.ascontiguousarray(sub[:2]), bt, 2, K, N, rhs_t=bool(rt))
    assert np.array_equal(cpu.reshape(2, N).view(np.uint32), ref[:2].view(np.uint32))
    if out == B.F32:
        got = got_all[rows]
        tol_rel, tol_max = 1e-5, 1e-4
    else:
        got = oracle.to_float(fmt, got_all.view(np.uint16)[rows]).reshape(len(rows), N)
        tol_rel, tol_max = 2e-3, 2e-2
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= tol_rel and np.abs(got - ref).max() <= tol_max * np.abs(ref).max(), (rel,)
    # every output written (no sentinel left)
    if out == B.F32:
        assert not np.any(got_all == 7.5)
    else:
        assert int(np.count_nonzero(got_all.view(np.uint16) == 0x1234)) < 64


@pytest.mark.parametrize("m,n,fmt,out,K", [(1024, 4096, 3, 3, 512), (1024, 4096, 3, 5, 320), (384, 640, 2, 2, 64),
                                           (128, 128, 3, 3, 192), (256, 1024, 2, 5, 1024)])
def test_mfma_gemm_128_tiles_vs_formal(hip, B, oracle, m, n, fmt, out, K):
    """Full 128x128 tiles where neither 256x256 nor 128x192 tiles are taken
    (the decoder layer's O projection, 1024 x 4096): the four-wave LDS-DMA
    kernel; k = 320, 192 and 64 give odd numbers of 128-byte K stages and a
    single one.  Sampled rows against the GPU formal lane (pinned to the CPU
    oracle on two rows), every output written; MFMA GEMM tolerances."""
    say("mfma gemm 128x128 tiles", m, n, fmt, out, K)
    rng = np.random.default_rng(m + n + fmt + out + K)
    a = rng.standard_normal((m, K)).astype(np.float32)
    b = (rng.standard_normal((n, K)) / math.sqrt(K)).astype(np.float32)
    if fmt == B.BF16:
        a, bt = oracle.f32_to_bf16(a).reshape(m, K), oracle.f32_to_bf16(b).reshape(n, K)
    else:
        a, bt = a.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    ad, bd = u16(a), u16(bt)
    if out == B.F32:
        dst = torch.full((m, n), 7.5, dtype=torch.float32, device="cuda")
    else:
        dst = torch.full((m, n), 0x1234, dtype=torch.int16, device="cuda")
    hip.gemm_mfma(ad, bd, dst, m, K, n, in_fmt=fmt, out_fmt=out, rhs_t=True)
    got_all = host(dst)
    rows = np.concatenate([[0, 1, 127, m - 1], rng.choice(m, 28, replace=False)])
    sub = np.ascontiguousarray(a[rows])
    ref_d = torch.zeros((len(rows), n), dtype=torch.float32, device="cuda")
    hip.gemm(u16(sub), bd, ref_d, len(rows), K, n, in_fmt=fmt, out_fmt=B.F32, rhs_t=True)
    ref = host(ref_d)
    cpu = oracle.gemm_formal(fmt, oracle.F32, np.ascontiguousarray(sub[:2]), bt, 2, K, n, rhs_t=True)
    assert np.array_equal(cpu.reshape(2, n).view(np.uint32), ref[:2].view(np.uint32))
    if out == B.F32:
        got = got_all[rows]
        tol_rel, tol_max = 1e-5, 1e-4
        assert not np.any(got_all == 7.5)
    else:
        got = oracle.to_float(fmt, got_all[rows].view(np.uint16)).reshape(len(rows), n)
        tol_rel, tol_max = 2e-3, 2e-2
        assert int(np.count_nonzero(got_all.view(np.uint16) == 0x1234)) < 64
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= tol_rel and np.abs(got - ref).max() <= tol_max * np.abs(ref).max(), (rel,)


def _narrowing_cases(oracle, rng, n):
    """bf16 pairs (x, y) whose exact f32 sum x + y lands on the cases RNE
    narrowing has to get right: ties to even (y = half an ulp of x, x with
    even and odd mantissa), just below and above a tie, carries into the
    exponent, the overflow edge (rounds to inf), infinities and NaNs."""
    e = rng.integers(-100, 120, n)
    mant = rng.integers(0, 128, n)
    sign = rng.choice([-1.0, 1.0], n)
    x = sign * (1.0 + mant / 128.0) * np.exp2(e.astype(np.float64))
    half = np.exp2(e - 8.0)
    kind = rng.integers(0, 5, n)
    y = np.select([kind == 0, kind == 1, kind == 2, kind == 3], [half, 0.75 * half, 1.5 * half, -half], 0.375 * half)
    y = y * sign
    x[:64] = sign[:64] * (2.0 - 1 / 128.0) * 2.0 ** 127   # largest finite bf16 ...
    y[:32] = sign[:32] * 2.0 ** 119                     # ... plus half an ulp: ties to inf
    y[32:64] = sign[32:64] * 2.0 ** 118                 # ... plus a quarter: stays finite
    # every x and y is a bf16 value, so these conversions are exact
    xb = oracle.f32_to_bf16(x.astype(np.float32)).reshape(n)
    yb = oracle.f32_to_bf16(y.astype(np.float32)).reshape(n)
    xb[64:72] = [0x7f80, 0xff80, 0x7fc0, 0x7fa1, 0xffd3, 0x7f81, 0x0000, 0x8000]  # inf, NaN payloads, zeros
    return xb, yb


@pytest.mark.parametrize("m,n", [(4096, 4096), (1024, 6144), (1024, 4096)])
def test_mfma_gemm_bf16_narrowing_bit_exact(hip, B, oracle, m, n):
    """The staged epilogues narrow f32 to bf16 with v_cvt_pk_bf16_f32 and set
    NaNs to the codec's 0x7fc0.  Here every output is an exact f32 sum
    x + y (A rows [1, 1, 0 ...], Bt rows [x, y, 0 ...], k = 64) chosen on
    RNE's edge cases, so the narrowed output must equal the oracle's
    f32_to_bf16 of x + y bit for bit (256x256 tiles at 4096 x 4096, 128x192
    at 1024 x 6144, 128x128 at 1024 x 4096)."""
    say("mfma gemm bf16 narrowing", m, n)
    rng = np.random.default_rng(m + n)
    K = 64
    xb, yb = _narrowing_cases(oracle, rng, n)
    a = np.zeros((m, K), dtype=np.uint16)
    a[:, 0] = a[:, 1] = 0x3F80
    bt = np.zeros((n, K), dtype=np.uint16)
    bt[:, 0], bt[:, 1] = xb, yb
    dst = torch.full((m, n), 0x1234, dtype=torch.int16, device="cuda")
    hip.gemm_mfma(u16(a), u16(bt), dst, m, K, n, in_fmt=B.BF16, out_fmt=B.BF16, rhs_t=True)
    got = host(dst).view(np.uint16)
    exact = (oracle.to_float(B.BF16, xb).astype(np.float64) + oracle.to_float(B.BF16, yb).astype(np.float64))
    assert np.all(np.isnan(exact) | np.isinf(exact) | (exact.astype(np.float32).astype(np.float64) == exact))
    want = oracle.f32_to_bf16(exact.astype(np.float32)).reshape(n)
    assert np.array_equal(got[0], want), np.nonzero(got[0] != want)[0][:8]
    assert np.array_equal(got, np.broadcast_to(want, got.shape))


def _f16_narrowing_cases(rng, n):
    """f16 triples (x, y, z) whose exact f32 sum x + y + z * 2^-14 lands on
    the cases f16 RNE narrowing has to get right: ties to even, just below
    and above a tie, carries into the exponent, 65504 + 16 (ties to inf) and
    65504 + 8 (stays finite), subnormal results that tie, round up or
    underflow to a signed zero (x a subnormal input, z * 2^-14 a fraction of
    the smallest subnormal), infinities and NaNs."""
    e = rng.integers(-10, 16, n)
    mant = rng.integers(0, 1024, n)
    sign = rng.choice([-1.0, 1.0], n)
    x = sign * (1.0 + mant / 1024.0) * np.exp2(e.astype(np.float64))
    half = np.exp2(e - 11.0)
    kind = rng.integers(0, 5, n)
    y = sign * np.select([kind == 0, kind == 1, kind == 2, kind == 3], [half, 0.75 * half, 1.5 * half, -half],
                         0.375 * half)
    z = np.zeros(n)
    x[:64] = sign[:64] * 65504.0
    y[:32] = sign[:32] * 16.0
    y[32:64] = sign[32:64] * 8.0
    sub = slice(72, 200)
    x[sub] = sign[sub] * rng.integers(0, 1024, 128) * 2.0 ** -24
    x[72:80] = sign[72:80] * 0.0                                   # the sum alone: underflow to a signed zero
    y[sub] = 0.0
    z[sub] = sign[sub] * rng.choice([2.0 ** -11, 1.5 * 2.0 ** -11, 2.0 ** -12, 0.75 * 2.0 ** -11], 128)
    bits = [v.astype(np.float16).view(np.uint16) for v in (x, y, z)]
    for v, b in zip((x, y, z), bits):
        assert np.array_equal(b.view(np.float16).astype(np.float64), v)  # every operand is an f16 value
    bits[0][64:72] = [0x7C00, 0xFC00, 0x7E00, 0x7D01, 0xFE13, 0x7C01, 0x0000, 0x8000]  # inf, NaN payloads, zeros
    return bits


@pytest.mark.parametrize("m,n", [(4096, 4096), (1024, 6144), (1024, 4096)])
def test_mfma_gemm_f16_narrowing_bit_exact(hip, B, oracle, m, n):
    """The staged epilogues narrow f32 to f16 with the hardware conversion
    (RNE, overflow to inf, gradual underflow) and set NaNs to the codec's
    0x7e00.  Every output is an exact f32 sum x + y + z * 2^-14 (A rows
    [1, 1, 2^-14, 0 ...], Bt rows [x, y, z, 0 ...], k = 64) chosen on RNE's
    edge cases, so the narrowed output must equal the oracle's f16 narrowing
    of that sum bit for bit; the subnormal x also pin that the f16 MFMA keeps
    subnormal inputs (256x256 tiles at 4096 x 4096, 128x192 at 1024 x 6144,
    128x128 at 1024 x 4096)."""
    say("mfma gemm f16 narrowing", m, n)
    rng = np.random.default_rng(m + 3 * n)
    K = 64
    xb, yb, zb = _f16_narrowing_cases(rng, n)
    a = np.zeros((m, K), dtype=np.uint16)
    a[:, 0] = a[:, 1] = 0x3C00
    a[:, 2] = 0x0400
    bt = np.zeros((n, K), dtype=np.uint16)
    bt[:, 0], bt[:, 1], bt[:, 2] = xb, yb, zb
    dst = torch.full((m, n), 0x1234, dtype=torch.int16, device="cuda")
    hip.gemm_mfma(u16(a), u16(bt), dst, m, K, n, in_fmt=B.F16, out_fmt=B.F16, rhs_t=True)
    got = host(dst).view(np.uint16)
    f = [oracle.to_float(B.F16, v).astype(np.float64) for v in (xb, yb, zb)]
    with np.errstate(invalid="ignore"):
        exact = f[0] + f[1] + f[2] * 2.0 ** -14
    assert np.all(np.isnan(exact) | np.isinf(exact) | (exact.astype(np.float32).astype(np.float64) == exact))
    want = oracle.f32_to_f16(exact.astype(np.float32))
    assert np.array_equal(got[0], want), np.nonzero(got[0] != want)[0][:8]
    assert np.array_equal(got, np.broadcast_to(want, got.shape))


@pytest.mark.parametrize("m,n,out,K", [(1024, 6144, 3, 256), (1024, 6144, 5, 256), (512, 12288, 3, 256),
                                       (1024, 6144, 3, 320), (1024, 6144, 5, 64)])
def test_mfma_gemm_192_tiles_vs_formal(hip, B, oracle, m, n, out, K):
    """Shapes that take the 128x192 tiles (one round of 256 workgroups where
    128x128 tiles need two: the decoder layer's QKV projection); k = 320 and
    64 give an odd number of 128-byte K stages and a single one.
    Sampled rows against the GPU formal lane (pinned to the CPU oracle on two
    rows), every output written; MFMA GEMM tolerances."""
    say("mfma gemm 128x192 tiles", m, n, out, K)
    rng = np.random.default_rng(m + n + out + K)
    a = oracle.f32_to_bf16(rng.standard_normal((m, K)).astype(np.float32)).reshape(m, K)
    bt = oracle.f32_to_bf16((rng.standard_normal((n, K)) / math.sqrt(K)).astype(np.float32)).reshape(n, K)
    ad, bd = u16(a), u16(bt)
    if out == B.F32:
        dst = torch.full((m, n), 7.5, dtype=torch.float32, device="cuda")
    else:
        dst = torch.full((m, n), 0x1234, dtype=torch.int16, device="cuda")
    hip.gemm_mfma(ad, bd, dst, m, K, n, in_fmt=B.BF16, out_fmt=out, rhs_t=True)
    got_all = host(dst)
    rows = np.concatenate([[0, 1, 127, 128, m - 1], rng.choice(m, 27, replace=False)])
    sub = np.ascontiguousarray(a[rows])
    ref_d = torch.zeros((len(rows), n), dtype=torch.float32, device="cuda")
    hip.gemm(u16(sub), bd, ref_d, len(rows), K, n, in_fmt=B.BF16, out_fmt=B.F32, rhs_t=True)
    ref = host(ref_d)
    cpu = oracle.gemm_formal(B.BF16, oracle.F32, np.ascontiguousarray(sub[:2]), bt, 2, K, n, rhs_t=True)
    assert np.array_equal(cpu.reshape(2, n).view(np.uint32), ref[:2].view(np.uint32))
    if out == B.F32:
        got = got_all[rows]
        tol_rel, tol_max = 1e-5, 1e-4
        assert not np.any(got_all == 7.5)
    else:
        got = oracle.to_float(B.BF16, got_all[rows].view(np.uint16)).reshape(len(rows), n)
        tol_rel, tol_max = 2e-3, 2e-2
        assert int(np.count_nonzero(got_all.view(np.uint16) == 0x1234)) < 64
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= tol_rel and np.abs(got - ref).max() <= tol_max * np.abs(ref).max(), (rel,)


@pytest.mark.parametrize("m,k,n,fmt,inplace,special", [
    (1024, 512, 4096, 3, False, False), (1024, 256, 6144, 3, True, False), (4096, 256, 4096, 3, False, True),
    (300, 128, 257, 3, False, True), (512, 256, 1024, 2, True, False), (4096, 256, 4096, 2, False, True),
    (1024, 256, 6144, 2, False, True), (77, 64, 130, 2, False, True), (512, 8192, 1024, 3, False, True),
    (512, 8192, 1024, 2, True, True), (1024, 14336, 4096, 3, False, False)])
def test_mfma_gemm_residual_equals_gemm_then_add(hip, B, m, k, n, fmt, inplace, special):
    """wafer_hip_gemm_mfma_residual gives the bits of the narrowed MFMA GEMM
    followed by the Add command: 128x128, 128x192 and 256x256 tiles with the
    staged epilogue, ragged shapes with the per-element one, split-K with the
    residual added by the fold launch (k 8192 and the decoder layer's down
    projection), in place (dst = residual) and not.  The special cases plant residuals at the
    format's largest finite value (sums that round to inf), infinities, NaNs
    and subnormals, so the epilogue's narrowing meets every rounding edge."""
    say("gemm residual", m, k, n, fmt, inplace, special)
    dt = torch.bfloat16 if fmt == B.BF16 else torch.float16
    gen = torch.Generator(device="cuda").manual_seed(m + k + n + fmt)
    a = torch.randn(m, k, generator=gen, device="cuda").to(dt)
    bt = (torch.randn(n, k, generator=gen, device="cuda") / math.sqrt(k)).to(dt)
    res = torch.randn(m, n, generator=gen, device="cuda").to(dt)
    if special:
        fi = torch.finfo(dt)
        res[0::7, 0::5] = fi.max
        res[1::7, 1::5] = -fi.max
        res[2::7, 2::5] = float("inf")
        res[3::7, 3::5] = float("nan")
        res[4::7, 0::3] = fi.smallest_normal / 4
        res[5::7, 1::3] = -fi.smallest_normal * 3 / 8
    prod = torch.empty(m, n, dtype=dt, device="cuda")
    hip.gemm_mfma(a, bt, prod, m, k, n, in_fmt=fmt, out_fmt=fmt, rhs_t=True)
    ref = torch.empty_like(prod)
    hip.elementwise(B.EW["Add"], fmt, prod, ref, res)
    if inplace:
        out = res.clone()
        hip.gemm_mfma_residual(a, bt, out, out, m, k, n, in_fmt=fmt, rhs_t=True)
    else:
        out = torch.full_like(res, 7.0)
        hip.gemm_mfma_residual(a, bt, res, out, m, k, n, in_fmt=fmt, rhs_t=True)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("m,k,n", [(1024, 128, 6144), (1024, 128, 28672)])
def test_i8_gemm_192_tiles_and_strips_bit_exact(hip, B, oracle, m, k, n):
    """int8 on the 128x192 tiles (n 6144) and on 448 256x256 tiles, whose
    workgroups walk per-XCD column strips (n 28672): y-only and acc_out runs,
    bit-exact against int64 products on sampled rows and a column checksum of
    the whole accumulator."""
    say("i8 gemm 192 tiles / strips", m, k, n)
    rng = np.random.default_rng(m + k + n)
    a = rng.integers(-128, 128, size=(m, k), dtype=np.int64).astype(np.int8)
    bt = rng.integers(-128, 128, size=(n, k), dtype=np.int64).astype(np.int8)
    scale = rng.uniform(0.001, 0.01, size=n).astype(np.float32)
    ad, bd, sd = dev(a), dev(bt), dev(scale)
    y = torch.full((m, n), 0x1234, dtype=torch.int16, device="cuda")
    hip.gemm_i8(ad, bd, sd, y, m, k, n, rhs_t=True)
    acc = torch.zeros((m, n), dtype=torch.int32, device="cuda")
    y2 = torch.zeros((m, n), dtype=torch.int16, device="cuda")
    hip.gemm_i8(ad, bd, sd, y2, m, k, n, acc_out=acc, rhs_t=True)
    gy, gy2, gacc = host(y).view(np.uint16), host(y2).view(np.uint16), host(acc)
    assert np.array_equal(gy, gy2)
    assert np.array_equal(gacc.astype(np.int64).sum(axis=0), a.astype(np.int64).sum(axis=0) @ bt.T.astype(np.int64))
    rows = np.concatenate([[0, 1, 127, 128, m - 1], rng.choice(m, 11, replace=False)])
    sub = np.ascontiguousarray(a[rows])
    acc_ref, y_ref = oracle.gemm_i8(sub, bt, scale, len(rows), k, n, rhs_t=True)
    assert np.array_equal(gacc[rows], acc_ref)
    assert np.array_equal(gy[rows], y_ref)


@pytest.mark.parametrize("m,k,n,rt,fmt", [(100, 96, 130, 0, 3), (1, 32, 1, 1, 2), (300, 256, 257, 1, 3),
                                          (77, 512, 384, 0, 2), (200, 160, 72, 0, 3), (513, 64, 129, 1, 3)])
def test_mfma_gemm_ragged_vs_formal(hip, B, oracle, m, k, n, rt, fmt):
    """m, n that the 128x128 tiles do not divide, with canary tails after the
    outputs; same tolerances as the aligned cases."""
    say("mfma gemm ragged", m, k, n, rt, fmt)
    rng = np.random.default_rng(11 * m + 13 * k + n + rt)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((k, n)) / math.sqrt(k)).astype(np.float32)
    if fmt == B.BF16:
        ah, bh = oracle.f32_to_bf16(a).reshape(a.shape), oracle.f32_to_bf16(b).reshape(b.shape)
    else:
        ah, bh = a.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    bt = np.ascontiguousarray(bh.T) if rt else bh
    ref = oracle.gemm_formal(fmt, oracle.F32, ah, bt, m, k, n, rhs_t=bool(rt)).reshape(m, n)
    pad = 2048
    out = torch.full((m * n + pad,), 7.5, dtype=torch.float32, device="cuda")
    hip.gemm_mfma(u16(ah), u16(bt), out, m, k, n, in_fmt=fmt, out_fmt=B.F32, rhs_t=bool(rt))
    go = host(out)
    got = go[:m * n].reshape(m, n)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= 1e-5 and np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
    assert np.all(go[m * n:] == 7.5)
    outn = torch.full((m * n + pad,), 0x1234, dtype=torch.int16, device="cuda")
    hip.gemm_mfma(u16(ah), u16(bt), outn, m, k, n, in_fmt=fmt, out_fmt=fmt, rhs_t=bool(rt))
    gn = host(outn).view(np.uint16)
    gf = oracle.to_float(fmt, gn[:m * n]).reshape(m, n)
    rel = np.linalg.norm(gf - ref) / np.linalg.norm(ref)
    assert rel <= 2e-3 and np.abs(gf - ref).max() <= 2e-2 * np.abs(ref).max()
    assert np.all(gn[m * n:] == 0x1234)


# ------------------------------------------------------------------ attention
def _bf16_randn(oracle, rng, shape):
    return oracle.f32_to_bf16(rng.standard_normal(shape).astype(np.float32)).reshape(shape)


@pytest.mark.parametrize("Bn,Hq,Hkv,S,causal", [(1, 2, 2, 256, True), (1, 2, 2, 256, False), (2, 4, 1, 384, True),
                                               (1, 8, 2, 128, True), (1, 1, 1, 640, False)])
def test_fa_prefill_vs_oracle(hip, B, oracle, Bn, Hq, Hkv, S, causal):
    say("fa prefill", Bn, Hq, Hkv, S, causal)
    rng = np.random.default_rng(S + Hq + causal)
    D = 128
    q, k, v = (_bf16_randn(oracle, rng, (Bn, hh, S, D)) for hh in (Hq, Hkv, Hkv))
    scale = 1.0 / math.sqrt(D)
    ref = oracle.attention_prefill(q, k, v, scale, causal=causal, block_k=64)
    o = torch.zeros((Bn, Hq, S, D), dtype=torch.int16, device="cuda")
    hip.attention_prefill(u16(q), u16(k), u16(v), o, scale, causal=causal)
    got = oracle.bf16_to_f32(from_u16(o)).reshape(o.shape)
    attention_gate(got, oracle.bf16_to_f32(ref).reshape(ref.shape), what="FA vs oracle")


@pytest.mark.parametrize("Bn,Hq,Hkv,Sq,Skv,causal", [(1, 4, 2, 256, 448, True), (2, 2, 2, 128, 320, False),
                                                     (1, 2, 1, 384, 640, True)])
def test_fa_prefill_longer_kv_vs_oracle(hip, B, oracle, Bn, Hq, Hkv, Sq, Skv, causal):
    """kv_len above q_len (a cached prefix): an odd number of 64-key blocks, so
    the two key halves of a phase get unequal block counts; causal masking is
    aligned at key 0 (key j visible to query i iff j <= i), as in the oracle."""
    say("fa prefill longer kv", Bn, Hq, Hkv, Sq, Skv, causal)
    rng = np.random.default_rng(Sq * 7 + Skv + causal)
    D = 128
    q = _bf16_randn(oracle, rng, (Bn, Hq, Sq, D))
    k, v = (_bf16_randn(oracle, rng, (Bn, Hkv, Skv, D)) for _ in range(2))
    scale = 1.0 / math.sqrt(D)
    ref = oracle.attention_prefill(q, k, v, scale, causal=causal, block_k=64)
    o = torch.zeros((Bn, Hq, Sq, D), dtype=torch.int16, device="cuda")
    hip.attention_prefill(u16(q), u16(k), u16(v), o, scale, causal=causal)
    got = oracle.bf16_to_f32(from_u16(o)).reshape(o.shape)
    attention_gate(got, oracle.bf16_to_f32(ref).reshape(ref.shape), what="FA (longer kv) vs oracle")


@pytest.mark.parametrize("Bn,Hq,Hkv,Sq,Skv,causal", [(1, 2, 2, 200, 200, True), (1, 3, 1, 77, 77, True),
                                                     (2, 2, 2, 130, 250, False), (1, 1, 1, 1, 1, True),
                                                     (1, 2, 1, 300, 100, True), (1, 1, 1, 64, 1000, False),
                                                     (1, 2, 2, 1000, 1000, True), (1, 2, 1, 17, 33, False)])
def test_fa_prefill_ragged_vs_oracle(hip, B, oracle, Bn, Hq, Hkv, Sq, Skv, causal):
    """Lengths that are not multiples of the 64-query / 64-key blocks: partial
    last query block (rows past q_len computed on a clamped row and never
    stored), partial last key block (zero-filled by the block's buffer range
    and masked), an odd number of query blocks (the middle block served alone),
    single-token sequences, and causal with kv_len below q_len (key j visible
    to query i iff j <= i and j < kv_len)."""
    say("fa prefill ragged", Bn, Hq, Hkv, Sq, Skv, causal)
    rng = np.random.default_rng(Sq * 13 + Skv * 3 + causal)
    D = 128
    q = _bf16_randn(oracle, rng, (Bn, Hq, Sq, D))
    k, v = (_bf16_randn(oracle, rng, (Bn, Hkv, Skv, D)) for _ in range(2))
    scale = 1.0 / math.sqrt(D)
    ref = oracle.attention_prefill(q, k, v, scale, causal=causal, block_k=64)
    # a canary row after the output: the kernel must not write past q_len
    n_out = Bn * Hq * Sq * D
    buf = torch.full((n_out + D,), 0x1234, dtype=torch.int16, device="cuda")
    hip.attention_prefill(u16(q), u16(k), u16(v), buf[:n_out].view(Bn, Hq, Sq, D), scale, causal=causal)
    oh = host(buf)
    got = oracle.bf16_to_f32(oh[:n_out].copy().view(np.uint16)).reshape(Bn, Hq, Sq, D)
    attention_gate(got, oracle.bf16_to_f32(ref).reshape(ref.shape), what="FA (ragged) vs oracle")
    assert (oh[n_out:] == 0x1234).all()


def test_fa_prefill_baseline_config(hip, B, oracle):
    """[1,16,2048,128] bf16 causal.  All heads against a
    torch float32 attention on the GPU (independent check); two heads
    against the CPU oracle."""
    say("fa prefill baseline config")
    rng = np.random.default_rng(20260803)
    Bn, H, S, D = 1, 16, 2048, 128
    q, k, v = (_bf16_randn(oracle, rng, (Bn, H, S, D)) for _ in range(3))
    scale = 1.0 / math.sqrt(D)
    o = torch.zeros((Bn, H, S, D), dtype=torch.int16, device="cuda")
    qd, kd, vd = u16(q), u16(k), u16(v)
    hip.attention_prefill(qd, kd, vd, o, scale, causal=True)
    got = oracle.bf16_to_f32(from_u16(o)).reshape(o.shape)
    qf, kf, vf = (torch.from_numpy(oracle.bf16_to_f32(t).reshape(t.shape)).cuda() for t in (q, k, v))
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scale
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool, device="cuda"), 1), float("-inf"))
    ref = torch.matmul(torch.softmax(s, -1), vf)
    attention_gate(got, host(ref), what="FA vs torch f32")
    heads = [0, 11]
    ro = oracle.attention_prefill(q[:, heads], k[:, heads], v[:, heads], scale, causal=True, block_k=64)
    attention_gate(got[:, heads], oracle.bf16_to_f32(ro).reshape(ro.shape), what="FA vs oracle (2 heads)")


def test_fa_prefill_gqa_equals_repeated_kv(hip, B, oracle):
    say("fa gqa == mha")
    rng = np.random.default_rng(9)
    q = _bf16_randn(oracle, rng, (1, 8, 256, 128))
    k = _bf16_randn(oracle, rng, (1, 2, 256, 128))
    v = _bf16_randn(oracle, rng, (1, 2, 256, 128))
    o1 = torch.zeros((1, 8, 256, 128), dtype=torch.int16, device="cuda")
    o2 = torch.zeros_like(o1)
    hip.attention_prefill(u16(q), u16(k), u16(v), o1, 0.088, causal=True)
    hip.attention_prefill(u16(q), u16(np.repeat(k, 4, 1)), u16(np.repeat(v, 4, 1)), o2, 0.088, causal=True)
    assert np.array_equal(host(o1), host(o2))


@pytest.mark.parametrize("Bn,Hq,Hkv,L,cap,chunks", [(2, 8, 2, 1024, 1024, 16), (1, 4, 4, 777, 1000, 16),
                                                   (3, 8, 1, 100, 128, 16), (1, 16, 2, 4096, 4096, 4),
                                                   (2, 4, 2, 513, 600, 1)])
def test_fd_decode_vs_oracle(hip, B, oracle, Bn, Hq, Hkv, L, cap, chunks):
    say("fd decode", Bn, Hq, Hkv, L, cap, chunks)
    rng = np.random.default_rng(L + chunks)
    D = 128
    q = _bf16_randn(oracle, rng, (Bn, Hq, 1, D))
    k = _bf16_randn(oracle, rng, (Bn, Hkv, cap, D))
    v = _bf16_randn(oracle, rng, (Bn, Hkv, cap, D))
    scale = 1.0 / math.sqrt(D)
    ref = oracle.attention_decode(q, k, v, scale, chunks=chunks, kv_len=L, block_k=64)
    o = torch.zeros((Bn, Hq, 1, D), dtype=torch.int16, device="cuda")
    hip.attention_decode(u16(q), u16(k), u16(v), o, scale, chunks=chunks, kv_len=L)
    got = oracle.bf16_to_f32(from_u16(o)).reshape(o.shape)
    attention_gate(got, oracle.bf16_to_f32(ref).reshape(ref.shape), what="FD vs oracle")


def test_fd_decode_baseline_config(hip, B, oracle):
    """Q [32,32,1,128], K/V [32,8,8192,128], 16 chunks.
    Four batches against the oracle, all batches against FA on the same
    single query (FD == FA within tolerance)."""
    say("fd decode baseline config")
    Bn, Hq, Hkv, L, D = 32, 32, 8, 8192, 128
    gen = torch.Generator(device="cuda").manual_seed(20260803)
    q = torch.randn((Bn, Hq, 1, D), device="cuda", generator=gen).to(torch.bfloat16)
    k = torch.randn((Bn, Hkv, L, D), device="cuda", generator=gen).to(torch.bfloat16)
    v = torch.randn((Bn, Hkv, L, D), device="cuda", generator=gen).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    o = torch.zeros((Bn, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    hip.attention_decode(q, k, v, o, scale, chunks=16)
    got = host(o.float())
    sel = [0, 7, 19, 31]
    qs, ks, vs = (host(t[sel].contiguous().view(torch.int16)).view(np.uint16) for t in (q, k, v))
    ref = oracle.attention_decode(qs, ks, vs, scale, chunks=16, block_k=64)
    attention_gate(got[sel], oracle.bf16_to_f32(ref).reshape(ref.shape), what="FD vs oracle (4 batches)")
    # all batches: float32 softmax attention on the GPU with GQA expansion
    kf = k.float().repeat_interleave(Hq // Hkv, dim=1)
    vf = v.float().repeat_interleave(Hq // Hkv, dim=1)
    s = torch.matmul(q.float(), kf.transpose(-1, -2).contiguous()) * scale
    ref_all = torch.matmul(torch.softmax(s, -1), vf)
    attention_gate(got, host(ref_all), what="FD vs torch f32 (all)")


# ------------------------------------------------------------------ managed lane
EXACT_OPS = ["Abs", "Neg", "Recip", "Square", "Max", "Min", "Add", "Sub", "Mul", "Relu", "Sqrt", "Rsqrt"]
TRANS_OPS = ["Log2", "Ln", "Pow2", "Exp", "ExpLp", "Sin", "Cos", "Tanh", "Sigmoid", "Softplus"]


@pytest.mark.parametrize("fmt", [5, 3, 2])
def test_elementwise_vs_oracle(hip, B, oracle, fmt):
    say("elementwise", fmt)
    rng = np.random.default_rng(fmt)
    n = 4099
    a = (rng.standard_normal(n) * 3).astype(np.float32)
    b = (rng.standard_normal(n) * 3).astype(np.float32)
    pos = (np.abs(a) + 0.05).astype(np.float32)
    enc = (lambda x: x) if fmt == B.F32 else (
        (lambda x: oracle.f32_to_bf16(x)) if fmt == B.BF16 else (lambda x: x.astype(np.float16).view(np.uint16)))
    todev = dev if fmt == B.F32 else u16
    for name in EXACT_OPS + TRANS_OPS:
        op = B.EW[name]
        src = pos if name in ("Sqrt", "Rsqrt", "Log2", "Ln") else a
        ea, eb = enc(src), enc(b)
        binary = name in ("Max", "Min", "Add", "Sub", "Mul")
        ref = oracle.elementwise(op, fmt, ea, eb if binary else None)
        out = torch.zeros(n, dtype=torch.float32 if fmt == B.F32 else torch.int16, device="cuda")
        hip.elementwise(op, fmt, todev(ea), out, in1=todev(eb) if binary else None)
        got = host(out)
        if fmt != B.F32:
            got = got.view(np.uint16)
        if name in EXACT_OPS:
            assert np.array_equal(got, ref), name
        else:
            gf, rf = oracle.to_float(fmt, got), oracle.to_float(fmt, ref)
            tol = 2e-6 if fmt == B.F32 else (8e-3 if fmt == B.BF16 else 1e-3)
            close = np.abs(gf - rf) <= tol * np.abs(rf) + 1e-30 + (tol if name in ("Sin", "Cos") else 0)
            assert np.all((gf == rf) | close), name


def test_elementwise_rejects_outside_managed_domain(hip, B):
    t = torch.zeros(8, dtype=torch.float32, device="cuda")
    for name in ("Eq", "LogicAnd", "SatRelu", "LeakyRelu"):
        with pytest.raises(B.WaferHipError) as e:
            hip.elementwise(B.EW[name], B.F32, t, t, in1=t)
        assert e.value.status == -3


def test_convert_routes_vs_oracle(hip, B, oracle, goldens):
    say("convert")
    rng = np.random.default_rng(12)
    f = (rng.standard_normal(5000) * 1000).astype(np.float32)
    f[:10] = [0.0, -0.0, 1.5, 2.5, -2.5, 65504.0, 65520.0, 1e-8, 3.4e38, -1e-40]
    bits = [h(x) for x in goldens["bf16_samples"]["input_f32"]]
    f[10:10 + len(bits)] = np.array(bits, np.uint32).view(np.float32)
    i32 = rng.integers(-2**31, 2**31, size=5000, dtype=np.int64).astype(np.int32)
    i32[:6] = [0, 1, -1, 16777217, 2**31 - 1, -2**31]
    i16 = rng.integers(-32768, 32768, size=5000, dtype=np.int64).astype(np.int16)
    cases = [(167, f, B.BF16), (166, f, B.F16), (149, i32, B.F32), (148, i32, B.BF16), (147, i32, B.F16),
             (145, i16, B.F32), (144, i16, B.BF16), (143, i16, B.F16),
             (155, oracle.f32_to_bf16(f), B.F32), (161, np.abs(f).astype(np.float16).view(np.uint16), B.F32),
             (154, oracle.f32_to_bf16(f), B.F16), (160, f.astype(np.float16).view(np.uint16), B.BF16),
             (165, np.clip(f, -1e9, 1e9), B.I32), (164, np.clip(f, -3e4, 3e4), B.I16)]
    for opcode, src, dfmt in cases:
        ref = oracle.convert(opcode, src, dfmt)
        sd = dev(src.view(np.int16)) if src.dtype == np.uint16 else dev(src)
        odt = {B.F32: torch.float32, B.BF16: torch.int16, B.F16: torch.int16, B.I32: torch.int32, B.I16: torch.int16}[dfmt]
        out = torch.zeros(src.size, dtype=odt, device="cuda")
        hip.convert(opcode, sd, out)
        got = host(out)
        assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), opcode
    with pytest.raises(B.WaferHipError):
        hip.convert(165, dev(np.array([np.inf], np.float32)), torch.zeros(1, dtype=torch.int32, device="cuda"))


@pytest.mark.parametrize("shape", [[1, 2, 3, 1031], [4, 5, 6, 7], [3, 64], [2, 3, 4, 5, 6]])
def test_reduce_vs_oracle_bit_exact(hip, B, oracle, goldens, shape):
    say("reduce", shape)
    rng = np.random.default_rng(len(shape) + shape[-1])
    x = rng.standard_normal(shape).astype(np.float32)
    for op in (0, 1, 2):
        for dim in (0, 1, 2, 3, 4, 5):
            rank = len(shape)
            if (dim <= 3 and dim >= rank) or (dim >= 4 and rank < 3):
                continue
            for fmt in ((B.F32,) if op == 0 else (B.F32, B.BF16)):
                src = x if fmt == B.F32 else oracle.f32_to_bf16(x).reshape(shape)
                ref = oracle.reduce(op, dim, fmt, shape, src)
                out = torch.zeros(ref.size, dtype=torch.float32 if fmt == B.F32 else torch.int16, device="cuda")
                hip.reduce(op, dim, fmt, shape, dev(src) if fmt == B.F32 else u16(src), out)
                got = host(out)
                assert np.array_equal(got.view(np.uint8), ref.ravel().view(np.uint8)), (op, dim, fmt)
    g = goldens["reduce_sum_ncx"]
    src = np.array([h(v) for v in g["input"]], np.uint32).view(np.float32)
    out = torch.zeros(2, dtype=torch.float32, device="cuda")
    hip.reduce(0, g["dim"], B.F32, g["shape"], dev(src), out)
    assert [int(v) for v in host(out).view(np.uint32)] == [h(v) for v in g["expect"]]


@pytest.mark.parametrize("fmt", [0, 2, 3, 5, 11])
@pytest.mark.parametrize("layout", [0, 2, 3])
@pytest.mark.parametrize("shape", [[5], [3, 1], [2, 3, 33], [1, 2, 3, 1025], [2, 2, 130], [3, 96], [2, 1, 129],
                                   [4, 8, 64, 200]])
def test_codec_vs_oracle(hip, B, oracle, fmt, layout, shape):
    nbytes = B.physical_bytes(fmt, layout, shape)
    geo = oracle.geometry(fmt, layout, shape)
    assert nbytes == geo["physical_bytes"]
    rng = np.random.default_rng(sum(shape) + fmt + layout)
    dt = oracle.storage_dtype(fmt)
    count = int(np.prod(shape))
    logical = rng.integers(0, 120, size=count).astype(dt)
    template = rng.integers(0, 256, size=nbytes).astype(np.uint8)
    ref = oracle.pack(fmt, layout, shape, logical, template)
    st = dev(template)
    hip.pack(fmt, layout, shape, dev(logical), st)
    assert np.array_equal(host(st), ref)
    back = torch.zeros(count * np.dtype(dt).itemsize, dtype=torch.uint8, device="cuda")
    hip.unpack(fmt, layout, shape, dev(ref), back)
    assert np.array_equal(host(back).view(dt), logical)


# ------------------------------------------------------------------ fused regions
def test_regions_vs_oracle(hip, B, oracle):
    say("regions")
    rng = np.random.default_rng(31)
    x = rng.standard_normal((64, 4096)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    xb, wb = oracle.f32_to_bf16(x).reshape(x.shape), oracle.f32_to_bf16(w)
    y = torch.zeros(x.shape, dtype=torch.int16, device="cuda")
    hip.rmsnorm(u16(xb), u16(wb), y, 1e-5, fmt=B.BF16)
    ref = oracle.rmsnorm(xb, wb, 1e-5)
    attention_gate(oracle.bf16_to_f32(from_u16(y)), oracle.bf16_to_f32(ref), what="rmsnorm")
    yf = torch.zeros(x.shape, dtype=torch.float32, device="cuda")
    hip.rmsnorm(dev(x), dev(w), yf, 1e-5, fmt=B.F32)
    rf = oracle.rmsnorm(x, w, 1e-5, fmt=oracle.F32)
    assert np.allclose(host(yf), rf, rtol=2e-6, atol=1e-7)
    hip.softmax(u16(xb), y, fmt=B.BF16)
    attention_gate(oracle.bf16_to_f32(from_u16(y)), oracle.bf16_to_f32(oracle.softmax(xb)), what="softmax")
    g, u = x[:, :2048].copy(), x[:, 2048:].copy()
    gb, ub = oracle.f32_to_bf16(g).reshape(g.shape), oracle.f32_to_bf16(u).reshape(u.shape)
    ys = torch.zeros(g.shape, dtype=torch.int16, device="cuda")
    hip.silu_mul(u16(gb), u16(ub), ys, fmt=B.BF16)
    attention_gate(oracle.bf16_to_f32(from_u16(ys)), oracle.bf16_to_f32(oracle.silu_mul(gb, ub)), what="swiglu")
    yg = torch.zeros(x.shape, dtype=torch.float32, device="cuda")
    hip.gelu_tanh(dev(x), yg, fmt=B.F32)
    rg = oracle.gelu_tanh(x, fmt=oracle.F32)
    assert np.all(np.abs(host(yg) - rg) <= 1e-5 * np.abs(rg) + 1e-6)
    T, H, D = 1024, 8, 128
    xr = rng.standard_normal((T, H, D)).astype(np.float32)
    xrb = oracle.f32_to_bf16(xr).reshape(xr.shape)
    pos = np.arange(T, dtype=np.int32)
    yr = torch.zeros(xr.shape, dtype=torch.int16, device="cuda")
    hip.rope(u16(xrb), yr, dev(pos), 1e4, fmt=B.BF16)
    attention_gate(oracle.bf16_to_f32(from_u16(yr)), oracle.bf16_to_f32(oracle.rope(xrb, pos, 1e4)), what="rope")
    bias = rng.standard_normal(4096).astype(np.float32)
    yb = torch.zeros(x.shape, dtype=torch.float32, device="cuda")
    hip.bias_add(dev(x), dev(bias), yb, fmt=B.F32)
    assert np.array_equal(host(yb), oracle.bias_add(x, bias))


def test_bias_add_past_one_grid_stride(hip, B, oracle):
    """bias_add over more 8-element chunks than its grid has threads (65536
    workgroups of 256: 134,217,728 elements), so threads take a second chunk
    whose column comes from the stride's remainder; 4104 columns make that
    remainder wrap rows.  Bit-exact against torch's float32 add, which is the
    oracle's one IEEE binary32 Add per element (pinned against the oracle on
    the first and last rows)."""
    rows, cols = 32800, 4104
    say("bias_add past one grid stride", rows, cols)
    gen = torch.Generator(device="cuda").manual_seed(4104)
    x = torch.randn(rows, cols, generator=gen, device="cuda")
    bias = torch.randn(cols, generator=gen, device="cuda")
    y = torch.full_like(x, 7.5)
    hip.bias_add(x, bias, y, fmt=B.F32)
    torch.cuda.synchronize()
    assert torch.equal(y, x + bias)
    for r in (0, rows - 1):
        assert np.array_equal(host(y[r:r + 1]), oracle.bias_add(host(x[r:r + 1]), host(bias)))
    del x, y


@pytest.mark.parametrize("rows,cols,fmt", [(7, 8, 3), (33, 2048, 3), (5, 2056, 3), (9, 6000, 2), (3, 8192, 5),
                                           (4, 9000, 3), (2, 24, 5)])
def test_softmax_shapes(hip, B, oracle, rows, cols, fmt):
    """Register-resident softmax at 1, 2 and 4 chunks per thread (cols a
    multiple of 8 up to 8192, with a partial last chunk), the scalar kernel
    beyond (cols 2056 and 9000), all three float formats."""
    say("softmax", rows, cols, fmt)
    rng = np.random.default_rng(rows * cols + fmt)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    if fmt == B.F32:
        xs, y = dev(x), torch.zeros(x.shape, dtype=torch.float32, device="cuda")
        hip.softmax(xs, y, fmt=fmt)
        ref = oracle.softmax(x, fmt=oracle.F32)
        assert np.allclose(host(y), ref, rtol=2e-5, atol=1e-8)
        return
    xb = oracle.f32_to_bf16(x).reshape(x.shape) if fmt == B.BF16 else x.astype(np.float16).view(np.uint16)
    y = torch.zeros(x.shape, dtype=torch.int16, device="cuda")
    hip.softmax(u16(xb), y, fmt=fmt)
    attention_gate(oracle.to_float(fmt, from_u16(y)).reshape(x.shape),
                   oracle.to_float(fmt, oracle.softmax(xb, fmt=fmt)).reshape(x.shape), what="softmax")


@pytest.mark.parametrize("rows,cols", [(1, 8), (67, 520), (1024, 4096), (3, 4104), (5, 6152), (2, 8192), (2, 8200),
                                       (9, 33), (4096, 8), (4097, 520), (4099, 1024), (4098, 2056), (4096, 4096)])
@pytest.mark.parametrize("fmt", [3, 5, 2])
def test_rmsnorm_shapes(hip, B, oracle, rows, cols, fmt):
    """Below 4096 rows the register-resident row kernel at 1, 2 and 4 chunks
    per thread (up to 8192 columns, partial last chunks) and the two-pass
    workgroup kernel beyond 8192 columns, the scalar kernel (33 columns), and
    from 4096 rows the wave-per-row kernel at 1, 2, 4 and 8 chunks per lane
    (row counts that leave a workgroup's last waves idle); all three float
    formats against the oracle."""
    say("rmsnorm", rows, cols, fmt)
    rng = np.random.default_rng(rows * cols + fmt)
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    if fmt == B.F32:
        y = torch.zeros(x.shape, dtype=torch.float32, device="cuda")
        hip.rmsnorm(dev(x), dev(w), y, 1e-5, fmt=fmt)
        ref = oracle.rmsnorm(x, w, 1e-5, fmt=oracle.F32)
        assert np.allclose(host(y), ref, rtol=2e-6, atol=1e-7)
        return
    cv = (lambda a: oracle.f32_to_bf16(a).reshape(a.shape)) if fmt == B.BF16 else \
        (lambda a: a.astype(np.float16).view(np.uint16))
    xb, wb = cv(x), cv(w)
    y = torch.zeros(x.shape, dtype=torch.int16, device="cuda")
    hip.rmsnorm(u16(xb), u16(wb), y, 1e-5, fmt=fmt)
    attention_gate(oracle.to_float(fmt, from_u16(y)).reshape(x.shape),
                   oracle.to_float(fmt, oracle.rmsnorm(xb, wb, 1e-5, fmt=fmt)).reshape(x.shape), what="rmsnorm")


@pytest.mark.parametrize("rows,cols", [(1024, 4096), (67, 520), (5, 2056), (3, 4104), (5, 6152), (2, 8200), (9, 33),
                                       (4097, 520), (4096, 4096)])
@pytest.mark.parametrize("fmt", [3, 5, 2])
def test_add_rmsnorm_equals_add_then_rmsnorm(hip, B, rows, cols, fmt):
    """The fused residual Add + RMSNorm gives the bits of the Add command
    followed by the RMSNorm region, for both outputs: the row kernels (below
    4096 rows or above 4096 columns: register-resident up to 8192 columns,
    two-pass beyond), the wave-per-row kernel (from 4096 rows), and the
    two-launch path for columns not a multiple of 8."""
    say("add_rmsnorm", rows, cols, fmt)
    dt = {3: torch.bfloat16, 5: torch.float32, 2: torch.float16}[fmt]
    iv = torch.int32 if fmt == 5 else torch.int16
    gen = torch.Generator(device="cuda").manual_seed(rows * 7 + cols + fmt)
    x = torch.randn(rows, cols, generator=gen, device="cuda").to(dt)
    r = (0.5 * torch.randn(rows, cols, generator=gen, device="cuda")).to(dt)
    w = (1 + 0.1 * torch.randn(cols, generator=gen, device="cuda")).to(dt)
    s_ref, y_ref = torch.empty_like(x), torch.empty_like(x)
    hip.elementwise(B.EW["Add"], fmt, x, s_ref, r)
    hip.rmsnorm(s_ref, w, y_ref, 1e-5, fmt=fmt)
    s, y = torch.full_like(x, 3.0), torch.full_like(x, 3.0)
    hip.add_rmsnorm(x, r, w, s, y, 1e-5, fmt=fmt)
    torch.cuda.synchronize()
    assert torch.equal(s.view(iv), s_ref.view(iv))
    assert torch.equal(y.view(iv), y_ref.view(iv))


@pytest.mark.parametrize("T,H,D", [(300, 1, 128), (64, 32, 128), (129, 5, 16), (77, 3, 64), (10, 2, 6)])
def test_rope_shapes(hip, B, oracle, T, H, D):
    """RoPE with the angles taken once per (token, frequency) and applied to
    every head: one head, 32 heads, head_dim 16 (one 8-frequency group),
    64, and the scalar kernel (head_dim 6)."""
    say("rope", T, H, D)
    rng = np.random.default_rng(T * H + D)
    x = rng.standard_normal((T, H, D)).astype(np.float32)
    xb = oracle.f32_to_bf16(x).reshape(x.shape)
    pos = rng.integers(0, 4096, T).astype(np.int32)
    y = torch.zeros(x.shape, dtype=torch.int16, device="cuda")
    hip.rope(u16(xb), y, dev(pos), 1e4, fmt=B.BF16)
    attention_gate(oracle.bf16_to_f32(from_u16(y)).reshape(x.shape),
                   oracle.bf16_to_f32(oracle.rope(xb, pos, 1e4)).reshape(x.shape), what="rope")
    # f32: positions below 32, where one ulp of the device powf in the
    # inverse frequency moves the angle by < 2e-6 (at position 4096 it moves
    # it by ~2.4e-4, beyond any f32 bound)
    pos_s = (pos % 32).astype(np.int32)
    yf = torch.zeros(x.shape, dtype=torch.float32, device="cuda")
    hip.rope(dev(x), yf, dev(pos_s), 1e4, fmt=B.F32)
    rf = oracle.rope(x, pos_s, 1e4, fmt=oracle.F32)
    assert np.allclose(host(yf), rf, rtol=1e-5, atol=1e-5)


def test_invalid_arguments_fail_without_launch(hip, B):
    t96 = torch.zeros(96, dtype=torch.int16, device="cuda")
    with pytest.raises(B.WaferHipError) as e:
        hip.attention_prefill(*(t96.view(1, 1, 1, 96),) * 4, 0.1)
    assert e.value.status == -3  # head_dim 96 is not served (128, or 1..64)
    t = torch.zeros(16, dtype=torch.int16, device="cuda")
    with pytest.raises(B.WaferHipError):
        hip.gemm(t, t, t, 0, 1, 1)
    with pytest.raises(ValueError):  # operands smaller than the shape: caught before the C call
        hip.gemm_i8(t, t, t, t, 100, 64, 128)
    big = torch.zeros(4096, dtype=torch.int16, device="cuda")
    i8, f32 = torch.zeros(4096, dtype=torch.int8, device="cuda"), torch.zeros(64, dtype=torch.float32, device="cuda")
    with pytest.raises(B.WaferHipError) as e:
        hip.gemm_i8(i8, i8, f32, big, 1, 100, 1)
    assert e.value.status == -3  # k not a multiple of one 64-byte stage
    with pytest.raises(B.WaferHipError) as e:
        hip.gemm_mfma(big, big, big, 1, 40, 1, out_fmt=B.BF16)
    assert e.value.status == -3


def test_repeated_launches_carry_no_state(hip, B, oracle):
    """No launch leaves state for the next: repeated FA launches are
    bit-identical, and FD shapes run large, small, then large again (the
    chunk-state workspace reused at other sizes) all pass the gate."""
    say("repeated launches")
    rng = np.random.default_rng(77)
    q, k, v = (_bf16_randn(oracle, rng, (1, 4, 1024, 128)) for _ in range(3))
    outs = []
    for _ in range(3):
        o = torch.zeros((1, 4, 1024, 128), dtype=torch.int16, device="cuda")
        hip.attention_prefill(u16(q), u16(k), u16(v), o, 0.088, causal=True)
        outs.append(host(o))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])
    ref = oracle.attention_prefill(q, k, v, 0.088, causal=True, block_k=64)
    attention_gate(oracle.bf16_to_f32(outs[0].view(np.uint16)), oracle.bf16_to_f32(ref), what="FA repeated")
    for (Bn, Hq, Hkv, L) in [(8, 16, 4, 2048), (2, 4, 2, 300), (8, 16, 4, 2048)]:
        qd = _bf16_randn(oracle, rng, (Bn, Hq, 1, 128))
        kd = _bf16_randn(oracle, rng, (Bn, Hkv, L, 128))
        vd = _bf16_randn(oracle, rng, (Bn, Hkv, L, 128))
        o = torch.zeros((Bn, Hq, 1, 128), dtype=torch.int16, device="cuda")
        hip.attention_decode(u16(qd), u16(kd), u16(vd), o, 0.088, chunks=16)
        ref = oracle.attention_decode(qd, kd, vd, 0.088, chunks=16, block_k=64)
        attention_gate(oracle.bf16_to_f32(from_u16(o)), oracle.bf16_to_f32(ref), what=f"FD {Bn}x{L}")


@pytest.mark.parametrize("Bn,Hq,Hkv,L,chunks", [(64, 8, 4, 2048, 16), (48, 16, 4, 1000, 5), (64, 4, 4, 777, 16),
                                               (32, 8, 8, 513, 3)])
def test_fd_decode_group_path(hip, B, oracle, Bn, Hq, Hkv, L, chunks):
    """Large batch*kv_heads takes the one-workgroup-per-(batch, kv head)
    path (16 waves, waves split the chunks); ragged chunk lengths included."""
    say("fd group path", Bn, Hq, Hkv, L, chunks)
    rng = np.random.default_rng(L + Bn)
    q = _bf16_randn(oracle, rng, (Bn, Hq, 1, 128))
    k = _bf16_randn(oracle, rng, (Bn, Hkv, L, 128))
    v = _bf16_randn(oracle, rng, (Bn, Hkv, L, 128))
    ref = oracle.attention_decode(q, k, v, 0.088, chunks=chunks, block_k=64)
    o = torch.zeros((Bn, Hq, 1, 128), dtype=torch.int16, device="cuda")
    hip.attention_decode(u16(q), u16(k), u16(v), o, 0.088, chunks=chunks)
    attention_gate(oracle.bf16_to_f32(from_u16(o)), oracle.bf16_to_f32(ref), what="FD group path")


def test_gelu_tanh_error_bound(hip, B):
    """gelu_tanh evaluates 0.5*x*(1 + tanh(k0*(x + k1*x^3))) as
    x / (1 + 2^(c*(x + k1*x^3))), c = -2*log2(e)*k0 (the same function:
    1 + tanh(z) = 2 / (1 + e^(-2z))).  Bound, against a float64 evaluation
    of that function over every finite bf16 value and dense f32 samples:
    relative error <= 2^-24 * (8 + 3*|a|), a = c*(x + k1*x^3) the
    exponent (v_exp_f32 and v_rcp_f32 add about an ulp each; the rounding of
    the exponent's argument grows with |a|, and where |a| is large the
    output is below |x| * 2^-|a|); outputs below 1e-30 within 1e-34
    absolute.  Measured: 4 ulps for |x| < 1, 17 for |x| < 3, 238 at
    |x| = 10 (a = 126, output ~1e-37).  Special values map as in the tanh
    form: +inf -> +inf, -inf -> NaN, NaN -> NaN, signed zeros kept."""
    bits = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    rng = np.random.default_rng(940)
    x = np.concatenate([bits[np.isfinite(bits)], rng.uniform(-10, 10, 1 << 21).astype(np.float32),
                        rng.uniform(-1e-2, 1e-2, 1 << 18).astype(np.float32)])
    y = torch.empty(len(x), dtype=torch.float32, device="cuda")
    hip.gelu_tanh(torch.from_numpy(x).cuda(), y, fmt=B.F32)
    g = y.cpu().numpy().astype(np.float64)
    xd = x.astype(np.float64)
    k0, k1 = math.sqrt(2 / math.pi), 0.044715
    with np.errstate(all="ignore"):
        a = -2 * math.log2(math.e) * k0 * (xd + k1 * xd ** 3)
        exact = xd / (1 + np.exp2(a))
    fin = np.isfinite(exact)
    assert np.array_equal(np.isfinite(g), fin)
    big = fin & (np.abs(exact) > 1e-30)
    err = np.abs(g - exact)
    bound = 2.0 ** -24 * (8 + 3 * np.abs(a)) * np.abs(exact)
    assert np.all(err[big] <= bound[big]), float(np.max(err[big] / bound[big]))
    assert np.all(err[fin & ~big] <= 1e-34)
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan], np.float32)
    ys = torch.empty(len(sp), dtype=torch.float32, device="cuda")
    hip.gelu_tanh(torch.from_numpy(sp).cuda(), ys, fmt=B.F32)
    r = ys.cpu().numpy()
    assert r[0] == 0 and not np.signbit(r[0]) and r[1] == 0 and np.signbit(r[1])
    assert r[2] == np.inf and np.isnan(r[3]) and np.isnan(r[4])
