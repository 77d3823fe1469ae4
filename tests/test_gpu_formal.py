"""GPU parity for the formal-lane commands: wafer_hip_elementwise_formal
(broadcast scalar / unit / grouped right operands, relations with Bool or
numeric results, logic operations, the formal zero / NaN rules) and
wafer_hip_pool (Max / Min in every float format, F32 Sum), against the CPU
oracle (oracle_elementwise_formal / oracle_pool) on identical raw bits,
including the reference's own kernel-test cases
(unittests/Simulator/Kernel/TargetModelKernelTest.cpp:882-1213, 1657-1722)
and its rejections.  Bar: bit-exact.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

F16, BF16, F32, BOOL = 2, 3, 5, 7
FLOATS = (F16, BF16, F32)
ONE = {F16: 0x3C00, BF16: 0x3F80, F32: 0x3F800000}
TWO = {F16: 0x4000, BF16: 0x4000, F32: 0x40000000}
EW = dict(Abs=0, Recip=1, Square=2, Neg=5, Max=6, Min=7, Add=8, Sub=9, Mul=10, Eq=12, Ne=13, Ge=14, Gt=15, Le=16,
          Lt=17, LogicNot=18, LogicAnd=19, LogicOr=20, LogicXor=21, Relu=31)
BINARY = ("Max", "Min", "Add", "Sub", "Mul", "Eq", "Ne", "Ge", "Gt", "Le", "Lt")
UNARY = ("Abs", "Recip", "Square", "Neg", "Relu")


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


def dev_bits(fmt, a):
    a = np.ascontiguousarray(a)
    if fmt == F32:
        return torch.from_numpy(a.astype(np.uint32).view(np.int32)).cuda()
    if fmt == BOOL:
        return torch.from_numpy(a.astype(np.uint8)).cuda()
    return torch.from_numpy(a.astype(np.uint16).view(np.int16)).cuda()


def host_bits(t):
    a = t.cpu().numpy()
    if a.dtype == np.int32:
        return a.view(np.uint32)
    if a.dtype == np.int16:
        return a.view(np.uint16)
    return a


def empty_out(fmt, n, bool_out):
    if bool_out:
        return torch.full((n,), 0xA5, dtype=torch.uint8, device="cuda")
    return torch.full((n,), -1, dtype=torch.int32 if fmt == F32 else torch.int16, device="cuda")


def run_ew(hip, op, fmt, lhs, rhs=None, *, scalar=None, unit=0, group=0, numeric=False):
    bool_out = fmt == BOOL or (12 <= EW[op] <= 17 and not numeric)
    out = empty_out(fmt, lhs.size, bool_out)
    hip.elementwise_formal(EW[op], fmt, dev_bits(fmt, lhs), out, None if rhs is None else dev_bits(fmt, rhs),
                           scalar=scalar, unit=unit, group=group, numeric=numeric)
    torch.cuda.synchronize()
    return host_bits(out)


def random_bits(rng, fmt, n):
    """Raw bits over the whole encoding space, with zeros, infinities, NaN
    payloads, subnormals and small integers mixed in."""
    width = 32 if fmt == F32 else 16
    a = rng.integers(0, 1 << width, n, dtype=np.uint64)
    sign = 1 << (width - 1)
    special = {F32: [0, sign, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0xFFC12345, 1, sign | 1, 0x00800000,
                     0x3F800000, 0xBF800000, 0x7F7FFFFF],
               F16: [0, sign, 0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFE33, 1, sign | 1, 0x0400, 0x3C00, 0xBC00, 0x7BFF],
               BF16: [0, sign, 0x7F80, 0xFF80, 0x7FC0, 0x7F81, 0xFFC3, 1, sign | 1, 0x0080, 0x3F80, 0xBF80,
                      0x7F7F]}[fmt]
    pick = rng.integers(0, len(special), n // 4)
    a[: n // 4] = np.array(special, dtype=np.uint64)[pick]
    if fmt == F32:  # values near each other so sums and differences round
        ints = rng.integers(-300, 300, n // 2 - n // 4).astype(np.float32)
        a[n // 4: n // 2] = ints.view(np.uint32)
    rng.shuffle(a)
    return a.astype(np.uint32 if fmt == F32 else np.uint16)


@pytest.mark.parametrize("fmt", FLOATS)
@pytest.mark.parametrize("op", UNARY + BINARY)
def test_full_form_random_bits(hip, oracle, fmt, op):
    say("formal full", fmt, op)
    rng = np.random.default_rng(100 + fmt * 40 + EW[op])
    n = 70001
    lhs = random_bits(rng, fmt, n)
    rhs = random_bits(rng, fmt, n) if op in BINARY else None
    for numeric in ((False, True) if 12 <= EW[op] <= 17 else (False,)):
        got = run_ew(hip, op, fmt, lhs, rhs, numeric=numeric)
        want = oracle.elementwise_formal(EW[op], fmt, lhs, rhs, numeric=numeric)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, (op, fmt, numeric, [(hex(lhs[i]), hex(rhs[i]) if rhs is not None else None,
                                                   hex(got[i]), hex(want[i])) for i in bad[:5]])


@pytest.mark.parametrize("fmt", FLOATS)
@pytest.mark.parametrize("op", BINARY)
@pytest.mark.parametrize("unit", (1, 7, 32, 64))
def test_unit_and_scalar_forms(hip, oracle, fmt, op, unit):
    say("formal unit/scalar", fmt, op, unit)
    rng = np.random.default_rng(7 * unit + EW[op] + fmt)
    n = 2 * 1031 * 64 + 5
    lhs = random_bits(rng, fmt, n)
    rhs = random_bits(rng, fmt, unit)
    numeric = 12 <= EW[op] <= 17 and unit % 2 == 1
    got = run_ew(hip, op, fmt, lhs, rhs, unit=unit, numeric=numeric)
    want = oracle.elementwise_formal(EW[op], fmt, lhs, rhs, unit=unit, numeric=numeric)
    assert (got == want).all()
    scalar = int(rhs[0])
    got = run_ew(hip, op, fmt, lhs, scalar=scalar, numeric=numeric)
    want = oracle.elementwise_formal(EW[op], fmt, lhs, scalar=scalar, numeric=numeric)
    assert (got == want).all()


@pytest.mark.parametrize("fmt", FLOATS)
@pytest.mark.parametrize("extent", (1024, 1025, 1031))
@pytest.mark.parametrize("op", ("Add", "Sub", "Mul", "Max", "Min"))
def test_reference_grouped_broadcast(hip, oracle, fmt, extent, op):
    say("formal grouped", fmt, extent, op)
    count = 2 * extent * 64

    def bits(v):
        f = np.float32(v)
        if fmt == F32:
            return int(f.view(np.uint32))
        if fmt == F16:
            return int(np.float16(v).view(np.uint16))
        return int(f.view(np.uint32)) >> 16

    lhs_value = 1 if op == "Mul" else (256 if op == "Min" else 0)
    lhs = np.full(count, bits(lhs_value))
    rhs = np.array([bits(i + 1) for i in range(128)])
    got = run_ew(hip, op, fmt, lhs, rhs, unit=64, group=extent * 64).reshape(2, extent, 64)
    for g in range(2):
        want = np.array([bits((-1 if op == "Sub" else 1) * (g * 64 + lane + 1)) for lane in range(64)])
        assert (got[g] == want[None, :]).all()
    # random operands through the same grouped walk
    rng = np.random.default_rng(extent + EW[op])
    lhs = random_bits(rng, fmt, count)
    rhs = random_bits(rng, fmt, 128)
    assert (run_ew(hip, op, fmt, lhs, rhs, unit=64, group=extent * 64) ==
            oracle.elementwise_formal(EW[op], fmt, lhs, rhs, unit=64, group=extent * 64)).all()


@pytest.mark.parametrize("fmt", FLOATS)
@pytest.mark.parametrize("form", (0, 1, 2))
@pytest.mark.parametrize("numeric", (False, True))
def test_reference_relations(hip, fmt, form, numeric):
    say("formal relations", fmt, form, numeric)
    extent = 1031
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
            got = run_ew(hip, name, fmt, lhs, scalar=ONE[fmt], numeric=numeric)
        else:
            got = run_ew(hip, name, fmt, lhs, rhs, unit=32 if form == 2 else 0, numeric=numeric)
        assert (got == np.where(fn(a, b), ONE[fmt] if numeric else 1, 0)).all(), name


@pytest.mark.parametrize("fmt", FLOATS)
def test_reference_scalar_immediates(hip, fmt):
    say("formal scalar immediates", fmt)
    inf = {F32: 0xFF800000, F16: 0xFC00, BF16: 0xFF80}[fmt]
    lhs = np.full(2 * 1025 * 32, ONE[fmt])
    assert (run_ew(hip, "Mul", fmt, lhs, scalar=TWO[fmt]) == TWO[fmt]).all()
    assert (run_ew(hip, "Add", fmt, lhs, scalar=inf) == inf).all()


def test_logic_ops(hip, oracle, B):
    say("formal logic")
    rng = np.random.default_rng(3)
    a = rng.integers(0, 2, 100003).astype(np.uint8)
    b = rng.integers(0, 2, 100003).astype(np.uint8)
    for op in ("LogicAnd", "LogicOr", "LogicXor"):
        assert (run_ew(hip, op, BOOL, a, b) == oracle.elementwise_formal(EW[op], BOOL, a, b)).all()
    assert (run_ew(hip, "LogicNot", BOOL, a) == 1 - a).all()
    bad = a.copy()
    bad[77777] = 2
    with pytest.raises(B.WaferHipError) as e:
        run_ew(hip, "LogicAnd", BOOL, bad, b)
    assert e.value.status == -5


def test_rejections(hip, B):
    say("formal rejections")
    # raw byte tensors: the wrapper checks only their size, the library validates the command
    x = torch.zeros(512, dtype=torch.uint8, device="cuda")
    out = torch.zeros(512, dtype=torch.uint8, device="cuda")
    cases = [
        (dict(op=EW["Add"], fmt=F32, rhs=None), -1, "arity"),
        (dict(op=EW["Add"], fmt=F32, rhs=x, scalar=ONE[F32]), -1, "arity"),
        (dict(op=EW["Add"], fmt=F32, rhs=x, unit=65), -1, "1..64"),
        (dict(op=EW["Add"], fmt=F32, rhs=x, unit=64, group=63), -1, "grouped"),
        (dict(op=EW["Add"], fmt=F32, rhs=x, unit=64, group=192), -1, "grouped"),  # 128 % 192
        (dict(op=EW["Eq"], fmt=F32, rhs=x, unit=64, group=64), -1, "grouped"),
        (dict(op=EW["Add"], fmt=F32, rhs=x, numeric=True), -1, "relation output"),
        (dict(op=EW["Add"], fmt=F16, scalar=0x10000, rhs=None), -1, "scalar"),
        (dict(op=EW["Add"], fmt=BOOL, rhs=x), -1, "logic"),
        (dict(op=32, fmt=F32, rhs=None), -5, "formal subset"),  # SatRelu
        (dict(op=33, fmt=F32, rhs=None), -5, "formal subset"),  # LeakyRelu
        (dict(op=3, fmt=F32, rhs=None), -5, "formal subset"),  # Sqrt
        (dict(op=EW["Add"], fmt=4, rhs=x), -5, "formats"),  # I32
        (dict(op=11, fmt=F32, rhs=x), -1, "registered"),
    ]
    for kw, status, text in cases:
        op, fmt = kw.pop("op"), kw.pop("fmt")
        rhs = kw.pop("rhs")
        with pytest.raises(B.WaferHipError) as e:
            hip.elementwise_formal(op, fmt, x, out, rhs, count=128, **kw)
        assert e.value.status == status, (op, fmt, kw, str(e.value))
        assert text in str(e.value), (text, str(e.value))


def _pool(hip, op, fmt, src, dst_hw, ks):
    n, _, _, c = src.shape
    s = dev_bits(fmt, src.reshape(-1)).reshape(src.shape)
    d = empty_out(fmt, n * dst_hw[0] * dst_hw[1] * c, False).reshape(n, dst_hw[0], dst_hw[1], c)
    hip.pool(op, fmt, s, d, ks)
    torch.cuda.synchronize()
    return host_bits(d)


@pytest.mark.parametrize("width", (1024, 1025))
@pytest.mark.parametrize("kind", (117, 119, 116))
def test_reference_pool_windows(hip, width, kind):
    say("pool reference", width, kind)
    h, w, c = np.meshgrid(np.arange(5), np.arange(width + 2), np.arange(2), indexing="ij")
    src = (h * 8 + w + c).astype(np.float32).view(np.uint32)[None]
    got = _pool(hip, kind, F32, src, (2, width), (3, 2, 1, 2)).view(np.float32)[0]
    oh, ow, oc = np.meshgrid(np.arange(2), np.arange(width), np.arange(2), indexing="ij")
    first = (oh * 16 + ow + oc).astype(np.float32)
    want = first + 10 if kind == 117 else (first if kind == 119 else first * 6 + 30)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


# Sum pooling is F32-only (the other formats are refused: test_pool_rejections)
@pytest.mark.parametrize("fmt,kind", [(f, k) for f in FLOATS for k in (117, 119)] + [(F32, 116)])
@pytest.mark.parametrize("geom", ((2, 17, 23, 5, 3, 2, 2, 3), (1, 9, 9, 64, 3, 3, 1, 1), (3, 6, 40, 2, 1, 1, 3, 2),
                                  (1, 64, 64, 16, 2, 2, 2, 2)))
def test_pool_random(hip, oracle, fmt, kind, geom):
    n, h, w, c, kw, kh, sw, sh = geom
    say("pool random", fmt, kind, geom)
    rng = np.random.default_rng(sum(geom) + kind + fmt)
    src = random_bits(rng, fmt, n * h * w * c).reshape(n, h, w, c)
    oh, ow = (h - kh) // sh + 1, (w - kw) // sw + 1
    got = _pool(hip, kind, fmt, src, (oh, ow), (kw, kh, sw, sh))
    want = oracle.pool(kind, fmt, src, (oh, ow), (kw, kh, sw, sh))
    assert (got == want).all()


def test_pool_integer_single_window(hip, B):
    say("pool integer 1x1")
    src = np.arange(2 * 5 * 6 * 3, dtype=np.int32).reshape(2, 5, 6, 3)
    s = torch.from_numpy(src).cuda()
    d = torch.zeros((2, 3, 3, 3), dtype=torch.int32, device="cuda")
    hip.pool(117, 4, s, d, (1, 1, 2, 2))
    torch.cuda.synchronize()
    assert (d.cpu().numpy() == src[:, ::2, ::2, :]).all()
    with pytest.raises(B.WaferHipError) as e:
        hip.pool(117, 4, s, torch.zeros((2, 2, 3, 3), dtype=torch.int32, device="cuda"), (2, 2, 2, 2))
    assert e.value.status == -5


def test_pool_rejections(hip, B):
    say("pool rejections")
    s = dev_bits(F32, np.zeros(1 * 5 * 6 * 2, np.uint32)).reshape(1, 5, 6, 2)
    d = dev_bits(F32, np.zeros(1 * 2 * 4 * 2, np.uint32)).reshape(1, 2, 4, 2)
    cases = [
        (dict(op=117, fmt=F32, ks=(3, 2, 1, 2), pads=(1, 0, 0, 0)), -3, "explicit input padding"),
        (dict(op=118, fmt=F32, ks=(3, 2, 1, 2), indexed_destination=True), -3, "explicit input padding"),
        (dict(op=118, fmt=F32, ks=(3, 2, 1, 2)), -1, "index destination"),
        (dict(op=115, fmt=F32, ks=(3, 2, 1, 2)), -3, "no qualified"),
        (dict(op=116, fmt=F16, ks=(3, 2, 1, 2)), -3, "F32 accumulation"),
        (dict(op=117, fmt=F32, ks=(3, 2, 1, 1)), -1, "window geometry"),
        (dict(op=117, fmt=F32, ks=(256, 2, 1, 2)), -1, "kernel_strides"),
        (dict(op=114, fmt=F32, ks=(3, 2, 1, 2)), -1, "registered"),
    ]
    for kw, status, text in cases:
        op, fmt, ks = kw.pop("op"), kw.pop("fmt"), kw.pop("ks")
        dd = d
        if fmt == F16:
            s16 = dev_bits(F16, np.zeros(1 * 5 * 6 * 2, np.uint16)).reshape(1, 5, 6, 2)
            d16 = dev_bits(F16, np.zeros(1 * 2 * 4 * 2, np.uint16)).reshape(1, 2, 4, 2)
            call = lambda: hip.pool(op, fmt, s16, d16, ks, **kw)  # noqa: E731
        else:
            call = lambda: hip.pool(op, fmt, s, dd, ks, **kw)  # noqa: E731
        with pytest.raises(B.WaferHipError) as e:
            call()
        assert e.value.status == status, (op, kw, str(e.value))
        assert text in str(e.value), (text, str(e.value))
    # batch / channel must be preserved
    with pytest.raises(B.WaferHipError) as e:
        hip.pool(117, F32, s, dev_bits(F32, np.zeros(1 * 2 * 4 * 1, np.uint32)).reshape(1, 2, 4, 1), (3, 2, 1, 2))
    assert "batch and channel" in str(e.value)
