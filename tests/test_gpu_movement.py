"""GPU parity of the movement and fill commands (strided copy / gather-
scatter, Memset, Bit2FP, MaskMove) against the CPU oracle, bit-exact, on
the reference's known-answer cases, seeded random layouts for every piece
size the kernel picks (16/8/4/2/1 bytes), the snapshot case (source and
destination overlapping in one buffer), the rejections, and at large sizes
through round trips and torch's own transpose."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

F16, BF16, F32, TF32, BOOL = 2, 3, 5, 6, 7
ONE = {F16: 0x3C00, BF16: 0x3F80, F32: 0x3F800000}


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


def test_movement_goldens(hip, oracle, goldens):
    m = goldens["movement"]
    say("movement goldens")
    g = m["rdma_wdma"]
    ddr = dev((np.arange(64) & 0xFF).astype(np.uint8))
    spm = torch.zeros(8, dtype=torch.uint8, device="cuda")
    hip.strided_copy(ddr, spm, g["inner"], g["strides"], g["iterations"], [g["inner"], 0, 0], [2, 1, 1])
    assert host(spm).tolist() == g["payload"]
    out = torch.zeros(16, dtype=torch.uint8, device="cuda")
    hip.strided_copy(spm, out, g["inner"], [g["inner"], 0, 0], [2, 1, 1], g["strides"], g["iterations"])
    o = host(out)
    assert o[0:4].tolist() == g["written"]["0"] and o[8:12].tolist() == g["written"]["8"] and not o[4:8].any()

    g = m["noncanonical_linear"]
    n = len(g["payload"])
    spm = torch.zeros(n, dtype=torch.uint8, device="cuda")
    hip.strided_copy(ddr, spm, g["inner"], g["strides"], g["iterations"], [g["inner"], 0, 0], [n // g["inner"], 1, 1])
    assert host(spm).tolist() == g["payload"]
    out = torch.zeros(16, dtype=torch.uint8, device="cuda")
    hip.strided_copy(spm, out, g["inner"], [g["inner"], 0, 0], [n // g["inner"], 1, 1], g["strides"], g["iterations"])
    assert host(out).tolist() == g["written16"]

    g = m["gather_overlapping_source"]
    buf = dev(np.array(g["buffer"], np.uint8))
    hip.strided_copy(buf, buf, g["inner"], g["src_strides"], g["src_iterations"], g["dst_strides"], g["dst_iterations"],
                     src_offset=g["src_offset"], dst_offset=g["dst_offset"])
    assert host(buf).tolist() == g["expect"]

    g = m["gather_repeated_source"]
    out = torch.zeros(4, dtype=torch.uint8, device="cuda")
    hip.strided_copy(dev(np.array(g["source"], np.uint8)), out, g["inner"], g["src_strides"], g["src_iterations"],
                     g["dst_strides"], g["dst_iterations"])
    assert host(out).tolist() == g["expect"]


def test_overlapping_destination_rejected_without_writes(hip, B, goldens):
    g = goldens["movement"]["gather_overlapping_destination"]
    say("overlapping destination")
    out = torch.zeros(4, dtype=torch.uint8, device="cuda")
    with pytest.raises(B.WaferHipError, match="overlap"):
        hip.strided_copy(dev(np.array(g["source"], np.uint8)), out, g["inner"], g["src_strides"], g["src_iterations"],
                         g["dst_strides"], g["dst_iterations"])
    assert host(out).tolist() == g["destination_after"]
    # partial overlap that only the exact interval check finds
    big = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    with pytest.raises(B.WaferHipError, match="overlap"):
        hip.strided_copy(big, big, 4, [4, 64, 0], [16, 4, 1], [4, 62, 0], [16, 4, 1], dst_offset=1024)
    assert not host(big).any()
    with pytest.raises(B.WaferHipError, match="must be positive"):
        hip.strided_copy(big, big, 4, [4, 0, 0], [0, 1, 1], [4, 0, 0], [0, 1, 1])


def test_large_transpose_golden(hip, goldens):
    g = goldens["movement"]["large_transpose"]
    cols, rows, inner = g["columns"], g["rows"], g["inner"]
    say("large transpose", cols, rows)
    seg = np.arange(cols * rows)
    payload = np.stack([seg & 0xFF, (seg >> 8) & 0xFF], axis=1).astype(np.uint8).reshape(-1)
    src = dev(payload)
    t = torch.zeros_like(src)
    hip.strided_copy(src, t, inner, g["src_strides"], g["iterations"], g["dst_strides"], g["iterations"])
    want = payload.view(np.uint16).reshape(rows, cols).T.copy().view(np.uint8).reshape(-1)
    assert np.array_equal(host(t), want)
    back = torch.zeros_like(src)
    hip.strided_copy(t, back, inner, g["dst_strides"], g["iterations"], g["src_strides"], g["iterations"])
    assert np.array_equal(host(back), payload)


def random_case(rng, inner, align):
    si = [int(x) for x in rng.integers(1, 9, 3)]
    # source strides: multiples of the piece size, repeats allowed
    ss = [int(x) * align for x in rng.integers(0, 24, 3)]
    di = [int(x) for x in rng.permutation(si)]
    order = rng.permutation(3)
    ds, step = [0, 0, 0], inner + align * int(rng.integers(0, 3))
    for d in order:
        ds[d] = step
        step *= di[d]
    src_bytes = inner + sum((i - 1) * s for s, i in zip(ss, si))
    return si, ss, di, ds, src_bytes, step


@pytest.mark.parametrize("inner,align", [(16, 16), (48, 16), (8, 8), (24, 8), (4, 4), (12, 4), (2, 2), (6, 2),
                                         (1, 1), (3, 1), (5, 1)])
def test_strided_copy_random_layouts(hip, oracle, inner, align):
    rng = np.random.default_rng(inner * 31 + align)
    for rep in range(4):
        si, ss, di, ds, src_bytes, dst_bytes = random_case(rng, inner, align)
        say("strided_copy", inner, ss, si, ds, di)
        src = rng.integers(0, 256, src_bytes + 64, dtype=np.uint8)
        dst = rng.integers(0, 256, dst_bytes + 64, dtype=np.uint8)
        st, want = oracle.strided_copy(src, dst, inner, ss, si, ds, di)
        assert st == 0
        d = dev(dst)
        hip.strided_copy(dev(src), d, inner, ss, si, ds, di)
        assert np.array_equal(host(d), want)


@pytest.mark.parametrize("inner", [1, 2, 4, 8, 16])
def test_strided_copy_tiled_transpose(hip, oracle, inner):
    # two-axis transposes of whole segments (the LDS-tiled kernel), ragged
    # edges, a batch axis, padded pitches, both orientations
    rng = np.random.default_rng(100 + inner)
    for rep in range(3):
        n0, n1, n2 = int(rng.integers(16, 150)), int(rng.integers(16, 150)), int(rng.integers(1, 4))
        p1, p2 = inner * int(rng.integers(0, 3)), inner * int(rng.integers(0, 3))
        ss = [inner, inner * n0 + p1, 0]
        ss[2] = ss[1] * n1 + p1
        ds = [inner * n1 + p2, inner, 0]
        ds[2] = ds[0] * n0 + p2
        it = [n0, n1, n2]
        if rep == 2:  # source contiguous along axis 1, destination along axis 0
            ss, ds = ds, ss
        say("tiled transpose", inner, ss, ds, it)
        src_bytes = inner + sum((i - 1) * s for s, i in zip(ss, it))
        dst_bytes = inner + sum((i - 1) * s for s, i in zip(ds, it))
        src = rng.integers(0, 256, src_bytes, dtype=np.uint8)
        dst = rng.integers(0, 256, dst_bytes, dtype=np.uint8)
        st, want = oracle.strided_copy(src, dst, inner, ss, it, ds, it)
        assert st == 0
        d = dev(dst)
        hip.strided_copy(dev(src), d, inner, ss, it, ds, it)
        assert np.array_equal(host(d), want)


@pytest.mark.parametrize("n0,n1,n2,pad,flip", [(64, 64, 1, 0, 0), (128, 192, 3, 16, 0), (192, 64, 2, 32, 1),
                                               (64, 512, 2, 16, 0), (256, 128, 1, 48, 1), (64, 128, 2, 2, 0)])
def test_strided_copy_transpose_b16_tiles(hip, oracle, n0, n1, n2, pad, flip):
    # 2-byte transposes on whole 64x64 tiles: 16-byte aligned pitches take
    # the vector kernel (padded rows, a batch axis, both orientations); a
    # 2-byte pad breaks the alignment and takes the element kernel
    rng = np.random.default_rng(n0 * 3 + n1 + n2 + pad)
    ss = [2, 2 * n0 + pad, 0]
    ss[2] = ss[1] * n1 + pad
    ds = [2 * n1 + pad, 2, 0]
    ds[2] = ds[0] * n0 + pad
    it = [n0, n1, n2]
    if flip:
        ss, ds = ds, ss
    say("b16 tile transpose", ss, ds, it)
    src_bytes = 2 + sum((i - 1) * s for s, i in zip(ss, it))
    dst_bytes = 2 + sum((i - 1) * s for s, i in zip(ds, it))
    src = rng.integers(0, 256, src_bytes, dtype=np.uint8)
    dst = rng.integers(0, 256, dst_bytes, dtype=np.uint8)
    st, want = oracle.strided_copy(src, dst, 2, ss, it, ds, it)
    assert st == 0
    d = dev(dst)
    hip.strided_copy(dev(src), d, 2, ss, it, ds, it)
    assert np.array_equal(host(d), want)


def test_strided_copy_snapshot_in_one_buffer(hip, oracle):
    rng = np.random.default_rng(11)
    for inner, so, do in [(16, 0, 32), (16, 64, 0), (4, 0, 4), (2, 6, 0), (3, 0, 5)]:
        say("snapshot", inner, so, do)
        buf = rng.integers(0, 256, 8192, dtype=np.uint8)
        ss, si = [inner * 2, inner * 16, 0], [8, 6, 1]
        ds, di = [inner, inner * 8, 0], [8, 6, 1]
        st, want = oracle.strided_copy_inplace(buf, so, do, inner, ss, si, ds, di)
        assert st == 0
        d = dev(buf)
        hip.strided_copy(d, d, inner, ss, si, ds, di, src_offset=so, dst_offset=do)
        assert np.array_equal(host(d), want)


def test_strided_copy_transpose_large(hip):
    # 4096 x 8192 bf16 transpose (64 MiB) and back, against torch's transpose
    rows, cols = 4096, 8192
    say("transpose", rows, cols)
    x = torch.randint(-32768, 32767, (rows, cols), dtype=torch.int16, device="cuda")
    t = torch.empty(cols, rows, dtype=torch.int16, device="cuda")
    hip.strided_copy(x, t, 2, [2, 2 * cols, 0], [cols, rows, 1], [2 * rows, 2, 0], [cols, rows, 1])
    torch.cuda.synchronize()
    assert torch.equal(t, x.t().contiguous())
    # 16-byte pieces: 8 bf16 columns per segment
    t8 = torch.empty(cols // 8, rows, 8, dtype=torch.int16, device="cuda")
    hip.strided_copy(x, t8, 16, [16, 2 * cols, 0], [cols // 8, rows, 1], [16 * rows, 16, 0], [cols // 8, rows, 1])
    torch.cuda.synchronize()
    assert torch.equal(t8, x.view(rows, cols // 8, 8).permute(1, 0, 2).contiguous())


def test_strided_copy_64bit_index_path(hip):
    # 2^31 + 2^16 one-byte segments: the 64-bit index kernel, checked as a
    # transpose of a [2^15 + 1, 2^16] byte matrix
    r, c = (1 << 15) + 1, 1 << 16
    say("64-bit path", r, c)
    x = torch.randint(0, 256, (r, c), dtype=torch.uint8, device="cuda")
    t = torch.empty(c, r, dtype=torch.uint8, device="cuda")
    hip.strided_copy(x, t, 1, [1, c, 0], [c, r, 1], [r, 1, 0], [c, r, 1])
    torch.cuda.synchronize()
    assert torch.equal(t, x.t().contiguous())
    del x, t
    torch.cuda.empty_cache()


@pytest.mark.parametrize("fmt,value,nbytes", [(0, 0x9C, 1), (1, 0xBEEF, 2), (F16, 0x3555, 2), (BF16, 0x3F80, 2),
                                              (4, 0x89ABCDEF, 4), (F32, 0xBF800000, 4), (TF32, 0x3F802000, 4),
                                              (11, 0xFEDCBA98, 8), (12, 7, 8), (8, 0xFF, 1)])
@pytest.mark.parametrize("count", [1, 5, 1000, 100003])
def test_memset_formats(hip, oracle, fmt, value, nbytes, count):
    say("memset", fmt, count)
    init = np.full(count * nbytes + 64, 0xA5, np.uint8)
    st, want = oracle.memset(init, fmt, value, count)
    assert st == 0
    d = dev(init)
    hip.memset(d, fmt, value, count)
    assert np.array_equal(host(d), want)


def test_memset_bool_and_rejections(hip, oracle, B, goldens):
    g = goldens["movement"]["memset_footprint"]["bool"]
    say("memset bool")
    d = dev(np.full(2, 0xA5, np.uint8))
    hip.memset(d, BOOL, g["value"], g["count"])
    assert host(d).tolist() == g["expect"]
    for value in (0, 1):
        init = np.full(4096, 0x5A, np.uint8)
        st, want = oracle.memset(init, BOOL, value, 8 * 4000)
        d = dev(init)
        hip.memset(d, BOOL, value, 8 * 4000)
        assert st == 0 and np.array_equal(host(d), want)
    d = dev(np.full(64, 0xA5, np.uint8))
    for fmt, value, count, what in [(BOOL, 1, 9, "multiple of 8"), (F16, 0x3C00, 0, "positive"),
                                    (F16, 0x13C00, 4, "storage width"), (TF32, 0x3F800001, 4, "padding"),
                                    (13, 0, 4, "unsupported")]:
        with pytest.raises(B.WaferHipError, match=what):
            hip.memset(d, fmt, value, count)
    assert (host(d) == 0xA5).all()


@pytest.mark.parametrize("fmt", [F16, BF16, F32])
def test_bit2fp_and_maskmove(hip, oracle, goldens, fmt):
    g = goldens["movement"]["bit2fp_maskmove"]
    dt_np = np.uint32 if fmt == F32 else np.uint16
    dt_t = torch.int32 if fmt == F32 else torch.int16
    rng = np.random.default_rng(fmt)
    for extent in g["extents"] + [1, 77, 1 << 20]:
        say("bit2fp/maskmove", fmt, extent)
        pred = (np.arange(extent) % 3 == 1) if extent in g["extents"] else rng.random(extent) < 0.4
        bits = np.packbits(pred, bitorder="little")
        want_mask = oracle.bit2fp(bits, fmt, extent)
        mask = torch.empty(extent, dtype=dt_t, device="cuda")
        hip.bit2fp(dev(bits), mask, fmt, extent)
        assert np.array_equal(host(mask).view(dt_np), want_mask)
        src = rng.integers(0, 1 << 16, extent, dtype=np.uint32).astype(dt_np)
        dst = rng.integers(0, 1 << 16, extent, dtype=np.uint32).astype(dt_np)
        if extent in g["extents"]:
            src[:] = ONE[fmt]
            dst[:] = 0
        st, want = oracle.mask_move(src, want_mask, dst, fmt)
        assert st == 0
        d = dev(dst.view(np.int32 if fmt == F32 else np.int16))
        hip.mask_move(dev(src.view(np.int32 if fmt == F32 else np.int16)), mask, d, fmt)
        assert np.array_equal(host(d).view(dt_np), want)


def test_maskmove_noncanonical_leaves_destination(hip, oracle, B):
    say("maskmove noncanonical")
    n = 4099
    rng = np.random.default_rng(9)
    src = rng.integers(0, 1 << 16, n, dtype=np.uint16)
    dst = rng.integers(0, 1 << 16, n, dtype=np.uint16)
    mask = np.where(rng.random(n) < 0.5, ONE[BF16], 0).astype(np.uint16)
    mask[n - 3] = 0x8000  # -0.0
    st, want = oracle.mask_move(src, mask, dst, BF16)
    assert st == -2 and np.array_equal(want, dst)
    d = dev(dst.view(np.int16))
    with pytest.raises(B.WaferHipError, match="canonical"):
        hip.mask_move(dev(src.view(np.int16)), dev(mask.view(np.int16)), d, BF16)
    assert np.array_equal(host(d).view(np.uint16), dst)
    with pytest.raises(B.WaferHipError, match="F16, BF16 or F32"):
        hip.mask_move(dev(src.view(np.int16)), dev(mask.view(np.int16)), d, 1)
    with pytest.raises(B.WaferHipError, match="F16, BF16 or F32"):
        hip.bit2fp(dev(np.zeros(8, np.uint8)), d, 4, 16)
