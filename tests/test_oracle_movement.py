"""The movement and fill oracle (strided copy, Memset, Bit2FP, MaskMove)
pinned against the reference's own known-answer tests
(unittests/Simulator/Kernel/TargetModelKernelTest.cpp, vectors in
tests/golden/reference_goldens.json "movement"), against an independent
numpy restatement of the segment enumeration (index arrays instead of
nested loops), and against numpy's own bit unpacking for the Bool codec.
All comparisons are bit-exact."""
import numpy as np
import pytest

F16, BF16, I32, F32, TF32, BOOL = 2, 3, 4, 5, 6, 7
ONE = {F16: 0x3C00, BF16: 0x3F80, F32: 0x3F800000}


def index_bytes(n):
    return (np.arange(n) & 0xFF).astype(np.uint8)


def starts_numpy(strides, iters):
    """Segment start offsets with iterations[0] innermost, built from
    broadcast index grids (no loop nest)."""
    i2, i1, i0 = np.meshgrid(np.arange(iters[2]), np.arange(iters[1]), np.arange(iters[0]), indexing="ij")
    return (i0 * strides[0] + i1 * strides[1] + i2 * strides[2]).reshape(-1)


def copy_numpy(src, dst, inner, ss, si, ds, di):
    gather = starts_numpy(ss, si)[:, None] + np.arange(inner)[None, :]
    scatter = starts_numpy(ds, di)[:, None] + np.arange(inner)[None, :]
    out = dst.copy()
    out[scatter.reshape(-1)] = src[gather.reshape(-1)]
    return out


def test_rdma_wdma_golden(oracle, goldens):
    g = goldens["movement"]["rdma_wdma"]
    ddr = index_bytes(64)
    st, payload = oracle.strided_copy(ddr, np.zeros(8, np.uint8), g["inner"], g["strides"], g["iterations"],
                                      [g["inner"], 0, 0], [2, 1, 1])
    assert st == 0 and payload.tolist() == g["payload"]
    st, out = oracle.strided_copy(payload, np.zeros(16, np.uint8), g["inner"], [g["inner"], 0, 0], [2, 1, 1],
                                  g["strides"], g["iterations"])
    assert st == 0
    for off, want in g["written"].items():
        assert out[int(off):int(off) + len(want)].tolist() == want
    assert out[4:8].tolist() == [0, 0, 0, 0]


def test_noncanonical_layout_golden(oracle, goldens):
    g = goldens["movement"]["noncanonical_linear"]
    ddr = index_bytes(64)
    n = len(g["payload"])
    st, payload = oracle.strided_copy(ddr, np.zeros(n, np.uint8), g["inner"], g["strides"], g["iterations"],
                                      [g["inner"], 0, 0], [n // g["inner"], 1, 1])
    assert st == 0 and payload.tolist() == g["payload"]
    st, out = oracle.strided_copy(payload, np.zeros(16, np.uint8), g["inner"], [g["inner"], 0, 0],
                                  [n // g["inner"], 1, 1], g["strides"], g["iterations"])
    assert st == 0 and out.tolist() == g["written16"]


def test_gather_goldens(oracle, goldens):
    m = goldens["movement"]
    g = m["gather_overlapping_source"]
    st, out = oracle.strided_copy_inplace(np.array(g["buffer"], np.uint8), g["src_offset"], g["dst_offset"], g["inner"],
                                          g["src_strides"], g["src_iterations"], g["dst_strides"], g["dst_iterations"])
    assert st == 0 and out.tolist() == g["expect"]
    g = m["gather_repeated_source"]
    st, out = oracle.strided_copy(np.array(g["source"], np.uint8), np.zeros(4, np.uint8), g["inner"], g["src_strides"],
                                  g["src_iterations"], g["dst_strides"], g["dst_iterations"])
    assert st == 0 and out.tolist() == g["expect"]
    g = m["gather_overlapping_destination"]
    st, out = oracle.strided_copy(np.array(g["source"], np.uint8), np.zeros(4, np.uint8), g["inner"], g["src_strides"],
                                  g["src_iterations"], g["dst_strides"], g["dst_iterations"])
    assert st == -2 and out.tolist() == g["destination_after"]


def test_large_transpose_golden(oracle, goldens):
    g = goldens["movement"]["large_transpose"]
    cols, rows, inner = g["columns"], g["rows"], g["inner"]
    seg = np.arange(cols * rows)
    payload = np.stack([seg & 0xFF, (seg >> 8) & 0xFF], axis=1).astype(np.uint8).reshape(-1)
    st, t = oracle.strided_copy(payload, np.zeros_like(payload), inner, g["src_strides"], g["iterations"],
                                g["dst_strides"], g["iterations"])
    assert st == 0
    for c, r in [(0, 0), (1, 0), (0, 1), (cols // 2, rows // 2), (cols - 1, rows - 1)]:
        s, d = r * cols + c, (c * rows + r) * inner
        assert t[d:d + 2].tolist() == payload[2 * s:2 * s + 2].tolist()
    # the whole transpose is numpy's transpose of 2-byte elements
    want = payload.view(np.uint16).reshape(rows, cols).T.copy().view(np.uint8).reshape(-1)
    assert np.array_equal(t, want)
    st, back = oracle.strided_copy(t, np.zeros_like(t), inner, g["dst_strides"], g["iterations"], g["src_strides"],
                                   g["iterations"])
    assert st == 0 and np.array_equal(back, payload)


@pytest.mark.parametrize("seed", range(12))
def test_strided_copy_matches_index_formulation(oracle, seed):
    rng = np.random.default_rng(seed)
    inner = int(rng.choice([1, 2, 3, 4, 8, 12, 16, 32]))
    si = [int(x) for x in rng.integers(1, 6, 3)]
    # source: any strides, repeats included
    ss = [int(x) for x in rng.integers(0, 40, 3)]
    # destination: a permuted dense layout (never overlapping)
    di = [int(x) for x in rng.permutation(si)] if seed % 2 else list(si)
    order = rng.permutation(3)
    ds, step = [0, 0, 0], inner + int(rng.integers(0, 3))
    for d in order:
        ds[d] = step
        step *= di[d]
    src = rng.integers(0, 256, 4096, dtype=np.uint8)
    dst = rng.integers(0, 256, step + 64, dtype=np.uint8)
    st, out = oracle.strided_copy(src, dst, inner, ss, si, ds, di)
    assert st == 0
    assert np.array_equal(out, copy_numpy(src, dst, inner, ss, si, ds, di))


def test_strided_copy_rejections(oracle):
    z = np.zeros(64, np.uint8)
    assert oracle.strided_copy(z, z, 2, [2, 0, 0], [0, 1, 1], [2, 0, 0], [0, 1, 1])[0] == -1
    assert oracle.strided_copy(z, z, 2, [2, 0, 0], [3, 1, 1], [2, 0, 0], [2, 1, 1])[0] == -1
    assert oracle.strided_copy(z, z, 0, [2, 0, 0], [2, 1, 1], [2, 0, 0], [2, 1, 1])[0] == -1
    # partially overlapping destination segments (stride below the segment)
    st, out = oracle.strided_copy(index_bytes(64), z, 4, [4, 0, 0], [3, 1, 1], [3, 0, 0], [3, 1, 1])
    assert st == -2 and not out.any()


def test_memset_goldens_and_formats(oracle, goldens):
    g = goldens["movement"]["memset_footprint"]
    f = g["f16"]
    st, out = oracle.memset(np.full(256, int(f["fill"], 16), np.uint8), F16, int(f["value"], 16), f["count"])
    assert st == 0 and out.reshape(-1, 2).tolist() == [f["expect_pair"]] * f["count"]
    b = g["bool"]
    st, out = oracle.memset(np.full(2, int(b["fill"], 16), np.uint8), BOOL, b["value"], b["count"])
    assert st == 0 and out.tolist() == b["expect"]
    v = goldens["movement"]["memset_validation"]
    for n in v["bool_counts_valid"]:
        assert oracle.memset(np.zeros(8, np.uint8), BOOL, 1, n)[0] == 0
    for n in v["bool_counts_invalid"]:
        assert oracle.memset(np.zeros(8, np.uint8), BOOL, 1, n)[0] == -1
    # every format writes its value little-endian (numpy's own encoding)
    for fmt, dt, val in [(0, np.uint8, 0x9C), (1, "<u2", 0xBEEF), (4, "<u4", 0x89ABCDEF), (11, "<u8", 0xFEDCBA98),
                         (12, "<u8", 7), (TF32, "<u4", 0x3F802000)]:
        st, out = oracle.memset(np.full(64, 0xA5, np.uint8), fmt, val, 5)
        n = 5 * np.dtype(dt).itemsize
        assert st == 0
        assert np.array_equal(out[:n].view(dt), np.full(5, val, dt))
        assert (out[n:] == 0xA5).all()


def test_memset_rejections(oracle):
    z = np.zeros(16, np.uint8)
    assert oracle.memset(z, F16, 0x3C00, 0)[0] == -1          # zero count
    assert oracle.memset(z, F16, 0x13C00, 1)[0] == -1         # bits past the width
    assert oracle.memset(z, 0, 0x100, 1)[0] == -1
    assert oracle.memset(z, TF32, 0x3F800001, 1)[0] == -1     # TF32 padding bits
    assert oracle.memset(z, BOOL, 2, 8)[0] == -1
    assert oracle.memset(z, 13, 0, 1)[0] == -1                # unknown format


@pytest.mark.parametrize("fmt", [F16, BF16, F32])
def test_bit2fp_and_maskmove_golden(oracle, goldens, fmt):
    g = goldens["movement"]["bit2fp_maskmove"]
    dt = np.uint32 if fmt == F32 else np.uint16
    for extent in g["extents"]:
        pred = (np.arange(extent) % 3 == 1)
        bits = np.packbits(pred, bitorder="little")
        mask = oracle.bit2fp(bits, fmt, extent)
        assert np.array_equal(mask, np.where(pred, ONE[fmt], 0).astype(dt))
        src = np.full(extent, ONE[fmt], dt)
        st, out = oracle.mask_move(src, mask, np.zeros(extent, dt), fmt)
        assert st == 0 and np.array_equal(out, mask)


def test_bit2fp_matches_unpackbits(oracle):
    rng = np.random.default_rng(3)
    for n in [1, 7, 8, 9, 1000, 4099]:
        bits = rng.integers(0, 256, (n + 7) // 8, dtype=np.uint8)
        want = np.unpackbits(bits, bitorder="little")[:n].astype(bool)
        got = oracle.bit2fp(bits, F32, n)
        assert np.array_equal(got, np.where(want, 0x3F800000, 0).astype(np.uint32))
        # 1.0 really is 1.0 in each format
        assert np.array_equal(oracle.bit2fp(bits, F16, n).view(np.float16).astype(np.float32), want.astype(np.float32))


def test_maskmove_noncanonical_and_selects(oracle):
    rng = np.random.default_rng(5)
    n = 777
    src = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    dst = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    sel = rng.random(n) < 0.5
    mask = np.where(sel, 0x3F800000, 0).astype(np.uint32)
    st, out = oracle.mask_move(src, mask, dst, F32)
    assert st == 0 and np.array_equal(out, np.where(sel, src, dst))
    # -0.0 is neither +0 nor 1.0: the command fails and dst is untouched
    mask[n // 2] = 0x80000000
    st, out = oracle.mask_move(src, mask, dst, F32)
    assert st == -2 and np.array_equal(out, dst)
