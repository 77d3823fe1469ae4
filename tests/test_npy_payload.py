"""The .npy payload loader (C++, libwafer_hip_seam.so) against the
reference's own loader tests (unittests/Frontend/NpyPayloadTest.cpp, vectors
in tests/golden/reference_goldens.json "npy") and against numpy's writer:
every accepted dtype in format versions 1 and 2 round-trips byte for byte,
and each rejection of NpyPayload.cpp is hit with its message.  Host code
only: runs without a GPU."""
import struct
import sys

import numpy as np
import pytest

DT = dict(bool=0, i8=1, u8=2, i16=3, u16=4, i32=5, u32=6, i64=7, u64=8, f16=9, bf16=10, f32=11, tf32=12, f64=13)


@pytest.fixture(scope="module")
def io():
    from vibe_compiler_amd import program_io
    program_io._lib()
    return program_io


def write_v1(path, descr, payload, shape="(2,)", fortran="False", major=1):
    """The reference test's writer (header padded to 64 bytes, newline)."""
    header = "{'descr': '%s', 'fortran_order': %s, 'shape': %s, }" % (descr, fortran, shape)
    prefix = 10 if major == 1 else 12
    pad = (64 - ((prefix + len(header) + 1) % 64)) % 64
    header = header + " " * pad + "\n"
    head = b"\x93NUMPY" + bytes([major, 0])
    head += struct.pack("<H", len(header)) if major == 1 else struct.pack("<I", len(header))
    path.write_bytes(head + header.encode() + bytes(payload))


def test_reference_goldens(io, goldens, tmp_path):
    g = goldens["npy"]
    for key in ("f16_little", "bf16_opaque"):
        c = g[key]
        p = tmp_path / (key + ".npy")
        write_v1(p, c["descr"], c["bytes"])
        dt, shape, data = io.load_npy(p)
        assert dt == DT[c["dtype"]] and list(shape) == c["shape"] and data.tolist() == c["bytes"]
    c = g["f16_big_endian"]
    p = tmp_path / "be.npy"
    write_v1(p, c["descr"], c["bytes"])
    with pytest.raises(io.NpyError, match=c["error"]):
        io.load_npy(p)
    c = g["f16_native"]
    p = tmp_path / "native.npy"
    write_v1(p, c["descr"], c["bytes"])
    assert sys.byteorder == "little"
    dt, shape, data = io.load_npy(p)
    assert dt == DT[c["dtype"]] and data.tolist() == c["bytes"]


@pytest.mark.parametrize("np_dtype,code", [("<f4", "f32"), ("<f8", "f64"), ("<f2", "f16"), ("|b1", "bool"),
                                           ("|i1", "i8"), ("<i2", "i16"), ("<i4", "i32"), ("<i8", "i64"),
                                           ("|V2", "bf16")])
@pytest.mark.parametrize("version", [(1, 0), (2, 0)])
@pytest.mark.parametrize("shape", [(), (0,), (3,), (2, 5), (4, 1, 3), (2, 0, 3)])
def test_numpy_writer_round_trip(io, tmp_path, np_dtype, code, version, shape):
    rng = np.random.default_rng(len(shape) * 7 + version[0])
    n = int(np.prod(shape))
    raw = rng.integers(0, 256, n * np.dtype(np_dtype).itemsize, dtype=np.uint8)
    if np_dtype == "|b1":
        raw = (raw & 1).astype(np.uint8)
    arr = raw.view(np.dtype(np_dtype)).reshape(shape)
    p = tmp_path / "a.npy"
    with open(p, "wb") as f:
        np.lib.format.write_array(f, arr, version=version)
    dt, got_shape, data = io.load_npy(p)
    assert dt == DT[code] and got_shape == shape
    assert np.array_equal(data, np.ascontiguousarray(arr).view(np.uint8).reshape(-1))


def test_rejections(io, tmp_path):
    p = tmp_path / "x.npy"
    # Fortran order
    with open(p, "wb") as f:
        np.lib.format.write_array(f, np.asfortranarray(np.ones((2, 3), np.float32)))
    with pytest.raises(io.NpyError, match="must be row-major"):
        io.load_npy(p)
    # unsupported dtypes (unsigned integers and complex are not in the table)
    for d in ("<u2", "<c8", ">f4", "|u1"):
        write_v1(p, d, [0] * 16, shape="(2,)")
        with pytest.raises(io.NpyError, match="unsupported dtype"):
            io.load_npy(p)
    # truncated payload
    write_v1(p, "<f4", [0] * 7)
    with pytest.raises(io.NpyError, match="truncated"):
        io.load_npy(p)
    # missing magic, unsupported version, malformed headers
    p.write_bytes(b"NUMPY\x01\x00" + b"\x00" * 20)
    with pytest.raises(io.NpyError, match="missing magic"):
        io.load_npy(p)
    write_v1(p, "<f4", [0] * 8)
    raw = bytearray(p.read_bytes())
    raw[6] = 3
    p.write_bytes(bytes(raw))
    with pytest.raises(io.NpyError, match="unsupported npy payload version"):
        io.load_npy(p)
    for shape in ("(2, -1)", "(2,", "[2]", "(2x,)"):
        write_v1(p, "<f4", [0] * 8, shape=shape)
        with pytest.raises(io.NpyError, match="invalid npy payload header"):
            io.load_npy(p)
    write_v1(p, "<f4", [0] * 8, fortran="Maybe")
    with pytest.raises(io.NpyError, match="invalid npy payload header"):
        io.load_npy(p)
    with pytest.raises(io.NpyError, match="failed to read"):
        io.load_npy(tmp_path / "missing.npy")
    # a header length past the end of the file
    p.write_bytes(b"\x93NUMPY\x01\x00" + struct.pack("<H", 4000) + b"{}")
    with pytest.raises(io.NpyError, match="truncated npy payload header"):
        io.load_npy(p)


def test_trailing_bytes_and_double_quotes(io, tmp_path):
    # bytes past the payload are ignored; double-quoted keys are accepted
    p = tmp_path / "q.npy"
    header = '{"descr": "<i4", "fortran_order": false, "shape": (3,), }'
    header = header + " " * ((64 - (10 + len(header) + 1) % 64) % 64) + "\n"
    payload = np.arange(3, dtype="<i4").tobytes()
    p.write_bytes(b"\x93NUMPY\x01\x00" + struct.pack("<H", len(header)) + header.encode() + payload + b"junk")
    dt, shape, data = io.load_npy(p)
    assert dt == DT["i32"] and shape == (3,) and data.tobytes() == payload
