"""Program-boundary I/O: .npy payloads in, device tensors out, results gated
on the GPU.

`load_npy` calls the C++ loader in libwafer_hip_seam.so (`wafer_npy_load`,
the restatement of loadNpyTensorPayload, lib/Wafer/Frontend/NpyPayload.cpp:368-413)
and returns (ProgramElementType code, shape, bytes).  `to_device` places
the bytes in HBM; `compare_npy` gates an actual payload against an expected
one with the GPU comparator (wafer_hip_compare_expected /
wafer_hip_compare_statistics), as the reference's source/model gate does
(ProgramTensorComparison.cpp:267-497)."""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

from . import backend as B

SEAM_PATH = pathlib.Path(__file__).resolve().parent / "lib" / "libwafer_hip_seam.so"
MAX_RANK = 32
_seam = None


def _lib() -> ctypes.CDLL:
    global _seam
    if _seam is None:
        if not SEAM_PATH.exists():
            raise RuntimeError(f"{SEAM_PATH} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(str(SEAM_PATH))
        L.wafer_npy_load.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int64),
                                     ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32),
                                     ctypes.POINTER(ctypes.POINTER(ctypes.c_uint8)), ctypes.POINTER(ctypes.c_uint64),
                                     ctypes.c_char_p, ctypes.c_size_t]
        L.wafer_npy_free.argtypes = [ctypes.POINTER(ctypes.c_uint8)]
        _seam = L
    return _seam


class NpyError(ValueError):
    pass


def load_npy(path) -> tuple[int, tuple, np.ndarray]:
    """(dtype code, shape, uint8 bytes) of a .npy payload; raises NpyError
    with the reference's message on a rejected file."""
    L = _lib()
    dtype, rank, nbytes = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
    shape = (ctypes.c_int64 * MAX_RANK)()
    data = ctypes.POINTER(ctypes.c_uint8)()
    err = ctypes.create_string_buffer(1024)
    if L.wafer_npy_load(str(path).encode(), ctypes.byref(dtype), shape, MAX_RANK, ctypes.byref(rank),
                        ctypes.byref(data), ctypes.byref(nbytes), err, 1024) != 0:
        raise NpyError(err.value.decode())
    try:
        out = np.ctypeslib.as_array(data, shape=(nbytes.value,)).copy() if nbytes.value else np.zeros(0, np.uint8)
    finally:
        L.wafer_npy_free(data)
    return dtype.value, tuple(shape[i] for i in range(rank.value)), out


def to_device(torch, payload):
    """(dtype, shape, bytes) -> (dtype, device uint8 tensor, shape), the form
    the comparator entries take."""
    dtype, shape, data = payload
    return dtype, torch.from_numpy(np.ascontiguousarray(data)).to("cuda"), shape


def compare_npy(ctx: B.Context, torch, actual_path, expected_path, atol, rtol, similarity=None, statistics=False):
    """Gate (or, with statistics=True, measure) an actual payload against an
    expected one on the GPU.  Returns what Context.compare_expected /
    compare_statistics return."""
    a = to_device(torch, load_npy(actual_path))
    e = to_device(torch, load_npy(expected_path))
    if statistics:
        return ctx.compare_statistics(a, e, atol, rtol)
    return ctx.compare_expected(a, e, atol, rtol, similarity)
