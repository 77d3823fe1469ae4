"""numpy front end of the CPU oracle (oracle/wafer_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker (or the timed CPU lane),
never as the product path.  Raw 16-bit floats travel as numpy uint16 arrays
holding their storage bits.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

I8, I16, F16, BF16, I32, F32 = 0, 1, 2, 3, 4, 5
TENSOR, NTENSOR, CX, NCX = 0, 1, 2, 3

_lib = None


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(L: ctypes.CDLL) -> None:
    vp, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
    L.oracle_f32_to_bf16.restype = ctypes.c_uint16
    L.oracle_f32_to_bf16.argtypes = [f32]
    L.oracle_explp.restype = f32
    L.oracle_explp.argtypes = [f32]
    L.oracle_gemm_fma.restype = f32
    L.oracle_gemm_fma.argtypes = [f32, f32, f32]
    L.oracle_f16_to_f32.restype = f32
    L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.oracle_f32_to_f16.restype = i32
    L.oracle_f32_to_f16.argtypes = [f32, ctypes.POINTER(ctypes.c_uint16)]
    L.oracle_format_bits.argtypes = [i32]
    L.oracle_geometry_compute.argtypes = [i32, i32, vp, i32, vp]
    L.oracle_bit_offset.restype = i64
    L.oracle_bit_offset.argtypes = [i32, i32, vp, i32, vp]
    L.oracle_pack.argtypes = [i32, i32, vp, i32, vp, vp, i64]
    L.oracle_unpack.argtypes = [i32, i32, vp, i32, vp, i64, vp]
    L.oracle_gemm_formal.argtypes = [i32, i32, vp, vp, vp, vp, i64, i64, i64, i64, i32, i32, i32]
    L.oracle_gemm_i8.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i32, i32]
    L.oracle_elementwise.argtypes = [i32, i32, vp, vp, vp, i64]
    L.oracle_elementwise_formal.argtypes = [i32, i32, i32, ctypes.c_uint32, ctypes.c_uint32, i32, ctypes.c_uint32,
                                            vp, vp, vp, i64]
    L.oracle_pool.argtypes = [i32, i32, vp, vp, vp, vp, vp]
    u32p = ctypes.POINTER(ctypes.c_uint32)
    L.oracle_strided_copy.argtypes = [vp, vp, ctypes.c_uint32, u32p, u32p, u32p, u32p]
    L.oracle_memset.argtypes = [vp, i32, ctypes.c_uint32, i64]
    L.oracle_bit2fp.argtypes = [vp, vp, i32, i64]
    L.oracle_mask_move.argtypes = [vp, vp, vp, i32, i64]
    d = ctypes.c_double
    L.oracle_compare_floats.argtypes = [i32, vp, vp, i64, d, d, i32, d, d, ctypes.POINTER(d), ctypes.POINTER(d),
                                        ctypes.POINTER(i64)]
    L.oracle_compare_statistics.argtypes = [i32, vp, vp, i64, d, d, ctypes.POINTER(CmpStats), ctypes.POINTER(i64)]
    L.oracle_convert.argtypes = [i32, i32, vp, vp, i64]
    L.oracle_reduce.argtypes = [i32, i32, i32, vp, i32, vp, vp]
    L.oracle_attention_prefill.argtypes = [i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, i32, i32]
    L.oracle_attention_decode.argtypes = [i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, i32, i32]
    L.oracle_attention_prefill_ex.argtypes = [i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, f32,
                                              ctypes.c_uint32, i64, i64, vp, i64, i64, i64, vp, i64, i64, i64,
                                              i32, i32]
    L.oracle_attention_score.argtypes = [i32, ctypes.c_uint32, f32, f32, ctypes.POINTER(ctypes.c_float)]
    L.oracle_attention_score.restype = ctypes.c_float
    L.oracle_rmsnorm.argtypes = [i32, vp, vp, vp, i64, i64, f32]
    L.oracle_softmax.argtypes = [i32, vp, vp, i64, i64]
    L.oracle_silu_mul.argtypes = [i32, vp, vp, vp, i64]
    L.oracle_gelu_tanh.argtypes = [i32, vp, vp, i64]
    L.oracle_rope.argtypes = [i32, vp, vp, i64, i64, i64, vp, f32]
    L.oracle_bias_add.argtypes = [i32, vp, vp, vp, i64, i64]


def _p(a):
    return None if a is None else a.ctypes.data


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with status {rc}")


def threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


# ---- scalar helpers ---------------------------------------------------------
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Vectorised RNE float32 -> bf16 bits (same rule as oracle_f32_to_bf16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """Float32 -> f16 bits through oracle_f32_to_f16 (RNE, overflow to inf,
    gradual underflow), a NaN set to the codec's 0x7e00 as store_float does."""
    src = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(src.size, dtype=np.uint16)
    h = ctypes.c_uint16()
    f = lib().oracle_f32_to_f16
    for i, v in enumerate(src.tolist()):
        out[i] = h.value if f(v, ctypes.byref(h)) == 0 else 0x7E00
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def storage_dtype(fmt: int):
    return {I8: np.int8, I16: np.int16, F16: np.uint16, BF16: np.uint16, I32: np.int32, F32: np.float32,
            6: np.uint32, 8: np.uint8, 9: np.uint16, 10: np.uint32, 11: np.int64, 12: np.uint64}[fmt]


def to_float(fmt: int, a: np.ndarray) -> np.ndarray:
    if fmt == F32:
        return np.asarray(a, dtype=np.float32)
    if fmt == BF16:
        return bf16_to_f32(a)
    if fmt == F16:
        return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float32)
    raise ValueError(fmt)


# ---- codec ------------------------------------------------------------------
def geometry(fmt: int, layout: int, shape) -> dict:
    shp = np.ascontiguousarray(shape, dtype=np.int64)
    g = np.zeros(11, dtype=np.int64)
    _check(lib().oracle_geometry_compute(fmt, layout, _p(shp), len(shp), _p(g)), "geometry")
    keys = ["physical_elements", "physical_bytes", "element_bits", "c_block", "cx_blocks", "c0",
            "aligned_c", "outer_elements", "block_outer_elements", "outer_slice_stride",
            "bank_align_elements"]
    return dict(zip(keys, (int(v) for v in g)))


def bit_offset(fmt: int, layout: int, shape, index) -> int:
    shp = np.ascontiguousarray(shape, dtype=np.int64)
    idx = np.ascontiguousarray(index, dtype=np.int64)
    return int(lib().oracle_bit_offset(fmt, layout, _p(shp), len(shp), _p(idx)))


def pack(fmt: int, layout: int, shape, logical: np.ndarray, template: np.ndarray) -> np.ndarray:
    shp = np.ascontiguousarray(shape, dtype=np.int64)
    out = np.array(template, dtype=np.uint8, copy=True)
    src = np.ascontiguousarray(logical)
    _check(lib().oracle_pack(fmt, layout, _p(shp), len(shp), _p(src), _p(out), out.size), "pack")
    return out


def unpack(fmt: int, layout: int, shape, storage: np.ndarray) -> np.ndarray:
    shp = np.ascontiguousarray(shape, dtype=np.int64)
    st = np.ascontiguousarray(storage, dtype=np.uint8)
    count = int(np.prod(shp)) if len(shp) else 1
    dt = np.uint8 if fmt == 7 else storage_dtype(fmt)
    out = np.zeros(count, dtype=dt)
    _check(lib().oracle_unpack(fmt, layout, _p(shp), len(shp), _p(st), st.size, _p(out)), "unpack")
    return out.reshape(tuple(shape))


# ---- GEMMs ------------------------------------------------------------------
def gemm_formal(in_fmt, out_fmt, lhs, rhs, m, k, n, batch=1, psum=None, lhs_t=False, rhs_t=False, nthreads=None):
    dst = np.zeros(batch * m * n, dtype=storage_dtype(out_fmt))
    lhs = np.ascontiguousarray(lhs)
    rhs = np.ascontiguousarray(rhs)
    ps = None if psum is None else np.ascontiguousarray(psum, dtype=np.float32)
    _check(lib().oracle_gemm_formal(in_fmt, out_fmt, _p(lhs), _p(rhs), _p(ps), _p(dst), m, k, n, batch,
                                    int(lhs_t), int(rhs_t), nthreads or threads()), "gemm")
    return dst


def gemm_i8(a, b, scale, m, k, n, rhs_t=False, nthreads=None, want_acc=True):
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    acc = np.zeros((m, n), dtype=np.int32) if want_acc else None
    y = np.zeros((m, n), dtype=np.uint16)
    _check(lib().oracle_gemm_i8(_p(a), _p(b), _p(scale), _p(acc), _p(y), m, k, n, int(rhs_t),
                                nthreads or threads()), "gemm_i8")
    return acc, y


# ---- managed lane -----------------------------------------------------------
def elementwise(op: int, fmt: int, a, b=None):
    a = np.ascontiguousarray(a)
    b = None if b is None else np.ascontiguousarray(b)
    out = np.zeros(a.size, dtype=storage_dtype(fmt))
    _check(lib().oracle_elementwise(op, fmt, _p(a), _p(b), _p(out), a.size), "elementwise")
    return out.reshape(a.shape)


BOOL = 7
RELATIONS = range(12, 18)


def formal_storage(fmt: int):
    """Storage dtype of a formal-lane logical tensor (raw bits; Bool one byte)."""
    return {F16: np.uint16, BF16: np.uint16, F32: np.uint32, BOOL: np.uint8}[fmt]


def elementwise_formal(op: int, fmt: int, lhs, rhs=None, *, scalar=None, unit=0, group=0, numeric=False):
    """Formal-lane elementwise command on raw bits; returns the result bits
    (Bool results as uint8 0 / 1, numeric results in the input storage)."""
    lhs = np.ascontiguousarray(lhs, dtype=formal_storage(fmt))
    count = lhs.size
    rhs_a = None if rhs is None else np.ascontiguousarray(rhs, dtype=formal_storage(fmt))
    bool_out = fmt == BOOL or (op in RELATIONS and not numeric)
    dst = np.zeros(count, dtype=np.uint8 if bool_out else formal_storage(fmt))
    rc = lib().oracle_elementwise_formal(op, fmt, int(bool(numeric)), unit, group, scalar is not None,
                                         0 if scalar is None else int(scalar), _p(lhs), _p(rhs_a), _p(dst), count)
    _check(rc, "elementwise_formal")
    return dst


def pool(op: int, fmt: int, src, dst_hw, kernel_strides):
    """Plain NHWC pooling on raw bits.  src is [N, H, W, C]; dst_hw = (H', W');
    kernel_strides = (kernel W, kernel H, stride W, stride H)."""
    src = np.ascontiguousarray(src, dtype=formal_storage(fmt))
    n, h, w, c = src.shape
    sshape = np.array([n, h, w, c], dtype=np.uint32)
    dshape = np.array([n, dst_hw[0], dst_hw[1], c], dtype=np.uint32)
    ks = np.ascontiguousarray(kernel_strides, dtype=np.uint32)
    dst = np.zeros((n, dst_hw[0], dst_hw[1], c), dtype=formal_storage(fmt))
    _check(lib().oracle_pool(op, fmt, _p(sshape), _p(dshape), _p(ks), _p(src), _p(dst)), "pool")
    return dst


def convert(opcode: int, src, dst_fmt: int):
    src = np.ascontiguousarray(src)
    out = np.zeros(src.size, dtype=storage_dtype(dst_fmt))
    _check(lib().oracle_convert(opcode, 0, _p(src), _p(out), src.size), "convert")
    return out.reshape(src.shape)


def reduce(op: int, dim: int, fmt: int, shape, src):
    shp = np.ascontiguousarray(shape, dtype=np.int64)
    rank = len(shp)
    mask = np.zeros(rank, dtype=bool)
    if dim <= 3:
        mask[rank - 1 - dim] = True
    elif dim == 4:
        mask[rank - 3] = mask[rank - 2] = True
    else:
        mask[rank - 3:] = True
    out_shape = [1 if mask[i] else int(shp[i]) for i in range(rank)]
    src = np.ascontiguousarray(src)
    out = np.zeros(int(np.prod(out_shape)), dtype=storage_dtype(fmt))
    _check(lib().oracle_reduce(op, dim, fmt, _p(shp), rank, _p(src), _p(out)), "reduce")
    return out.reshape(out_shape)


# ---- attention ----------------------------------------------------------------
def attention_prefill(q, k, v, scale, causal=True, block_k=64, fmt=BF16, nthreads=None):
    B, Hq, Sq, D = q.shape
    _, Hkv, Skv, _ = k.shape
    q, k, v = (np.ascontiguousarray(t, dtype=np.uint16) for t in (q, k, v))
    o = np.zeros((B, Hq, Sq, D), dtype=np.uint16)
    _check(lib().oracle_attention_prefill(fmt, _p(q), _p(k), _p(v), _p(o), B, Hq, Hkv, Sq, Skv, D,
                                          float(scale), int(causal), block_k, nthreads or threads()),
           "attention_prefill")
    return o


ATT_CAUSAL, ATT_WINDOW, ATT_ROUND_SCALED, ATT_ROUND_BIASED = 1, 2, 4, 8


def _mask_operand(m, dtype, B, Hq, Sq, kv_len):
    """A [b, h, q, kv] mask broadcast over size-1 leading dims -> (array, strides)."""
    if m is None:
        return None, (0, 0, 0)
    m = np.ascontiguousarray(m, dtype=dtype)
    if m.ndim != 4 or m.shape[0] not in (1, B) or m.shape[1] not in (1, Hq) or m.shape[2] not in (1, Sq) \
            or m.shape[3] < kv_len:
        raise ValueError(f"mask shape {m.shape} does not broadcast to [{B}, {Hq}, {Sq}, >={kv_len}]")
    st = [m.strides[i] // m.itemsize if m.shape[i] > 1 else 0 for i in range(3)]
    return m, tuple(st)


def attention_prefill_ex(q, k, v, scale, *, kv_len=None, causal=False, diagonal=0, window=0, bias=None,
                         keep=None, round_scaled=False, round_biased=False, block_k=64, fmt=BF16, nthreads=None):
    """FA prefill with masks: k/v [B, Hkv, capacity, D] of which kv_len tokens are valid; causal: key j
    visible to query i iff j <= i + diagonal; window > 0: and j > i + diagonal - window; bias: additive
    f32 [b|1, h|1, q|1, >=kv_len]; keep: boolean mask of the same form (nonzero = visible)."""
    B, Hq, Sq, D = q.shape
    _, Hkv, cap, _ = k.shape
    kv_len = cap if kv_len is None else kv_len
    q, k, v = (np.ascontiguousarray(t, dtype=np.uint16) for t in (q, k, v))
    bias, bst = _mask_operand(bias, np.float32, B, Hq, Sq, kv_len)
    keep, kst = _mask_operand(keep, np.uint8, B, Hq, Sq, kv_len)
    flags = (ATT_CAUSAL if causal else 0) | (ATT_WINDOW if window > 0 else 0) | \
        (ATT_ROUND_SCALED if round_scaled else 0) | (ATT_ROUND_BIASED if round_biased else 0)
    o = np.zeros((B, Hq, Sq, D), dtype=np.uint16)
    _check(lib().oracle_attention_prefill_ex(fmt, _p(q), _p(k), _p(v), _p(o), B, Hq, Hkv, Sq, kv_len, cap, D,
                                             float(scale), flags, int(diagonal), int(window),
                                             _p(bias) if bias is not None else None, *bst,
                                             _p(keep) if keep is not None else None, *kst,
                                             block_k, nthreads or threads()),
           "attention_prefill_ex")
    return o


def attention_score(raw, scale, bias=None, round_scaled=False, round_biased=False, fmt=F16):
    """The score region element by element (oracle_attention_score), as float32."""
    raw = np.asarray(raw, dtype=np.float32).ravel()
    flags = (ATT_ROUND_SCALED if round_scaled else 0) | (ATT_ROUND_BIASED if round_biased else 0)
    out = np.empty_like(raw)
    b = None if bias is None else np.asarray(bias, dtype=np.float32).ravel()
    cell = ctypes.c_float()
    for i in range(raw.size):
        if b is not None:
            cell.value = float(b[i])
        out[i] = lib().oracle_attention_score(fmt, flags, float(raw[i]), float(scale),
                                              ctypes.byref(cell) if b is not None else None)
    return out


def attention_decode(q, k, v, scale, chunks=16, kv_len=None, block_k=64, fmt=BF16, nthreads=None):
    B, Hq, _, D = q.shape
    _, Hkv, cap, _ = k.shape
    kv_len = cap if kv_len is None else kv_len
    q, k, v = (np.ascontiguousarray(t, dtype=np.uint16) for t in (q, k, v))
    o = np.zeros((B, Hq, 1, D), dtype=np.uint16)
    _check(lib().oracle_attention_decode(fmt, _p(q), _p(k), _p(v), _p(o), B, Hq, Hkv, kv_len, cap, D,
                                         float(scale), chunks, block_k, nthreads or threads()),
           "attention_decode")
    return o


# ---- fused regions ----------------------------------------------------------
def rmsnorm(x, w, eps, fmt=BF16):
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w)
    rows, cols = int(np.prod(x.shape[:-1])), x.shape[-1]
    y = np.zeros_like(x)
    _check(lib().oracle_rmsnorm(fmt, _p(x), _p(w), _p(y), rows, cols, float(eps)), "rmsnorm")
    return y


def softmax(x, fmt=BF16):
    x = np.ascontiguousarray(x)
    rows, cols = int(np.prod(x.shape[:-1])), x.shape[-1]
    y = np.zeros_like(x)
    _check(lib().oracle_softmax(fmt, _p(x), _p(y), rows, cols), "softmax")
    return y


def silu_mul(g, u, fmt=BF16):
    g = np.ascontiguousarray(g)
    u = np.ascontiguousarray(u)
    y = np.zeros_like(g)
    _check(lib().oracle_silu_mul(fmt, _p(g), _p(u), _p(y), g.size), "silu_mul")
    return y


def gelu_tanh(x, fmt=BF16):
    x = np.ascontiguousarray(x)
    y = np.zeros_like(x)
    _check(lib().oracle_gelu_tanh(fmt, _p(x), _p(y), x.size), "gelu_tanh")
    return y


def rope(x, positions, theta, fmt=BF16):
    """x: [tokens, heads, D] storage array."""
    x = np.ascontiguousarray(x)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    T, H, D = x.shape
    y = np.zeros_like(x)
    _check(lib().oracle_rope(fmt, _p(x), _p(y), T, H, D, _p(pos), float(theta)), "rope")
    return y


def bias_add(x, bias, fmt=F32):
    x = np.ascontiguousarray(x)
    b = np.ascontiguousarray(bias, dtype=np.float32)
    rows, cols = int(np.prod(x.shape[:-1])), x.shape[-1]
    y = np.zeros_like(x)
    _check(lib().oracle_bias_add(fmt, _p(x), _p(b), _p(y), rows, cols), "bias_add")
    return y


# ---- movement and fill commands ---------------------------------------------
def _u32x3(v):
    return (ctypes.c_uint32 * 3)(*[int(x) for x in v])


def strided_copy(src, dst, inner_bytes, src_strides, src_iterations, dst_strides, dst_iterations):
    """Gather `src` (uint8) through the source layout into the payload and
    write it through the destination layout into a copy of `dst`.  Returns
    (status, result): 0 ok, -1 rejected command, -2 overlapping destination
    segments (result then equals dst)."""
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.array(dst, dtype=np.uint8, copy=True)
    st = lib().oracle_strided_copy(_p(src), _p(out), inner_bytes, _u32x3(src_strides), _u32x3(src_iterations),
                                   _u32x3(dst_strides), _u32x3(dst_iterations))
    return st, out


def strided_copy_inplace(buf, src_offset, dst_offset, inner_bytes, src_strides, src_iterations, dst_strides,
                         dst_iterations):
    """The same command with source and destination in one buffer (the
    payload is read completely before any byte is written)."""
    out = np.array(buf, dtype=np.uint8, copy=True)
    view = out[src_offset:]
    tmp = np.array(view, copy=True)
    st = lib().oracle_strided_copy(_p(tmp), _p(out[dst_offset:]), inner_bytes, _u32x3(src_strides),
                                   _u32x3(src_iterations), _u32x3(dst_strides), _u32x3(dst_iterations))
    return st, out


def memset(dst, fmt, value, count):
    """Returns (status, result): 0 ok, -1 rejected command (result == dst)."""
    out = np.array(dst, dtype=np.uint8, copy=True)
    st = lib().oracle_memset(_p(out), fmt, value, count)
    return st, out


def bit2fp(bits, fmt, count):
    bits = np.ascontiguousarray(bits, dtype=np.uint8)
    out = np.zeros(count, dtype=np.uint32 if fmt == F32 else np.uint16)
    _check(lib().oracle_bit2fp(_p(bits), _p(out), fmt, count), "bit2fp")
    return out


def mask_move(src, mask, dst, fmt):
    """Returns (status, result): status 0 ok, -2 for a noncanonical mask
    (result then equals dst)."""
    src, mask = np.ascontiguousarray(src), np.ascontiguousarray(mask)
    out = np.array(dst, copy=True)
    st = lib().oracle_mask_move(_p(src), _p(mask), _p(out), fmt, out.size)
    return st, out


# ---- program-boundary comparison ---------------------------------------------
# ProgramElementType (include/Wafer/Frontend/ProgramElementType.h:17-32)
DT = dict(bool=0, i8=1, u8=2, i16=3, u16=4, i32=5, u32=6, i64=7, u64=8, f16=9, bf16=10, f32=11, tf32=12, f64=13)
DT_NAME = {v: k for k, v in DT.items()}
DT_BYTES = {0: 1, 1: 1, 2: 1, 3: 2, 4: 2, 5: 4, 6: 4, 7: 8, 8: 8, 9: 2, 10: 2, 11: 4, 12: 4, 13: 8}
# ProgramTensorComparisonErrorCode + 1 (0: accepted)
CMP = dict(accepted=0, invalid_tolerance=1, dtype_mismatch=2, shape_mismatch=3, byte_size_mismatch=4,
           unsupported_floating_dtype=5, unsupported_statistics_dtype=6, actual_nonfinite=7,
           expected_nonfinite=8, numeric_mismatch=9, raw_mismatch=10)


class CmpStats(ctypes.Structure):
    _fields_ = [("element_count", ctypes.c_uint64), ("exact_element_count", ctypes.c_uint64),
                ("exact_fraction", ctypes.c_double), ("mean_absolute_error", ctypes.c_double),
                ("p99_absolute_error", ctypes.c_double), ("p999_absolute_error", ctypes.c_double),
                ("maximum_absolute_error", ctypes.c_double), ("elementwise_mismatch_count", ctypes.c_uint64),
                ("cosine_similarity", ctypes.c_double), ("relative_l2_error", ctypes.c_double),
                ("mean_ulp_distance", ctypes.c_double), ("p99_ulp_distance", ctypes.c_uint64),
                ("p999_ulp_distance", ctypes.c_uint64), ("maximum_ulp_distance", ctypes.c_uint64)]


def _policy_ok(atol, rtol, similarity):
    """validateProgramTensorComparisonPolicy (ProgramTensorComparison.cpp:499-516)."""
    import math
    if not (math.isfinite(atol) and math.isfinite(rtol)) or atol < 0 or rtol < 0:
        return False
    if similarity is not None:
        c, r = similarity
        if not math.isfinite(c) or c < 0 or c > 1 or not math.isfinite(r) or r < 0:
            return False
    return True


def _metadata(actual, expected):
    """(dtype, shape, bytes) checks in the reference's order; tensors are
    (dtype, shape, uint8 array)."""
    if actual[0] != expected[0]:
        return CMP["dtype_mismatch"]
    if tuple(actual[1]) != tuple(expected[1]):
        return CMP["shape_mismatch"]
    if actual[2].size != expected[2].size:
        return CMP["byte_size_mismatch"]
    return None


def compare_expected(actual, expected, atol, rtol, similarity=None):
    """compareProgramTensorExpectedOutput (ProgramTensorComparison.cpp:267-387).
    Returns (verdict, info): info is the raw first differing byte for a raw
    mismatch, else the oracle's [scan end, mismatches, first, max_abs, max_ratio]
    element indices plus cosine and relative L2."""
    if not _policy_ok(atol, rtol, similarity):
        return CMP["invalid_tolerance"], None
    m = _metadata(actual, expected)
    if m is not None:
        return m, None
    dt = actual[0]
    if dt in (DT["tf32"], DT["f64"]):
        return CMP["unsupported_floating_dtype"], None
    a = np.ascontiguousarray(actual[2], dtype=np.uint8)
    e = np.ascontiguousarray(expected[2], dtype=np.uint8)
    if dt not in (DT["f16"], DT["bf16"], DT["f32"]):
        diff = np.nonzero(a != e)[0]
        return (CMP["raw_mismatch"], int(diff[0])) if diff.size else (CMP["accepted"], None)
    n = a.size // DT_BYTES[dt]
    info = (ctypes.c_int64 * 5)()
    c, r = ctypes.c_double(), ctypes.c_double()
    sim = similarity or (0.0, 0.0)
    v = lib().oracle_compare_floats(dt, _p(a), _p(e), n, atol, rtol, int(similarity is not None), sim[0], sim[1],
                                    ctypes.byref(c), ctypes.byref(r), info)
    return v, dict(scan_end=info[0], mismatches=info[1], first=info[2], max_abs=info[3], max_ratio=info[4],
                   cosine=c.value, relative_l2=r.value)


def compare_statistics(actual, expected, atol=0.0, rtol=0.0):
    """computeProgramTensorComparisonStatistics (ProgramTensorComparison.cpp:389-497).
    Returns (verdict, stats dict or None)."""
    if not _policy_ok(atol, rtol, None):
        return CMP["invalid_tolerance"], None
    m = _metadata(actual, expected)
    if m is not None:
        return m, None
    dt = actual[0]
    if dt not in (DT["f16"], DT["bf16"], DT["f32"]):
        return CMP["unsupported_statistics_dtype"], None
    a = np.ascontiguousarray(actual[2], dtype=np.uint8)
    e = np.ascontiguousarray(expected[2], dtype=np.uint8)
    out = CmpStats()
    bad = ctypes.c_int64()
    v = lib().oracle_compare_statistics(dt, _p(a), _p(e), a.size // DT_BYTES[dt], atol, rtol, ctypes.byref(out),
                                        ctypes.byref(bad))
    if v != 0:
        return v, None
    return 0, {k: getattr(out, k) for k, _ in CmpStats._fields_}
