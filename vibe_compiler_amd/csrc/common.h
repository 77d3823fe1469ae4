// common.h -- shared helpers for the gfx950 numeric backend: status plumbing,
// scalar codecs (f32 <-> bf16/f16 with the reference's rounding rules), and
// MFMA operand vector types.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "wafer_hip.h"

struct wafer_hip_context {
  int device = 0;
  hipStream_t stream = nullptr;
  // FD chunk states of the small-batch path (grown on demand, freed with
  // the context).
  void *workspace = nullptr;
  size_t workspace_bytes = 0;
  // Error word of the convert kernel.
  int *status = nullptr;
  // Scratch for operand re-layout (transposed rhs), grown on demand.
  void *relayout = nullptr;
  size_t relayout_bytes = 0;
  // Split-K partial tiles of the 16-bit and f32 MFMA GEMMs, grown on demand.
  void *partials = nullptr;
  size_t partials_bytes = 0;
  int cu_count = 0;
  // Buffers a workspace slot outgrew.  They stay allocated until the
  // context is destroyed, so a graph captured while a smaller buffer was
  // current keeps valid memory after a later eager call grows the slot.
  std::vector<void *> retired;
};

namespace wafer {

// Thread-local last error, set by fail() and returned by wafer_hip_last_error.
void set_error(const std::string &message);
int fail(int code, const std::string &message);
int check_hip(hipError_t err, const char *what);
int ensure_workspace(wafer_hip_context *ctx, void **slot, size_t *slot_bytes,
                     size_t need);
int launch_status(const char *kernel);
// Fails with WAFER_HIP_E_UNSUPPORTED when the context's stream is capturing:
// for entries that synchronise the stream, read results back to the host or
// (re)allocate memory, none of which a graph capture can record.
int refuse_capture(wafer_hip_context *ctx, const char *what);
// The context's 256-byte device word area (allocated on first use), after
// refusing a capturing stream.  Layout: bytes [0,4) the convert / MaskMove
// status word, [64,72) a 64-bit first-index word.
int status_words(wafer_hip_context *ctx, const char *what, uint8_t **words);
// Sets n 32-bit words at p to `value` with a one-wave kernel on the context's
// stream (a memset node recorded into a graph has given wrong results on
// later replays, so device words are never cleared with hipMemsetAsync).
int fill_words(wafer_hip_context *ctx, void *p, uint32_t n, uint32_t value);
// Resolves the device address of the no-allocation decode scratch on
// `device` (fd_decode.hip); wafer_hip_context_create calls it.
int noalloc_scratch_lookup(int device);
// FA prefill through the masked-attention kernels (fa_masked.hip): the
// body of wafer_hip_attention_prefill_masked, also taken by
// wafer_hip_attention_prefill for the cases its own kernel does not serve.
int attention_prefill_masked(wafer_hip_context *ctx, uint32_t format, const void *q, const void *k, const void *v,
                             void *o, uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t q_len,
                             uint32_t kv_len, uint32_t head_dim, float scale, const wafer_hip_attention_mask *mask);

#define WAFER_CHECK_CTX(ctx)                                                   \
  do {                                                                         \
    if (!(ctx)) return ::wafer::fail(WAFER_HIP_E_INVALID_FIELD, "null context"); \
  } while (0)

#define WAFER_TRY(expr)                                                        \
  do {                                                                         \
    int _st = (expr);                                                          \
    if (_st != WAFER_HIP_OK) return _st;                                       \
  } while (0)

inline bool is_float_format(uint32_t f) {
  return f == WAFER_FMT_F32 || f == WAFER_FMT_BF16 || f == WAFER_FMT_F16;
}
inline int format_bytes(uint32_t f) {
  switch (f) {
  case WAFER_FMT_I8: case WAFER_FMT_U8: case WAFER_FMT_BOOL: return 1;
  case WAFER_FMT_I16: case WAFER_FMT_F16: case WAFER_FMT_BF16: case WAFER_FMT_U16: return 2;
  case WAFER_FMT_I32: case WAFER_FMT_F32: case WAFER_FMT_TF32: case WAFER_FMT_U32: return 4;
  case WAFER_FMT_I64: case WAFER_FMT_U64: return 8;
  default: return 0;
  }
}

// ---------------------------------------------------------------------------
// Device scalar codecs.  These restate the reference's conversions bit for
// bit: F32 -> BF16 RNE with the canonical quiet NaN 0x7fc0
// (lib/Wafer/Target/PhysicalTensor/TargetScalarConversion.cpp:282-290), F16
// via halfToBits / halfFromBits
// (lib/Wafer/Simulator/Reference/ManagedReferenceTargetModel.cpp:60-135).
// ---------------------------------------------------------------------------
__host__ __device__ inline uint32_t f2u(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
}
__host__ __device__ inline float u2f(uint32_t u) {
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

__host__ __device__ inline uint16_t f32_to_bf16(float v) {
  uint32_t u = f2u(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__host__ __device__ inline float bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }
// Two f32 -> packed bf16 (lo in bits 0..15) by v_cvt_pk_bf16_f32: RNE with
// gradual underflow and overflow to inf, the bits of f32_to_bf16 for every
// non-NaN input (checked over halfway cases, denormals and the overflow
// edge); the instruction keeps a NaN's sign and payload, so NaNs are set to
// the codec's canonical 0x7fc0 afterwards.
__device__ inline uint32_t bf16x2_rne(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  uint32_t r = __builtin_bit_cast(uint32_t, v);
  r = lo != lo ? (r & 0xffff0000u) | 0x7fc0u : r;
  r = hi != hi ? (r & 0x0000ffffu) | 0x7fc00000u : r;
  return r;
}

__host__ __device__ inline float f16_to_f32(uint16_t bits) {
  uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
  uint32_t exponent = (bits >> 10) & 0x1fu;
  uint32_t fraction = bits & 0x03ffu;
  if (exponent == 0) {
    if (fraction == 0) return u2f(sign);
    int32_t e = -14;
    while ((fraction & 0x0400u) == 0) { fraction <<= 1; --e; }
    fraction &= 0x03ffu;
    return u2f(sign | ((uint32_t)(e + 127) << 23) | (fraction << 13));
  }
  if (exponent == 31) return u2f(sign | 0x7f800000u | (fraction << 13));
  return u2f(sign | ((exponent - 15 + 127) << 23) | (fraction << 13));
}

// F32 -> F16, RNE, overflow to +-inf, gradual underflow; NaN -> 0x7e00.
__host__ __device__ inline uint16_t f32_to_f16(float value) {
  uint32_t bits = f2u(value);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  uint32_t eb = (bits >> 23) & 0xffu;
  uint32_t fraction = bits & 0x007fffffu;
  if (eb == 0xffu) return fraction ? (uint16_t)0x7e00u : (uint16_t)(sign | 0x7c00u);
  int32_t exponent = (int32_t)eb - 127;
  if (exponent > 15) return (uint16_t)(sign | 0x7c00u);
  if (exponent >= -14) {
    uint32_t de = (uint32_t)(exponent + 15);
    uint32_t df = fraction >> 13;
    uint32_t rem = fraction & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (df & 1u))) {
      ++df;
      if (df == 0x400u) {
        df = 0;
        ++de;
        if (de >= 0x1fu) return (uint16_t)(sign | 0x7c00u);
      }
    }
    return (uint16_t)(sign | (de << 10) | df);
  }
  if (exponent < -25) return sign;
  uint32_t significand = fraction | 0x00800000u;
  uint32_t shift = (uint32_t)(-exponent - 1);
  uint32_t df = significand >> shift;
  uint32_t rem = significand & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (df & 1u))) ++df;
  return (uint16_t)(sign | df);
}

// An f32 result made opaque to the compiler before it is narrowed to f16: the
// reference rounds each operation to f32 and then narrows, while a multiply
// or add feeding an f16 conversion would otherwise be fused into one
// v_fma_mix{lo,hi}_f16, which rounds the exact result once (a different f16
// in rare double-rounding cases).  No instruction is emitted.
__device__ inline float f32_rounded(float x) {
  asm("" : "+v"(x));
  return x;
}
// f32 -> f16 by v_cvt_f16_f32: RNE with gradual underflow and overflow to
// inf, the bits of f32_to_f16 for every non-NaN input (checked on the GPU
// over tie remainders at every exponent of f16's range, the overflow edge
// and half the smallest subnormal); a NaN is set to the codec's 0x7e00 (the
// instruction keeps sign and payload).  The pin keeps the compiler from
// fusing a preceding multiply into v_fma_mix (one rounding instead of two).
__device__ inline uint32_t f16_rne(float x) {
  x = f32_rounded(x);
  return x != x ? 0x7e00u : (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// ExpLp (ManagedReferenceTargetModel.cpp:265-270): exp2f(x * log2(e))
__device__ inline float explp_acc(float x) { return exp2f(x * 0x1.715476p+0f); }
// SwiGLU element: y = g * Recip(1 + ExpLp(-g)) * u (ComputeLowering.cpp:2555-2606
// has no tile-level Sigmoid; the region is ExpLp, Add, Recip, Mul, Mul).
// Shared by the silu_mul region and the GEMM's fused SwiGLU epilogue, so the
// two give identical bits.
__device__ inline float silu_mul_1(float g, float u) {
  const float sig = 1.0f / (1.0f + explp_acc(-g));
  return g * sig * u;
}
// y = 0.5*x*(1 + Tanh(sqrt(2/pi)*(x + 0.044715*x^3))) (the gelu_tanh
// region), evaluated through the identity 1 + tanh(z) = 2 / (1 + e^(-2z)):
// y = x / (1 + 2^(c*(x + 0.044715*x^3))), c = -2*log2(e)*sqrt(2/pi).  One
// v_exp_f32 and one v_rcp_f32 (each within 1 ulp) replace tanhf, and the
// form has no cancellation where tanh is near -1.  Same value as the tanh
// form up to f32 rounding; the measured bound against a float64 evaluation
// is in the GPU parity tests.  Infinities and NaN map as in the tanh form
// (+inf -> +inf, -inf -> NaN, NaN -> NaN).  Shared by the gelu_tanh region
// and the f32 GEMM's fused epilogue (same bits).
__device__ inline float gelu_tanh_1(float v) {
  const float k1 = 0.044715f, c = -0x1.26aec2p+1f;
  const float inner = v + k1 * (v * v * v);
  const float e = __builtin_amdgcn_exp2f(c * inner);
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}

template <uint32_t F> __device__ inline float load_as_f32(const void *base, int64_t i);
template <> __device__ inline float load_as_f32<WAFER_FMT_F32>(const void *b, int64_t i) {
  return ((const float *)b)[i];
}
template <> __device__ inline float load_as_f32<WAFER_FMT_BF16>(const void *b, int64_t i) {
  return bf16_to_f32(((const uint16_t *)b)[i]);
}
template <> __device__ inline float load_as_f32<WAFER_FMT_F16>(const void *b, int64_t i) {
  return f16_to_f32(((const uint16_t *)b)[i]);
}
template <uint32_t F> __device__ inline void store_from_f32(void *base, int64_t i, float v);
template <> __device__ inline void store_from_f32<WAFER_FMT_F32>(void *b, int64_t i, float v) {
  ((float *)b)[i] = v;
}
template <> __device__ inline void store_from_f32<WAFER_FMT_BF16>(void *b, int64_t i, float v) {
  ((uint16_t *)b)[i] = (uint16_t)bf16x2_rne(v, v);
}
template <> __device__ inline void store_from_f32<WAFER_FMT_F16>(void *b, int64_t i, float v) {
  ((uint16_t *)b)[i] = (uint16_t)f16_rne(v);
}

// ExpLp: one RNE multiply by log2(e) = 0x1.715476p+0, then exp2
// (ManagedReferenceTargetModel.cpp:265-270).  v_exp_f32 is the exp2.
__device__ inline float explp(float x) {
  return __builtin_amdgcn_exp2f(x * 0x1.715476p+0f);
}

// ---------------------------------------------------------------------------
// MFMA operand types.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Eight consecutive elements from element index i (a multiple of 8) with
// 16-byte accesses: one for 16-bit formats, two for F32.  The caller checks
// 16-byte alignment of the base.
// v rounded to the storage format F and widened back (what a store then a
// load of v gives)
template <uint32_t F> __device__ inline float round_to(float v) {
  if constexpr (F == WAFER_FMT_BF16) return u2f(bf16x2_rne(v, v) << 16);
  else if constexpr (F == WAFER_FMT_F16) return f16_to_f32((uint16_t)f16_rne(v));
  else return v;
}
template <uint32_t F> __device__ inline void load8(const void *b, int64_t i, float (&v)[8]) {
  if constexpr (F == WAFER_FMT_F32) {
    const u32x4 lo = ((const u32x4 *)b)[i / 4], hi = ((const u32x4 *)b)[i / 4 + 1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = u2f(lo[e]);
      v[4 + e] = u2f(hi[e]);
    }
  } else {
    const u32x4 w = ((const u32x4 *)b)[i / 8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t l = (uint16_t)(w[e] & 0xffffu), h = (uint16_t)(w[e] >> 16);
      v[2 * e] = F == WAFER_FMT_BF16 ? bf16_to_f32(l) : f16_to_f32(l);
      v[2 * e + 1] = F == WAFER_FMT_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
    }
  }
}
// load8 with non-temporal loads, for streams read exactly once (no L2
// allocation for data nothing reads again)
template <uint32_t F> __device__ inline void load8_nt(const void *b, int64_t i, float (&v)[8]) {
  if constexpr (F == WAFER_FMT_F32) {
    const u32x4 lo = __builtin_nontemporal_load((const u32x4 *)b + i / 4);
    const u32x4 hi = __builtin_nontemporal_load((const u32x4 *)b + i / 4 + 1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = u2f(lo[e]);
      v[4 + e] = u2f(hi[e]);
    }
  } else {
    const u32x4 w = __builtin_nontemporal_load((const u32x4 *)b + i / 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t l = (uint16_t)(w[e] & 0xffffu), h = (uint16_t)(w[e] >> 16);
      v[2 * e] = F == WAFER_FMT_BF16 ? bf16_to_f32(l) : f16_to_f32(l);
      v[2 * e + 1] = F == WAFER_FMT_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
    }
  }
}
template <uint32_t F> __device__ inline void store8(void *b, int64_t i, const float (&v)[8]) {
  if constexpr (F == WAFER_FMT_F32) {
    u32x4 lo, hi;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo[e] = f2u(v[e]);
      hi[e] = f2u(v[4 + e]);
    }
    ((u32x4 *)b)[i / 4] = lo;
    ((u32x4 *)b)[i / 4 + 1] = hi;
  } else {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = F == WAFER_FMT_BF16 ? bf16x2_rne(v[2 * e], v[2 * e + 1]) : f16_rne(v[2 * e]) | (f16_rne(v[2 * e + 1]) << 16);
    ((u32x4 *)b)[i / 8] = w;
  }
}
inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }


}  // namespace wafer
