// gemm_mfma.hip -- matrix-core GEMMs for gfx950: bf16/f16 (f32 accumulate)
// and int8 (exact int32 accumulate, fused dequant to bf16).
//
// Both run one kernel template on the "NT" operand form, A [M, K] and
// Bt [N, K], both K-contiguous, so every lane's MFMA operand is one 16-byte
// LDS read:
//   bf16/f16: v_mfma_f32_32x32x16_{bf16,f16}  (16 elements = 32 B of K/step)
//   int8:     v_mfma_i32_32x32x32_i8          (32 elements = 32 B of K/step)
// A workgroup of 4 waves computes a BMxBN tile (256x256 or 128x128; waves
// 2x2), staging 64-byte K slices of A and Bt through double-buffered LDS.
// LDS rows are 64 B with the 16-byte chunk index XOR-swizzled by
// ((row >> 1) & 3) so the 8 lanes that share a bank window read 8 different
// chunks (conflict-free ds_read_b128).  A normal (K-major) rhs is first
// re-laid out to Bt by a tiled transpose kernel into context scratch.
// Workgroup ids are mapped so that the 32 tiles served by one XCD form a
// 4x8 block of the output, bounding that XCD's L2 working set.
//
// int8 semantics (no reference implementation exists; the closed form on the
// reference's conversion routes): acc = sum_k int32(a)*int32(b) exactly
// (|acc| <= k*127*128 < 2^31 for k <= 131071), y = bf16_RNE(f32_RNE(
// f32_RNE(acc) * scale[n])) -- int32_fp32 route, CT Mul, fp32_bf16 route
// (lib/Wafer/Target/TargetFormat.cpp:174,192).  Integer sums are
// order-independent, so the result is bit-exact.
#include "common.h"

namespace wafer {
namespace {

enum { KIND_BF16 = 0, KIND_F16 = 1, KIND_I8 = 2 };
constexpr int BKB = 64;  // bytes of K per LDS stage (2 MFMA steps)

__device__ inline int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 3); }

template <int KIND> struct Acc;
template <> struct Acc<KIND_BF16> { typedef f32x16 T; };
template <> struct Acc<KIND_F16> { typedef f32x16 T; };
template <> struct Acc<KIND_I8> { typedef i32x16 T; };

template <int KIND>
__device__ inline typename Acc<KIND>::T mfma(u32x4 a, u32x4 b, typename Acc<KIND>::T c);
template <>
__device__ inline f32x16 mfma<KIND_BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ inline f32x16 mfma<KIND_F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <>
__device__ inline i32x16 mfma<KIND_I8>(u32x4 a, u32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a),
                                               __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// Epilogue selectors.
enum { OUT_F32 = 0, OUT_NARROW = 1, OUT_I8_DEQUANT = 2 };

struct GemmArgs {
  const uint8_t *a;    // [M, K] elements, K-contiguous
  const uint8_t *bt;   // [N, K]
  void *y;             // [M, N]
  int32_t *acc_out;    // int8 only, optional [M, N]
  const float *scale;  // int8 only, [N]
  int m, n, kbytes;    // K in bytes
  int tiles_n;         // N / BN
};

template <int KIND, int BM, int BN, int OUT>
__global__ __launch_bounds__(256) void gemm_nt_kernel(GemmArgs args) {
  constexpr int WTM = BM / 64, WTN = BN / 64;  // 32x32 MFMA tiles per wave (waves 2x2)
  constexpr int A_LOADS = BM * 4 / 256, B_LOADS = BN * 4 / 256;
  __shared__ __align__(16) u32x4 sA[2][BM * 4];
  __shared__ __align__(16) u32x4 sB[2][BN * 4];

  // XCD-aware tile order: ids are dealt round-robin over 8 XCDs; the ids one
  // XCD receives cover a 4 x 8 block of output tiles when the grid allows it.
  const int tiles_m = args.m / BM, tiles_n = args.tiles_n;
  int tm, tn;
  {
    const int bid = blockIdx.x;
    const int total = tiles_m * tiles_n;
    if (total % 256 == 0 && tiles_m % 4 == 0 && tiles_n % 8 == 0) {
      const int group = bid / 256, inner = bid % 256;  // 256 tiles per round
      const int xcd = inner % 8, j = inner / 8;        // 32 tiles per XCD
      const int gm = tiles_m / 4, gn = tiles_n / 8;    // 4x8 blocks in the grid
      const int blocks_per_round = 8;
      const int blk = group * blocks_per_round + xcd;  // which 4x8 block
      const int bm = blk / gn, bn = blk % gn;
      tm = bm * 4 + j / 8;
      tn = bn * 8 + j % 8;
      (void)gm;
    } else {
      tm = bid / tiles_n;
      tn = bid % tiles_n;
    }
  }
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, g = lane >> 5;

  typename Acc<KIND>::T acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int ld_row = tid >> 2, ld_chunk = tid & 3;  // rows ld_row + 64 i
  u32x4 ra[A_LOADS], rb[B_LOADS];
  const size_t kb = (size_t)args.kbytes;
  auto gload = [&](int kt) {
    const size_t koff = (size_t)kt * BKB + ld_chunk * 16;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      ra[i] = *(const u32x4 *)(args.a + (size_t)(m0 + ld_row + 64 * i) * kb + koff);
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i)
      rb[i] = *(const u32x4 *)(args.bt + (size_t)(n0 + ld_row + 64 * i) * kb + koff);
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int row = ld_row + 64 * i;
      sA[buf][row * 4 + swz(row, ld_chunk)] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int row = ld_row + 64 * i;
      sB[buf][row * 4 + swz(row, ld_chunk)] = rb[i];
    }
  };

  const int nkt = args.kbytes / BKB;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nkt) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int chunk = ks * 2 + g;
      u32x4 fa[WTM], fb[WTN];
#pragma unroll
      for (int i = 0; i < WTM; ++i) {
        const int row = wm * (BM / 2) + i * 32 + l32;
        fa[i] = sA[buf][row * 4 + swz(row, chunk)];
      }
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const int row = wn * (BN / 2) + j * 32 + l32;
        fb[j] = sB[buf][row * 4 + swz(row, chunk)];
      }
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j) acc[i][j] = mfma<KIND>(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < nkt) {
      sstore(buf ^ 1);
      __syncthreads();
    }
  }

  // epilogue: lane holds column l32 and rows 8*(r/4) + 4*g + r%4 of each tile
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
      const int col = n0 + wn * (BN / 2) + j * 32 + l32;
      float sc = 0.0f;
      if (OUT == OUT_I8_DEQUANT) sc = args.scale[col];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        const size_t o = (size_t)row * args.n + col;
        if (OUT == OUT_F32) {
          ((float *)args.y)[o] = (float)acc[i][j][r];
        } else if (OUT == OUT_NARROW) {
          const float v = (float)acc[i][j][r];
          ((uint16_t *)args.y)[o] = KIND == KIND_F16 ? f32_to_f16(v) : f32_to_bf16(v);
        } else {
          const int32_t a32 = (int32_t)acc[i][j][r];
          if (args.acc_out) args.acc_out[o] = a32;
          ((uint16_t *)args.y)[o] = f32_to_bf16((float)a32 * sc);
        }
      }
      // keep the scheduler from hoisting every tile's conversion at once
      __builtin_amdgcn_sched_barrier(0);
    }
}

// [rows, cols] -> [cols, rows] for 1- or 2-byte elements, 64x64 tiles.
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T *__restrict__ src, T *__restrict__ dst,
                                                        int rows, int cols) {
  __shared__ T tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    if (r < rows && c < cols) tile[i][tx] = src[(size_t)r * cols + c];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i, r = r0 + tx;
    if (r < rows && c < cols) dst[(size_t)c * rows + r] = tile[tx][i];
  }
}

template <int KIND, int OUT>
int launch_gemm(hipStream_t st, GemmArgs args, int ctas_256) {
  if (args.m % 256 == 0 && args.n % 256 == 0 && ctas_256 >= 192) {
    args.tiles_n = args.n / 256;
    dim3 grid((args.m / 256) * args.tiles_n);
    hipLaunchKernelGGL((gemm_nt_kernel<KIND, 256, 256, OUT>), grid, dim3(256), 0, st, args);
  } else {
    args.tiles_n = args.n / 128;
    dim3 grid((args.m / 128) * args.tiles_n);
    hipLaunchKernelGGL((gemm_nt_kernel<KIND, 128, 128, OUT>), grid, dim3(256), 0, st, args);
  }
  return launch_status("gemm_nt_kernel");
}

int relayout_rhs(wafer_hip_context *ctx, const void *rhs, uint32_t k, uint32_t n, int esize,
                 const uint8_t **bt) {
  const size_t need = (size_t)k * n * esize;
  WAFER_TRY(ensure_workspace(ctx, &ctx->relayout, &ctx->relayout_bytes, need));
  dim3 grid((n + 63) / 64, (k + 63) / 64);
  if (esize == 1)
    hipLaunchKernelGGL(transpose_kernel<uint8_t>, grid, dim3(256), 0, ctx->stream,
                       (const uint8_t *)rhs, (uint8_t *)ctx->relayout, (int)k, (int)n);
  else
    hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, dim3(256), 0, ctx->stream,
                       (const uint16_t *)rhs, (uint16_t *)ctx->relayout, (int)k, (int)n);
  WAFER_TRY(launch_status("transpose_kernel"));
  *bt = (const uint8_t *)ctx->relayout;
  return WAFER_HIP_OK;
}

int check_shape(uint32_t m, uint32_t k, uint32_t n, int esize, const char *what) {
  if (m == 0 || k == 0 || n == 0) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(what) + ": empty dimension");
  if (m % 128 || n % 128 || ((uint64_t)k * esize) % BKB)
    return fail(WAFER_HIP_E_UNSUPPORTED,
                std::string(what) + ": needs m, n multiples of 128 and k*elem_bytes a multiple of 64");
  if ((uint64_t)m * k * esize > 0x7fffffffffull || (uint64_t)k * esize > 0x7fffffffull)
    return fail(WAFER_HIP_E_INVALID_FIELD, std::string(what) + ": operand too large");
  return WAFER_HIP_OK;
}

}  // namespace
}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_gemm_mfma(wafer_hip_context *ctx, const void *lhs, const void *rhs,
                                   void *dst, uint32_t m, uint32_t k, uint32_t n,
                                   uint32_t in_format, uint32_t out_format,
                                   uint32_t rhs_orientation) {
  WAFER_CHECK_CTX(ctx);
  if (in_format != WAFER_FMT_BF16 && in_format != WAFER_FMT_F16)
    return fail(WAFER_HIP_E_UNSUPPORTED, "gemm_mfma: input format must be BF16 or F16");
  if (out_format != WAFER_FMT_F32 && out_format != in_format)
    return fail(WAFER_HIP_E_UNSUPPORTED, "gemm_mfma: output format must be F32 or the input format");
  if (rhs_orientation > 1) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_mfma: bad orientation");
  if (!lhs || !rhs || !dst) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_mfma: null tensor");
  WAFER_TRY(check_shape(m, k, n, 2, "gemm_mfma"));
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const uint8_t *bt = (const uint8_t *)rhs;
  if (rhs_orientation == WAFER_GEMM_NORMAL) WAFER_TRY(relayout_rhs(ctx, rhs, k, n, 2, &bt));
  GemmArgs args{(const uint8_t *)lhs, bt, dst, nullptr, nullptr, (int)m, (int)n, (int)(k * 2), 0};
  const int ctas = (int)((m / 256) * (n / 256));
  const bool f32 = out_format == WAFER_FMT_F32;
  if (in_format == WAFER_FMT_BF16)
    return f32 ? launch_gemm<KIND_BF16, OUT_F32>(ctx->stream, args, ctas)
               : launch_gemm<KIND_BF16, OUT_NARROW>(ctx->stream, args, ctas);
  return f32 ? launch_gemm<KIND_F16, OUT_F32>(ctx->stream, args, ctas)
             : launch_gemm<KIND_F16, OUT_NARROW>(ctx->stream, args, ctas);
}

extern "C" int wafer_hip_gemm_i8(wafer_hip_context *ctx, const int8_t *a, const int8_t *b,
                                 const float *scale, int32_t *acc_out, uint16_t *y, uint32_t m,
                                 uint32_t k, uint32_t n, uint32_t rhs_orientation) {
  WAFER_CHECK_CTX(ctx);
  if (!a || !b || !scale || !y) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_i8: null tensor");
  if (rhs_orientation > 1) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_i8: bad orientation");
  if (k > 131071) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_i8: k above 131071 can overflow int32");
  WAFER_TRY(check_shape(m, k, n, 1, "gemm_i8"));
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const uint8_t *bt = (const uint8_t *)b;
  if (rhs_orientation == WAFER_GEMM_NORMAL) WAFER_TRY(relayout_rhs(ctx, b, k, n, 1, &bt));
  GemmArgs args{(const uint8_t *)a, bt, y, acc_out, scale, (int)m, (int)n, (int)k, 0};
  return launch_gemm<KIND_I8, OUT_I8_DEQUANT>(ctx->stream, args, (int)((m / 256) * (n / 256)));
}
