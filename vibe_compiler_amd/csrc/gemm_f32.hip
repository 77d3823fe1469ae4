// gemm_f32.hip -- f32 GEMM on v_mfma_f32_32x32x2_f32 with the bias and
// tanh-GELU regions fused into its epilogue: the tolerance-class f32 lane
// (the counterpart of the reference's deterministic strict-f32 oneDNN matmul,
// lib/Wafer/Simulator/OneDNN/OneDNNGemmAdapter.cpp:278-420) for small-M
// blocks such as an MLP's two projections.
//
// Work split.  One workgroup of 4 waves (one per SIMD) computes a 32x32
// output tile over one k-range; its waves take consecutive quarters of that
// range and fold their partial tiles through LDS in wave order.  When the
// output has too few tiles to fill the CUs the k extent is also split over
// workgroups: each writes its folded partial tile to a [ksplit][m][n] area
// and a second launch adds the splits in split order and applies the
// epilogue.  Every sum has a fixed order, so results repeat bit for bit.
//
// Operands go global -> VGPR directly in the MFMA operand layout (no LDS).
// For a T x T tile (T = 32: v_mfma_f32_32x32x2_f32, T = 16:
// v_mfma_f32_16x16x4_f32) lane l supplies A[l%T][slot l/T] and
// B[slot l/T][l%T].  A group of 4 MFMAs covers 4 * 64/T k: lane slot h takes
// k0 + 4h .. k0 + 4h + 3 with one 16-byte A load, MFMA j component j, so both
// operands use the same k in each slot and the sum is the GEMM's.  16x16
// tiles serve outputs with too few 32x32 tiles to fill the CUs without a
// second (split-k fold) launch.
#include "common.h"

namespace wafer {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int EPI_NONE = WAFER_HIP_EPILOGUE_NONE;
constexpr int EPI_BIAS = WAFER_HIP_EPILOGUE_BIAS;
constexpr int EPI_GELU = WAFER_HIP_EPILOGUE_BIAS_GELU_TANH;

// Groups of 4 MFMAs in flight per wave (loads issued this many groups ahead).
constexpr int DEPTH = 8;

struct F32GemmArgs {
  const float *a;     // [m, k]
  const float *b;     // [k, n] (Normal) or [n, k] (Transpose)
  const float *bias;  // [n] for the bias epilogues
  float *y;           // [m, n]
  float *part;        // [ksplit, m, n] when ksplit > 1
  int m, k, n;
  int kchunk;         // k per split, a multiple of 4 * (k per group)
  int ksplit, tiles_m, tiles_n;
};

template <int EPI> __device__ inline float epilogue(float v, const float *bias, int col) {
  if constexpr (EPI == EPI_NONE) {
    return v;
  } else {
    const float t = v + bias[col];  // the bias_add region
    return EPI == EPI_GELU ? gelu_tanh_1(t) : t;
  }
}

template <int T> struct Mfma;
template <> struct Mfma<32> {
  typedef float acc_t __attribute__((ext_vector_type(16)));
  __device__ static acc_t step(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  // row within the tile of accumulator register r in lane slot h
  __device__ static int row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }
};
template <> struct Mfma<16> {
  typedef float acc_t __attribute__((ext_vector_type(4)));
  __device__ static acc_t step(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  __device__ static int row(int r, int h) { return 4 * h + r; }
};

template <int T, bool RHS_T, int EPI>
__global__ __launch_bounds__(256) void gemm_f32_kernel(F32GemmArgs args) {
  constexpr int NACC = T * T / 64;  // accumulator registers per lane
  constexpr int KG = 4 * (64 / T);  // k per group of 4 MFMAs
  __shared__ float red[4][NACC][64];  // [wave][acc register][lane]
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // XCD-aware order: workgroup ids go round-robin over the 8 XCDs, so
  // consecutive logical tiles are given to one XCD (tm fastest, then tn,
  // then the split): each XCD reads a few B column panels and one k-range.
  const int groups = gridDim.x;
  const int id = blockIdx.x;
  const int logical = (groups % 8 == 0) ? (id % 8) * (groups / 8) + id / 8 : id;
  const int tm = logical % args.tiles_m;
  const int tn = (logical / args.tiles_m) % args.tiles_n;
  const int split = logical / (args.tiles_m * args.tiles_n);
  const int m0 = tm * T, n0 = tn * T;
  const int quarter = args.kchunk / 4;
  const int kb = split * args.kchunk + wave * quarter;
  const int ke = min(kb + quarter, args.k);
  const int ngroups = ke > kb ? (ke - kb) / KG : 0;  // k is a multiple of KG

  // rows and columns past the matrix read the last real one and are never
  // stored
  const int row = min(m0 + lane % T, args.m - 1);
  const int col = min(n0 + lane % T, args.n - 1);
  const int slot = lane / T;
  const float *ap = args.a + (size_t)row * args.k + kb + 4 * slot;
  const float *bp = RHS_T ? args.b + (size_t)col * args.k + kb + 4 * slot
                          : args.b + (size_t)(kb + 4 * slot) * args.n + col;

  typedef f32x4 vec4;
  auto load = [&](int g, vec4 &va, vec4 &vb) __attribute__((always_inline)) {
    va = *(const vec4 *)(ap + KG * g);
    if constexpr (RHS_T) {
      vb = *(const vec4 *)(bp + KG * g);
    } else {
      const float *q = bp + (size_t)(KG * g) * args.n;
      vb = vec4{q[0], q[(size_t)args.n], q[2 * (size_t)args.n], q[3 * (size_t)args.n]};
    }
  };

  // Register queue of DEPTH groups.  Every load inside the main loop is
  // unconditional (the group index clamped to the last one, which only the
  // final main iteration can reach), so the compiler's vmcnt waits count
  // exactly the loads issued behind each group; the tail issues none.
  typename Mfma<T>::acc_t acc = {};
  vec4 qa[DEPTH], qb[DEPTH];
  if (ngroups > 0) {
    const int last = ngroups - 1;
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load(min(d, last), qa[d], qb[d]);
    int g0 = 0;
    for (; g0 + DEPTH < ngroups; g0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = Mfma<T>::step(qa[d][j], qb[d][j], acc);
        load(min(g0 + DEPTH + d, last), qa[d], qb[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (g0 + d < ngroups) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = Mfma<T>::step(qa[d][j], qb[d][j], acc);
      }
  }

  // fold the 4 waves' partial tiles in wave order; thread t then owns
  // NACC / 4 consecutive columns of tile row t / (T / (NACC / 4))
#pragma unroll
  for (int r = 0; r < NACC; ++r) red[wave][r][lane] = acc[r];
  __syncthreads();
  constexpr int CPT = NACC / 4;          // columns per thread: 4 (T 32) or 1 (T 16)
  constexpr int TPR = T / CPT;           // threads per tile row
  const int i = threadIdx.x / TPR, c0 = (threadIdx.x % TPR) * CPT;
  const int h = T == 32 ? (i >> 2) & 1 : i >> 2;
  const int r = T == 32 ? ((i >> 3) << 2) | (i & 3) : i & 3;
  float v[CPT];
#pragma unroll
  for (int e = 0; e < CPT; ++e) {
    const int l = c0 + e + T * h;
    v[e] = ((red[0][r][l] + red[1][r][l]) + red[2][r][l]) + red[3][r][l];
  }
  const int orow = m0 + i;
  if (orow >= args.m) return;
  float *dst = args.ksplit > 1 ? args.part + (size_t)split * args.m * args.n : args.y;
  if (args.ksplit == 1) {
#pragma unroll
    for (int e = 0; e < CPT; ++e) v[e] = epilogue<EPI>(v[e], args.bias, min(n0 + c0 + e, args.n - 1));
  }
  float *o = dst + (size_t)orow * args.n + n0 + c0;
  if (CPT == 4 && (args.n & 3) == 0 && n0 + c0 + 3 < args.n) {
    *(vec4 *)o = vec4{v[0], v[CPT > 1 ? 1 : 0], v[CPT > 2 ? 2 : 0], v[CPT > 3 ? 3 : 0]};
  } else {
#pragma unroll
    for (int e = 0; e < CPT; ++e)
      if (n0 + c0 + e < args.n) o[e] = v[e];
  }
}

// y[e] = epilogue(part[0][e] + part[1][e] + ... ) in split order.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_f32_fold_kernel(const float *__restrict__ part,
                                                            const float *__restrict__ bias,
                                                            float *__restrict__ y, int64_t count,
                                                            int n, int ksplit) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < count; e += stride) {
    float v = part[e];
    for (int s = 1; s < ksplit; ++s) v = v + part[(size_t)s * count + e];
    y[e] = epilogue<EPI>(v, bias, (int)(e % n));
  }
}

template <int T, bool RHS_T, int EPI> int launch_f32(wafer_hip_context *ctx, const F32GemmArgs &a) {
  const int groups = a.tiles_m * a.tiles_n * a.ksplit;
  hipLaunchKernelGGL((gemm_f32_kernel<T, RHS_T, EPI>), dim3(groups), dim3(256), 0, ctx->stream, a);
  WAFER_TRY(launch_status("gemm_f32_kernel"));
  if (a.ksplit > 1) {
    const int64_t count = (int64_t)a.m * a.n;
    const unsigned grid = (unsigned)std::min<int64_t>((count + 255) / 256, 4096);
    hipLaunchKernelGGL((gemm_f32_fold_kernel<EPI>), dim3(grid), dim3(256), 0, ctx->stream, a.part, a.bias, a.y,
                       count, a.n, a.ksplit);
    WAFER_TRY(launch_status("gemm_f32_fold_kernel"));
  }
  return WAFER_HIP_OK;
}

template <int T, bool RHS_T> int dispatch_epi(wafer_hip_context *ctx, const F32GemmArgs &a, uint32_t epi) {
  switch (epi) {
    case EPI_NONE: return launch_f32<T, RHS_T, EPI_NONE>(ctx, a);
    case EPI_BIAS: return launch_f32<T, RHS_T, EPI_BIAS>(ctx, a);
    default: return launch_f32<T, RHS_T, EPI_GELU>(ctx, a);
  }
}

template <int T> int dispatch_rhs(wafer_hip_context *ctx, const F32GemmArgs &a, uint32_t rhs_t, uint32_t epi) {
  return rhs_t ? dispatch_epi<T, true>(ctx, a, epi) : dispatch_epi<T, false>(ctx, a, epi);
}

}  // namespace
}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_gemm_f32_mfma(wafer_hip_context *ctx, const float *lhs, const float *rhs,
                                       const float *bias, float *dst, uint32_t m, uint32_t k, uint32_t n,
                                       uint32_t rhs_orientation, uint32_t epilogue) {
  WAFER_CHECK_CTX(ctx);
  if (!lhs || !rhs || !dst) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_f32_mfma: null operand");
  if (m == 0 || n == 0 || k == 0) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_f32_mfma: empty extent");
  if (rhs_orientation > WAFER_GEMM_TRANSPOSE)
    return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_f32_mfma: rhs orientation must be Normal or Transpose");
  if (epilogue > WAFER_HIP_EPILOGUE_BIAS_GELU_TANH)
    return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_f32_mfma: unknown epilogue");
  if (epilogue != WAFER_HIP_EPILOGUE_NONE && !bias)
    return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_f32_mfma: the bias epilogues need a bias vector");
  if (k % 8 != 0) return fail(WAFER_HIP_E_UNSUPPORTED, "gemm_f32_mfma: k must be a multiple of 8");
  if (m > (1u << 24) || n > (1u << 24) || k > (1u << 24) || (uint64_t)m * k > (1ull << 31) ||
      (uint64_t)k * n > (1ull << 31) || (uint64_t)m * n > (1ull << 31))
    return fail(WAFER_HIP_E_UNSUPPORTED, "gemm_f32_mfma: an operand exceeds 2^31 elements");
  if ((((uintptr_t)lhs) & 15) || (rhs_orientation == WAFER_GEMM_TRANSPOSE && (((uintptr_t)rhs) & 15)) ||
      (((uintptr_t)dst) & 15))
    return fail(WAFER_HIP_E_UNSUPPORTED, "gemm_f32_mfma: lhs, dst and a Transposed rhs must be 16-byte aligned");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));

  F32GemmArgs a{};
  a.a = lhs;
  a.b = rhs;
  a.bias = bias;
  a.y = dst;
  a.m = (int)m;
  a.k = (int)k;
  a.n = (int)n;
  // Tile choice: 32x32 tiles when they fill the CUs; else 16x16 tiles when
  // those do (a quarter of the work per tile, no fold launch); else split k
  // over workgroups (at least 32 k per wave) and fold in a second launch.
  const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  const int64_t tiles32 = (int64_t)((m + 31) / 32) * ((n + 31) / 32);
  const int64_t tiles16 = (int64_t)((m + 15) / 16) * ((n + 15) / 16);
  const int T = tiles32 >= cus || tiles16 < cus || k % 16 != 0 ? 32 : 16;
  a.tiles_m = (int)((m + T - 1) / T);
  a.tiles_n = (int)((n + T - 1) / T);
  const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
  const int kg4 = 4 * 4 * (64 / T);  // k per split granule: 4 waves x one group
  const int64_t ksplit = tiles >= cus ? 1 : std::max<int64_t>(1, std::min<int64_t>(cus / tiles, k / 128));
  a.kchunk = (int)(((k + ksplit - 1) / ksplit + kg4 - 1) / kg4 * kg4);
  a.ksplit = (int)((k + a.kchunk - 1) / a.kchunk);
  if ((int64_t)a.tiles_m * a.tiles_n * a.ksplit > 0x7fffffff)
    return fail(WAFER_HIP_E_UNSUPPORTED, "gemm_f32_mfma: grid too large");
  if (a.ksplit > 1) {
    WAFER_TRY(ensure_workspace(ctx, &ctx->partials, &ctx->partials_bytes,
                               (size_t)a.ksplit * m * n * sizeof(float)));
    a.part = (float *)ctx->partials;
  }
  return T == 32 ? dispatch_rhs<32>(ctx, a, rhs_orientation, epilogue)
                 : dispatch_rhs<16>(ctx, a, rhs_orientation, epilogue);
}
