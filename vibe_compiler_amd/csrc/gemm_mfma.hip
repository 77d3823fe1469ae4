// gemm_mfma.hip -- matrix-core GEMMs for gfx950: bf16/f16 (f32 accumulate)
// and int8 (exact int32 accumulate, fused dequant to bf16).
//
// Both run one kernel template on the "NT" operand form, A [M, K] and
// Bt [N, K], both K-contiguous, so every lane's MFMA operand is one 16-byte
// LDS read:
//   bf16/f16: v_mfma_f32_32x32x16_{bf16,f16}  (16 elements = 32 B of K/step)
//   int8:     v_mfma_i32_32x32x32_i8          (32 elements = 32 B of K/step)
// A workgroup of 8 waves (2 x 4) computes a BMxBN tile (256x256, or 128x128
// when the 256 grid would leave CUs idle); each wave owns (BM/2) x (BN/4),
// two waves per SIMD.  K slices of A and Bt (128 bytes per stage when K
// allows, else 64) go global -> LDS directly (global_load_lds_dwordx4, no
// VGPR round trip) into a ring of stage buffers filling 128 KiB (2 stages
// of 128-byte slices for 256x256 tiles, else 4), issued NS-1 stages ahead;
// one barrier per stage, placed before the stage's last k-step so that each
// k-step's fragment reads overlap the previous k-step's MFMAs.  The 16-byte
// chunks of each LDS row are XOR-swizzled so that the rows one fragment
// read touches hit distinct bank groups (conflict-free ds_read_b128).  A normal
// (K-major) rhs is first re-laid out to Bt by a transpose kernel into
// context scratch.  Workgroup ids are mapped so that the 32 tiles one XCD
// runs at a time form a 4x8 block of the output (whole rounds of 256 tiles),
// or walk that XCD's own column strip in 4-row groups (other grids whose tile
// rows divide by 4 and tile columns by 8), bounding the XCD's L2 working set.
// Tiles are 256x256 when they fill the chip, 128x192 where that saves a round
// of workgroups, else 128x128.  For 16-bit operands the 256x256, 256x224
// (SwiGLU) and 128x192 tiles run on a 4-wave kernel instead (one wave per
// SIMD, K slices moved by LDS DMA into a ring of 128 KiB), and long-K grids
// of at most one round of 128x128 tiles split K over 4 workgroups of
// 256x256 tiles with a fold launch.
//
// int8 semantics (no reference implementation exists; the closed form on the
// reference's conversion routes): acc = sum_k int32(a)*int32(b) exactly
// (|acc| <= k*128*128 < 2^31 for k <= 131071), y = bf16_RNE(f32_RNE(
// f32_RNE(acc) * scale[n])) -- int32_fp32 route, CT Mul, fp32_bf16 route
// (lib/Wafer/Target/TargetFormat.cpp:174,192).  Integer sums are
// order-independent, so the result is bit-exact.
#include "common.h"

#include <type_traits>

namespace wafer {
namespace {

enum { KIND_BF16 = 0, KIND_F16 = 1, KIND_I8 = 2 };
typedef int v2i32 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i32 lds_v2i32;
constexpr int BKB = 64;  // K bytes must be a multiple of the smaller LDS stage

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
// OUT_SWIGLU (bf16 or f16): the rhs rows come in 32-row groups, 16 gate rows
// then the 16 up rows of the same features, and y[m, f] =
// T(silu_mul(T(gate), T(up))) over N/2 features, T the storage format (the narrowed
// products, then the silu_mul region).  In a 32x32 MFMA tile the gate
// values of 16 features sit in lanes l32 < 16 and their up values in lanes
// l32 + 16; one v_permlane16_swap per register pair brings both to one
// lane (swiglu_pair).
// OUT_NARROW_RES: the narrowed product plus a residual tensor of the same
// format and shape, y = Add(narrow(acc), res) -- the GEMM's narrow output
// followed by the CT Add command, bit for bit (y may be res itself: every
// element is read before it is written, by the same lane).
enum { OUT_F32 = 0, OUT_NARROW = 1, OUT_I8_DEQUANT = 2, OUT_SWIGLU = 3, OUT_NARROW_RES = 4 };

// f16 -> f32 by v_cvt_f32_f16: exact for every finite f16 (subnormals
// included, f16 denormals are on); a NaN keeps a NaN, and the sum it enters
// narrows to the canonical f16 NaN either way, so the residual sum matches
// the portable widening bit for bit.
__device__ inline float widen_f16(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// f32 -> f16 by v_cvt_f16_f32 in the default round-to-nearest-even mode, with
// gradual underflow and overflow to +-inf; a NaN narrows to the canonical
// 0x7e00 as f32_to_f16 does.
__device__ inline uint16_t narrow_f16(float x) {
  x = f32_rounded(x);
  return x != x ? (uint16_t)0x7e00u : __builtin_bit_cast(uint16_t, (_Float16)x);
}

// SwiGLU from accumulator registers r and r + 1 (r even: rows q and q + 1)
// of a 32x32 tile whose columns 0..15 are gate and 16..31 up features:
// v_permlane16_swap exchanges lanes 16..31 of `a` with lanes 0..15 of `b`
// (and 48..63 with 32..47), after which lane l holds gate and up of feature
// l % 16 for row q (l % 32 < 16) or q + 1 (l % 32 >= 16).  Returns the bf16
// silu_mul of the narrowed pair in the storage format (bf16 or f16).
template <int KIND>
__device__ inline uint16_t swiglu_pair(float a, float b) {
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  if constexpr (KIND == KIND_F16) {
    const float gv = widen_f16(narrow_f16(__uint_as_float(t[0])));
    const float uv = widen_f16(narrow_f16(__uint_as_float(t[1])));
    return narrow_f16(silu_mul_1(gv, uv));
  } else {
    const uint32_t gu = bf16x2_rne(__uint_as_float(t[0]), __uint_as_float(t[1]));
    const float gv = __uint_as_float(gu << 16), uv = __uint_as_float(gu & 0xffff0000u);
    const float y = silu_mul_1(gv, uv);
    return (uint16_t)bf16x2_rne(y, y);
  }
}

struct GemmArgs {
  const uint8_t *a;    // [M, K] elements, K-contiguous
  const uint8_t *bt;   // [N, K] ([K, N] for the BKN int8 kernel)
  void *y;             // [M, N]
  int32_t *acc_out;    // int8 only, optional [M, N]
  const float *scale;  // int8 only, [N]
  int m, n, kbytes;    // K in bytes
  int tiles_m, tiles_n;  // ceil(M / BM), ceil(N / BN)
  const uint16_t *res;   // OUT_NARROW_RES only, [M, N]
  // split-K (4-wave kernel only): ksplit > 1 workgroups per tile each take
  // kbytes / ksplit of K and store f32 partial tiles to part [ksplit, M, N],
  // which a fold launch adds in split order
  int ksplit;
  float *part;
};

// XCD-aware tile order: workgroup ids are dealt round-robin over the 8
// XCDs; the ids one XCD receives cover a 4 x 8 block of output tiles when the
// grid is whole rounds of 256 tiles, else (tile rows divisible by 4, tile
// columns by 8) the XCD's own column strip walked in 4-row groups.
__device__ inline void tile_coords(const GemmArgs &args, int bid, int &tm, int &tn) {
  const int tiles_m = args.tiles_m, tiles_n = args.tiles_n;
  const int total = tiles_m * tiles_n;
  if (total % 256 == 0 && tiles_m % 4 == 0 && tiles_n % 8 == 0) {
    const int group = bid / 256, inner = bid % 256;  // 256 tiles per round
    const int xcd = inner % 8, j = inner / 8;        // 32 tiles per XCD
    const int gn = tiles_n / 8;                      // 4x8 blocks across the grid
    const int blk = group * 8 + xcd;                 // which 4x8 block
    const int bm = blk / gn, bn = blk % gn;
    tm = bm * 4 + j / 8;
    tn = bn * 8 + j % 8;
  } else if (tiles_m % 4 == 0 && tiles_n % 8 == 0) {
    // XCD x owns the column strip [x sw, (x + 1) sw) of the grid, walked in
    // groups of 4 tile rows, column by column within a group: the 32 tiles
    // an XCD runs at once span 4 rows and 8 columns
    const int xcd = bid % 8, j = bid / 8;
    const int sw = tiles_n / 8, per_group = 4 * sw;
    const int grp = j / per_group, w = j % per_group;
    tm = grp * 4 + w % 4;
    tn = xcd * sw + w / 4;
  } else {
    tm = bid / tiles_n;
    tn = bid % tiles_n;
  }
}

// Epilogue shared by the GEMM kernels: lane holds column l32 and rows
// 8*(r/4) + 4*g + r%4 of each 32x32 tile of its wave's sub-tile.  `stage` is
// this wave's LDS staging area of (BM/WM) x (output columns per wave) 16-bit
// values, used after a barrier that retires every wave's main-loop LDS
// traffic.
template <int KIND, int BM, int BN, int OUT, bool TAIL, int WM, int WN, bool STAGE = true>
__device__ __attribute__((always_inline)) inline void gemm_store(
    const GemmArgs &args, typename Acc<KIND>::T (&acc)[BM / WM / 32][BN / WN / 32], int m0, int n0,
    char *stage) {
  constexpr int WTM = BM / WM / 32, WTN = BN / WN / 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, g = lane >> 5;
  // Staged epilogue (16-bit outputs of full tiles): each wave narrows its
  // sub-tile into LDS as row-major [OR][OC] 16-bit values (16-byte chunks of
  // a row XOR-swizzled by (row / 4) % CPR, so the two row groups of one
  // ds_write_b16 land in distinct banks), then reads it back 16 bytes per
  // lane and stores whole 16-byte row segments (64 lanes cover 1 KiB of
  // consecutive rows) instead of scattered 2-byte stores.  The sub-tiles are
  // staged in sA, then sB, after a barrier that retires every wave's fragment
  // reads and stage moves.
  if constexpr (OUT != OUT_F32) {
    constexpr int OR = BM / WM;                                     // rows per wave
    constexpr int OC = OUT == OUT_SWIGLU ? BN / WN / 2 : BN / WN;   // output columns per wave
    constexpr int CPR = OC * 2 / 16;                                // 16-byte chunks per row
    static_assert(OR * CPR % 64 == 0, "whole 16-byte store rounds");
    // position of 16-byte chunk c in a staged row: XOR when CPR is a power of
    // two, else a rotation; either way rows 4 apart put a chunk in different
    // positions
    auto spos = [](int row, int c) __attribute__((always_inline)) {
      return (CPR & (CPR - 1)) == 0 ? c ^ ((row >> 2) & (CPR - 1)) : (c + (row >> 2)) % CPR;
    };
    // the first IN_A waves stage in sA, the others in sB
    const int ldy = OUT == OUT_SWIGLU ? args.n / 2 : args.n;
    const bool staged = STAGE && !TAIL && ldy % 8 == 0 && (((uintptr_t)args.y) & 15) == 0 &&
                        (OUT != OUT_NARROW_RES || (((uintptr_t)args.res) & 15) == 0) &&
                        (OUT != OUT_I8_DEQUANT || args.acc_out == nullptr);
    if (staged) {
      // the residual chunks this lane stores load first, behind the staging
      // (up to 8 per lane; the 256x256 tiles' 16 load in the store loop)
      constexpr int NQ = OR * CPR / 64;
      constexpr bool PRE = OUT == OUT_NARROW_RES && NQ <= 8;
      const int col0 = OUT == OUT_SWIGLU ? (n0 + wn * (BN / WN)) / 2 : n0 + wn * (BN / WN);
      u32x4 rr[PRE ? NQ : 1];
      if constexpr (PRE) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const int idx = q * 64 + lane, row = idx / CPR, c = idx % CPR;
          rr[q] = *(const u32x4 *)(args.res + (size_t)(m0 + wm * OR + row) * ldy + col0 + c * 8);
        }
      }
      __syncthreads();
      auto put = [&](int row, int col, uint16_t v) __attribute__((always_inline)) {
        *(uint16_t *)(stage + row * (CPR * 16) + (spos(row, col >> 3) << 4) + (col & 7) * 2) = v;
      };
      if constexpr (OUT == OUT_SWIGLU) {
        static_assert(KIND == KIND_BF16 || KIND == KIND_F16, "the fused epilogue serves bf16 and f16");
        const int hi = (l32 >> 4) & 1;  // lanes 16..31 of each half take the odd row
#pragma unroll
        for (int i = 0; i < WTM; ++i)
#pragma unroll
          for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int r = 0; r < 16; r += 2)
              put(i * 32 + 8 * (r >> 2) + 4 * g + (r & 3) + hi, j * 16 + (l32 & 15),
                  swiglu_pair<KIND>((float)acc[i][j][r], (float)acc[i][j][r + 1]));
      } else {
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
          float sc = 0.0f;
          if (OUT == OUT_I8_DEQUANT) sc = args.scale[n0 + wn * (BN / WN) + j * 32 + l32];
#pragma unroll
          for (int i = 0; i < WTM; ++i)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
              // rows r and r + 1 of the lane's column, narrowed as a pair
              uint32_t v2;
              if constexpr (OUT == OUT_NARROW || OUT == OUT_NARROW_RES) {
                if constexpr (KIND == KIND_F16)
                  v2 = (uint32_t)narrow_f16((float)acc[i][j][r]) | ((uint32_t)narrow_f16((float)acc[i][j][r + 1]) << 16);
                else
                  v2 = bf16x2_rne((float)acc[i][j][r], (float)acc[i][j][r + 1]);
              } else {
                v2 = bf16x2_rne((float)(int32_t)acc[i][j][r] * sc, (float)(int32_t)acc[i][j][r + 1] * sc);
              }
              const int row = i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
              put(row, j * 32 + l32, (uint16_t)v2);
              put(row + 1, j * 32 + l32, (uint16_t)(v2 >> 16));
            }
          // 128-row sub-tiles: bound the accumulators read out at once
          if constexpr (WTM * WTN > 8) __builtin_amdgcn_sched_barrier(0);
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's own sub-tile
      uint16_t *ybase = (uint16_t *)args.y + (size_t)(m0 + wm * OR) * ldy + col0;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int idx = q * 64 + lane, row = idx / CPR, c = idx % CPR;
        u32x4 v = *(const u32x4 *)(stage + row * (CPR * 16) + (spos(row, c) << 4));
        if constexpr (OUT == OUT_NARROW_RES) {  // + the residual chunk at the same place
          const u32x4 rq =
              PRE ? rr[PRE ? q : 0] : *(const u32x4 *)(args.res + (size_t)(m0 + wm * OR + row) * ldy + col0 + c * 8);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t a = v[e], b = rq[e];
            const float lo = KIND == KIND_F16 ? widen_f16((uint16_t)a) + widen_f16((uint16_t)b)
                                              : bf16_to_f32((uint16_t)a) + bf16_to_f32((uint16_t)b);
            const float hi = KIND == KIND_F16 ? widen_f16((uint16_t)(a >> 16)) + widen_f16((uint16_t)(b >> 16))
                                              : bf16_to_f32((uint16_t)(a >> 16)) + bf16_to_f32((uint16_t)(b >> 16));
            v[e] = KIND == KIND_F16 ? ((uint32_t)narrow_f16(lo) | ((uint32_t)narrow_f16(hi) << 16))
                                    : bf16x2_rne(lo, hi);
          }
        }
        // the int8 GEMM's bf16 output streams out with non-temporal stores
        // (4096^3: 62.9-63.3 -> 62.2-62.7 us on one box); the 16-bit GEMMs
        // keep plain stores, their outputs feed the next kernel of a layer
        if constexpr (OUT == OUT_I8_DEQUANT)
          __builtin_nontemporal_store(v, (u32x4 *)(ybase + (size_t)row * ldy + c * 8));
        else
          *(u32x4 *)(ybase + (size_t)row * ldy + c * 8) = v;
        // keep the in-loop residual loads (and, past 16 rounds, the staged
        // reads) from all hoisting at once
        if constexpr (OUT == OUT_NARROW_RES && !PRE) __builtin_amdgcn_sched_barrier(0);
        else if constexpr (NQ > 16) {
          if ((q & 7) == 7) __builtin_amdgcn_sched_barrier(0);
        }
      }
      return;
    }
  }
  // epilogue: lane holds column l32 and rows 8*(r/4) + 4*g + r%4 of each tile
  if constexpr (OUT == OUT_SWIGLU) {
    // each 32-column tile holds 16 features (gate columns 0..15, up 16..31)
    static_assert(KIND == KIND_BF16 || KIND == KIND_F16, "the fused epilogues serve bf16 and f16");
    const int nf = args.n / 2;
    const int hi = (l32 >> 4) & 1;
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const int feat = (n0 + wn * (BN / WN) + j * 32) / 2 + (l32 & 15);
        const bool col_ok = !TAIL || feat < nf;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          // every lane takes part in the swap before the tail test
          const uint16_t v = swiglu_pair<KIND>((float)acc[i][j][r], (float)acc[i][j][r + 1]);
          const int row = m0 + wm * (BM / WM) + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3) + hi;
          if (TAIL && !(col_ok && row < args.m)) continue;
          ((uint16_t *)args.y)[(size_t)row * nf + feat] = v;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
      const int col = n0 + wn * (BN / WN) + j * 32 + l32;
      const bool col_ok = !TAIL || col < args.n;
      float sc = 0.0f;
      if (OUT == OUT_I8_DEQUANT && col_ok) sc = args.scale[col];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * (BM / WM) + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (TAIL && !(col_ok && row < args.m)) continue;
        const size_t o = (size_t)row * args.n + col;
        if (OUT == OUT_F32) {
          ((float *)args.y)[o] = (float)acc[i][j][r];
        } else if (OUT == OUT_NARROW) {
          const float v = (float)acc[i][j][r];
          ((uint16_t *)args.y)[o] = KIND == KIND_F16 ? narrow_f16(v) : f32_to_bf16(v);
        } else if (OUT == OUT_NARROW_RES) {
          const float v = (float)acc[i][j][r];
          const float nv = KIND == KIND_F16 ? widen_f16(narrow_f16(v)) : bf16_to_f32(f32_to_bf16(v));
          const float rv = KIND == KIND_F16 ? widen_f16(args.res[o]) : bf16_to_f32(args.res[o]);
          ((uint16_t *)args.y)[o] = KIND == KIND_F16 ? narrow_f16(nv + rv) : f32_to_bf16(nv + rv);
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


// TAIL: the grid's last tile row / column may hold fewer than BM / BN rows /
// columns.  Those tiles load their last real A row (Bt row) again in place of
// the missing ones, so every load stays inside the operands, and store only
// the outputs that exist.
//
//
// WM x WN waves, each owning a (BM/WM) x (BN/WN) sub-tile: 2 x 4 (8 waves,
// two per SIMD) by default; 4 x 2 serves tiles whose width is not a multiple
// of 128 (128 x 192, 128 x 384); 2 x 2 (4 waves, one per SIMD with all 512
// registers) halves the LDS fragment traffic per MFMA.
//
// BKN (int8, 256-column tiles): the rhs is read as stored, [K, N] row-major
// (`bt` points at it), with no re-layout pass.  A B stage then holds SB rows
// of K, BN bytes each; 16-byte chunk c of k-row r sits at position
// c ^ 2 (r & 7).  The MFMA's B fragment (16 consecutive k of one column) is
// gathered by two ds_read_b64_tr_b8: in each 16-lane group lane i addresses
// k-row i / 2, bytes 8 (i % 2) .. +7 of one chunk, and receives byte i of
// each of the 8 rows, so the 16 lanes get 8 k of the chunk's 16 columns.
// The 8 rows of a group sit at 8 distinct chunk positions of one parity, and
// the neighbouring group (the next chunk) at the other parity: no bank
// conflicts.
template <int KIND, int BM, int BN, int OUT, bool TAIL, int SB, int WM = 2, int WN = 4, bool BKN = false>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(1, WM * WN == 4 ? 1 : 2))) void
gemm_nt_kernel(GemmArgs args) {
  static_assert(!BKN || (KIND == KIND_I8 && BN == 256 && !TAIL && (BN / WN) % 32 == 0), "[K,N] rhs: int8, 256 columns");
  constexpr int NT = 64 * WM * WN, NW = WM * WN;
  static_assert(BM % (32 * WM) == 0 && BN % (32 * WN) == 0, "whole 32x32 MFMA tiles per wave");
  constexpr int WTM = BM / WM / 32, WTN = BN / WN / 32;  // 32x32 MFMA tiles per wave
  // SB bytes of K per stage (2 or 4 MFMA k-steps); NS stages fill 128 KiB
  constexpr int CH = SB / 16, KS = SB / 32;
  constexpr int NS = (128 * 1024) / ((BM + BN) * SB) < 4 ? (128 * 1024) / ((BM + BN) * SB) : 4;
  static_assert(NS >= 2, "at least two stages");
  // one LDS object holding the A stages, then the B stages (with A and B in
  // two objects the compiler put an s_waitcnt vmcnt before the A fragment
  // reads for the A moves in flight)
  __shared__ __align__(1024) uint8_t lds[NS * (BM + BN) * SB];
  u32x4 (*const sA)[BM * CH] = (u32x4 (*)[BM * CH])lds;
  u32x4 (*const sB)[BN * CH] = (u32x4 (*)[BN * CH])(lds + NS * BM * SB);
  // 16-byte chunk c of row r sits at position swz(r, c) (an involution in c):
  // 16 consecutive rows read at one chunk hit 16 distinct 16-byte bank
  // groups, and so do 32 consecutive rows for 128-byte rows
  // (BKN: chunk ^ ((row >> 1) & 7), a function of row % 16, so the DMA's
  // per-lane offsets take two forms, by instruction parity)
  auto swz = [](int row, int chunk) __attribute__((always_inline)) {
    if constexpr (BKN) return chunk ^ ((row >> 1) & 7);
    return SB == 64 ? chunk ^ ((row >> 2) & 3) : chunk ^ (((row >> 1) ^ (row >> 4)) & 7);
  };

  int tm, tn;
  tile_coords(args, blockIdx.x, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, g = lane >> 5;

  typename Acc<KIND>::T acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // Direct-to-LDS staging: NS stage buffers in a ring, loads issued NS-1
  // stages ahead with global_load_lds_dwordx4 (no VGPR round trip).  One
  // instruction fills 1 KiB = 1024/SB rows x CH chunks of a stage buffer:
  // lane l writes LDS chunk position l % CH of row l / CH, so it loads the
  // global chunk that the swizzle maps there.
  constexpr int RPI = 1024 / SB;                           // rows per instruction
  constexpr int A_INSTR = BM / RPI, B_INSTR = BN / RPI;
  constexpr int PER_WAVE = (A_INSTR + B_INSTR) / (NT / 64);
  static_assert((A_INSTR + B_INSTR) % (NT / 64) == 0, "DMA instructions must split evenly over the waves");
  const uint32_t kb32 = (uint32_t)args.kbytes;
  const int nkt = args.kbytes / SB;
  const size_t kb = (size_t)args.kbytes;
  const uint8_t *abase = args.a + (size_t)m0 * kb;
  const uint8_t *bbase = BKN ? args.bt + n0 : args.bt + (size_t)n0 * kb;
  const uint32_t npitch = (uint32_t)args.n;  // [K, N] rhs row pitch
  const int dma_row = lane / CH, dma_pos = lane % CH;
  // last row of the tile that exists in A / Bt (BM - 1 / BN - 1 unless TAIL)
  const int last_a = TAIL ? min(BM, args.m - m0) - 1 : BM - 1;
  const int last_b = TAIL ? min(BN, args.n - n0) - 1 : BN - 1;
  // BKN: buffer-resource DMA with a scalar offset per instruction.  Each
  // wave moves PA instructions of A, then PB of B, so the operand of an
  // issue slot is known at compile time; the per-lane offsets are set up
  // once, two forms each by instruction parity (the A swizzle and the B
  // k-row swizzle repeat every 16 rows / 8 k-rows).  The offsets are 32-bit:
  // the entry keeps K * N below 2^31 on this path.
  constexpr int PA = BKN ? A_INSTR / NW : 0, PB = BKN ? B_INSTR / NW : 0;
  static_assert(!BKN || (SB == 128 && A_INSTR % NW == 0 && B_INSTR % NW == 0 && PA + PB == PER_WAVE &&
                         PA % 2 == 0 && PB % 2 == 0), "BKN DMA: whole, even instruction shares per wave");
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void *)abase, 0, BKN ? BM * (int)kb32 : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void *)bbase, 0, BKN ? (int)(kb32 * npitch - (uint32_t)n0) : 0, 0x00020000);
  int voa[2] = {0, 0}, vob[2] = {0, 0};
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  if constexpr (BKN) {
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int r16 = par * RPI + lane / CH;           // A row within its 16-row group
      voa[par] = (lane / CH) * (int)kb32 + (((lane % CH) ^ ((r16 >> 1) & 7)) << 4);
      const int kr8 = par * (1024 / BN) + lane / 16;  // B k-row within its 8-row group
      vob[par] = (lane / 16) * (int)npitch + (((lane & 15) ^ (2 * kr8)) << 4);
    }
  }
  // instructions q0 .. q1-1 of this wave's PER_WAVE for stage kt
  auto issue = [&](int kt, int q0, int q1) __attribute__((always_inline)) {
    const int st = kt % NS;
    const uint32_t koff = (uint32_t)min(kt, nkt - 1) * SB;
    if constexpr (BKN) {
#pragma unroll
      for (int q = q0; q < q1; ++q) {
        if (q < PA) {
          const int rel = wv * PA + q;
          const int soff = __builtin_amdgcn_readfirstlane(rel * RPI * (int)kb32 + (int)koff);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              ra, (__attribute__((address_space(3))) void *)((char *)&sA[st][0] + rel * 1024), 16, voa[q & 1],
              soff, 0, 0);
        } else {
          const int rel = wv * PB + (q - PA);
          const int soff = __builtin_amdgcn_readfirstlane(((int)koff + rel * (1024 / BN)) * (int)npitch);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rb, (__attribute__((address_space(3))) void *)((char *)&sB[st][0] + rel * 1024), 16,
              vob[(q - PA) & 1], soff, 0, 0);
        }
      }
      return;
    }
#pragma unroll
    for (int q = q0; q < q1; ++q) {
      const int ins = wave * PER_WAVE + q;  // 0 .. A_INSTR + B_INSTR - 1
      const bool is_a = ins < A_INSTR;
      const int row = (is_a ? ins : ins - A_INSTR) * RPI + dma_row;
      const int chunk = swz(row, dma_pos);
      const int src_row = TAIL ? min(row, is_a ? last_a : last_b) : row;
      const uint8_t *src = (is_a ? abase : bbase) + (src_row * kb32 + koff + chunk * 16);
      u32x4 *dst = is_a ? &sA[st][(ins * RPI) * CH] : &sB[st][((ins - A_INSTR) * RPI) * CH];
      __builtin_amdgcn_global_load_lds((const void *)src, (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
    }
  };

  u32x4 fa[2][WTM], fb[2][WTN];  // fragments of two k-steps
  auto read_frags = [&](int buf, int ks, int f) __attribute__((always_inline)) {
    const int chunk = ks * 2 + g;
#pragma unroll
    for (int i = 0; i < WTM; ++i) {
      const int row = wm * (BM / WM) + i * 32 + l32;
      fa[f][i] = sA[buf][row * CH + swz(row, chunk)];
    }
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
      const int row = wn * (BN / WN) + j * 32 + l32;
      fb[f][j] = sB[buf][row * CH + swz(row, chunk)];
    }
  };
  auto mfmas = [&](int f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j) acc[i][j] = mfma<KIND>(fa[f][i], fb[f][j], acc[i][j]);
  };

  // Software pipeline over the KS k-steps of a stage, with the stage barrier
  // before the last one: each k-step's fragment reads are issued between
  // the MFMAs of the previous one, so LDS latency hides behind matrix work.
  // The stage's DMA issues ride in the first k-steps.  sched_barrier fences
  // keep the compiler from moving MFMAs across the barrier; sched_group_barrier
  // pins the interleave (masks: 0x008 MFMA, 0x100 LDS read, 0x010 VMEM,
  // which covers the DMA issues).
  if constexpr (BKN) {
    // [K,N] rhs: every B fragment of a stage is read right after the
    // barrier that makes the stage visible (k-steps 0 .. KS-2, k-step KS-1's
    // at the start of k-step 0), and the next stage's DMA moves go out only
    // after them.  ds_read_b64_tr_b8 carries no LDS alias information, so the
    // compiler puts an s_waitcnt vmcnt(0) before each one issued while an LDS
    // DMA may be in flight; read this way, every such wait falls where the
    // stage barrier has already drained the DMA.  A fragments (plain LDS
    // loads) keep the per-k-step pipeline.
    u32x4 fbs[KS][WTN];
    const char *sbb = (const char *)&sB[0][0];
    const int l16 = lane & 15;
    // k-rows 32 ks + 16 g + 8 h + lane % 16 / 2 (h = 0, 1), chunk of
    // columns wn * BN / WN + 32 j + 16 (lane / 16 % 2); the row's swizzle
    // is 2 (row & 7) = 2 (lane % 16 / 2)
    auto read_b = [&](int buf, int ks) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const int c = (wn * (BN / WN) + j * 32) / 16 + ((lane >> 4) & 1);
        const int off = buf * (SB * BN) + (ks * 32 + 16 * g + (l16 >> 1)) * BN + ((c ^ (2 * (l16 >> 1))) * 16) +
                        8 * (l16 & 1);
        const v2i32 lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i32 *)(sbb + off));
        const v2i32 hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i32 *)(sbb + off + 8 * BN));
        fbs[ks][j] = __builtin_bit_cast(u32x4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3));
      }
    };
    auto read_a = [&](int buf, int ks, int f) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < WTM; ++i) {
        const int row = wm * (BM / WM) + i * 32 + l32;
        fa[f][i] = sA[buf][row * CH + swz(row, ks * 2 + g)];
      }
    };
    auto mfmas_b = [&](int f, int ks) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j) acc[i][j] = mfma<KIND>(fa[f][i], fbs[ks][j], acc[i][j]);
    };
    constexpr int NM = WTM * WTN;
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue(s, 0, PER_WAVE);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 2) * PER_WAVE) : "memory");
    read_a(0, 0, 0);
#pragma unroll
    for (int ks = 0; ks < KS - 1; ++ks) read_b(0, ks);
    for (int kt = 0; kt < nkt; ++kt) {
      const int buf = kt % NS;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int cur = ks & 1;
        if (ks == 0) {
          // the stage's last B fragments, then stage kt+NS-1's moves into
          // slot (kt-1) % NS, which every wave finished reading before the
          // last barrier
          read_b(buf, KS - 1);
          read_a(buf, 1, cur ^ 1);
          mfmas_b(cur, 0);
          issue(kt + NS - 1, 0, PER_WAVE);
          __builtin_amdgcn_sched_group_barrier(0x100, 2 * WTN, 0);
#pragma unroll
          for (int t = 0; t < NM; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (t < WTM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (t < PER_WAVE) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
        } else if (ks < KS - 1) {
          read_a(buf, ks + 1, cur ^ 1);
          mfmas_b(cur, ks);
#pragma unroll
          for (int t = 0; t < NM; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (t < WTM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
        } else {
          // stage kt+1 has landed for this wave and its reads of stage kt
          // are complete; after the barrier stage kt+1 is visible to every
          // wave (past the last stage a clamped copy, read but unused)
          asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NS - 2) * PER_WAVE) : "memory");
          __builtin_amdgcn_sched_barrier(0);
          read_a((kt + 1) % NS, 0, cur ^ 1);
#pragma unroll
          for (int k2 = 0; k2 < KS - 1; ++k2) read_b((kt + 1) % NS, k2);
          mfmas_b(cur, KS - 1);
#pragma unroll
          for (int t = 0; t < NM; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, (WTM + 2 * WTN * (KS - 1) + NM - 1) / NM, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  } else {
    constexpr int NR = WTM + WTN;                  // fragment reads per k-step
    constexpr int DKS = KS > 2 ? KS - 2 : 1;       // k-steps that carry DMA issues
    constexpr int NV = (PER_WAVE + DKS - 1) / DKS;  // DMA issues per such k-step
  #pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue(s, 0, PER_WAVE);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 2) * PER_WAVE) : "memory");
    read_frags(0, 0, 0);
    for (int kt = 0; kt < nkt; ++kt) {
      const int buf = kt % NS;
  #pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int cur = ks & 1;
        if (ks < KS - 1) {
          read_frags(buf, ks + 1, cur ^ 1);
          mfmas(cur);
          // into buffer (kt - 1) % NS, which every wave finished reading
          // before the last barrier
          if (ks < DKS) issue(kt + NS - 1, min(ks * NV, PER_WAVE), min((ks + 1) * NV, PER_WAVE));
  #pragma unroll
          for (int r = 0; r < NR; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (ks < DKS && r < NV) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
          }
          if (ks < DKS && NV > NR) {
  #pragma unroll
            for (int v = NR; v < NV; ++v) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
            }
          }
          __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
          __builtin_amdgcn_sched_barrier(0);
        } else {
          // this wave's stage-(kt+1) loads have landed (the NS-2 later stages
          // may stay in flight) and its reads of stage kt are complete; after
          // the barrier stage kt+1 is visible to every wave and buffer kt % NS
          // is free
          asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NS - 2) * PER_WAVE) : "memory");
          __builtin_amdgcn_sched_barrier(0);
          // stage kt+1's first fragments (past the last stage a clamped copy, unused)
          read_frags((kt + 1) % NS, 0, cur ^ 1);
          mfmas(cur);
  #pragma unroll
          for (int r = 0; r < NR; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }
  // the clamped tail loads are still in flight: drain before the LDS goes away
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  {
    constexpr int OR = BM / WM, OC = OUT == OUT_SWIGLU ? BN / WN / 2 : BN / WN;
    constexpr int PER = OR * OC * 2, IN_A = (NS * BM * CH * 16) / PER < NW ? (NS * BM * CH * 16) / PER : NW;
    static_assert(OUT == OUT_F32 || (NW - IN_A) * PER <= NS * BN * CH * 16, "the staged sub-tiles fit in sA and sB");
    char *stage = wave < IN_A ? (char *)&sA[0][0] + wave * PER : (char *)&sB[0][0] + (wave - IN_A) * PER;
    gemm_store<KIND, BM, BN, OUT, TAIL, WM, WN>(args, acc, m0, n0, stage);
  }
}

// Scheduling pins for one k-step of the 4-wave kernel: slot t holds one
// MFMA, then (t+1) NR / NM - t NR / NM fragment reads and the same shares of
// XL buffer loads and XW LDS writes.
template <int T, int NM, int NR, int XL, int XW>
__device__ __attribute__((always_inline)) inline void pin_slots() {
  if constexpr (T < NM) {
    constexpr int nr = ((T + 1) * NR) / NM - (T * NR) / NM;
    constexpr int nl = ((T + 1) * XL) / NM - (T * XL) / NM;
    constexpr int nw = ((T + 1) * XW) / NM - (T * XW) / NM;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (nr > 0) __builtin_amdgcn_sched_group_barrier(0x100, nr, 0);
    if constexpr (nl > 0) __builtin_amdgcn_sched_group_barrier(0x020, nl, 0);
    if constexpr (nw > 0) __builtin_amdgcn_sched_group_barrier(0x200, nw, 0);
    pin_slots<T + 1, NM, NR, XL, XW>();
  }
}

// 4-wave tiles (2 x 2 waves, one per SIMD, the accumulators in AGPRs).
// Against the 8-wave kernel each wave's sub-tile is twice as large, so the
// LDS fragment reads per MFMA halve (256 x 256: 128 x 128 per wave).  K
// slices of SB bytes are staged global -> VGPR -> LDS (16-byte buffer loads,
// then ds_write_b128) instead of by LDS DMA, two register sets deep: the
// loads for stage kt+2 are issued over the first half of stage kt's k-steps
// and written to LDS in stage kt+1's second-to-last k-step, a stage and a
// half of lead.  LDS rows are SB + 16 bytes (one 16-byte pad), so 16
// consecutive rows read at one 16-byte chunk hit all 64 banks once and every
// fragment address is a per-lane base plus an immediate.  K bytes a multiple
// of 2 SB (an even number of stages); full tiles only.  16-bit operands (int8
// keeps the 8-wave kernel: with the per-element dequant epilogue compiled in
// this one spills the accumulators, and with the staged epilogue alone it is
// bit-identical but no faster at 4096^3).  STAGE selects the LDS-staged
// epilogue (else per-element stores).
template <int KIND, int OUT, int BM, int BN, int SB, bool STAGE, int WM = 2, int WN = 2, bool SPLIT = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_nt_rs_kernel(GemmArgs args) {
  static_assert(WM * WN == 4, "four waves");
  constexpr int PITCH = SB + 16, KS = SB / 32, CH = SB / 16, RPI = 64 / CH;
  constexpr int WTM = BM / WM / 32, WTN = BN / WN / 32;
  constexpr int A_INSTR = BM / RPI, B_INSTR = BN / RPI;  // RPI rows of SB bytes per wave instruction
  constexpr int PER_WAVE = (A_INSTR + B_INSTR) / 4, NR = WTM + WTN, NM = WTM * WTN;
  // k-steps carrying loads (the first half, else the first KS - 1, else the first) and loads per such k-step
  constexpr int LK = PER_WAVE % (KS / 2) == 0 ? KS / 2 : PER_WAVE % (KS - 1) == 0 ? KS - 1 : 1;
  constexpr int LPK = PER_WAVE / LK;
  constexpr int WK = KS - 2;                             // the k-step that writes the older set to LDS
  static_assert((A_INSTR + B_INSTR) % 4 == 0 && PER_WAVE % LK == 0, "loads split evenly");
  constexpr int OC = OUT == OUT_SWIGLU ? BN / WN / 2 : BN / WN;
  static_assert(!STAGE || 4 * (BM / WM) * OC * 2 <= 2 * (BM + BN) * PITCH, "staging fits in the ring");
  __shared__ __align__(16) uint8_t lds[2 * (BM + BN) * PITCH];
  // split-K: workgroup ids [s tiles, (s + 1) tiles) take split s
  const int tiles = args.tiles_m * args.tiles_n;
  const int split = SPLIT ? (int)blockIdx.x / tiles : 0;
  int tm, tn;
  tile_coords(args, (int)blockIdx.x - split * tiles, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wv / WN, wn = wv % WN;
  const int l32 = lane & 31, g = lane >> 5;

  typename Acc<KIND>::T acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // row stride kb; this workgroup's K slice starts at byte k0 and spans nkt stages
  const int kb = args.kbytes;
  const int kchunk = SPLIT ? kb / args.ksplit : kb;
  const int k0 = split * kchunk, nkt = kchunk / SB;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void *)(args.a + (size_t)m0 * kb + k0), 0, BM * kb - k0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void *)(args.bt + (size_t)n0 * kb + k0), 0, BN * kb - k0, 0x00020000);
  // lane l moves 16-byte chunk l % CH of row l / CH of an RPI-row group
  const int voff = (lane / CH) * kb + (lane % CH) * 16;
  const int woff = (lane / CH) * PITCH + (lane % CH) * 16;

  u32x4 stg[2][PER_WAVE];
  auto gload = [&](int set, int kt, int q0, int q1) __attribute__((always_inline)) {
    const int koff = min(kt, nkt - 1) * SB;  // past the last stage: a clamped copy, never used
#pragma unroll
    for (int q = q0; q < q1; ++q) {
      const int ins = wv * PER_WAVE + q;
      const bool is_a = ins < A_INSTR;
      const int rel = is_a ? ins : ins - A_INSTR;
      const int soff = __builtin_amdgcn_readfirstlane(rel * RPI * kb + koff);
      stg[set][q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(is_a ? ra : rb, voff, soff, 0));
    }
  };
  auto lwrite = [&](int set, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) {
      const int ins = wv * PER_WAVE + q;
      const bool is_a = ins < A_INSTR;
      const int rel = is_a ? ins : ins - A_INSTR;
      *(u32x4 *)(lds + buf * (BM + BN) * PITCH + (is_a ? 0 : BM * PITCH) + rel * RPI * PITCH + woff) = stg[set][q];
    }
  };
  // fragment rows wm*(BM/WM) + 32 i + l32 (A) and wn*(BN/WN) + 32 j + l32
  // (Bt), 16-byte chunk 2 ks + g of the stage's slice
  const int fa_base = (wm * (BM / WM) + l32) * PITCH + g * 16;
  const int fb_base = (BM + wn * (BN / WN) + l32) * PITCH + g * 16;
  u32x4 fa[2][WTM], fb[2][WTN];
  // in the order the next k-step's MFMAs (row-major over i, j) consume them
  auto read_frags = [&](int buf, int ks, int f) __attribute__((always_inline)) {
    const uint8_t *base = lds + buf * (BM + BN) * PITCH + ks * 32;
    fa[f][0] = *(const u32x4 *)(base + fa_base);
#pragma unroll
    for (int j = 0; j < WTN; ++j) fb[f][j] = *(const u32x4 *)(base + fb_base + j * 32 * PITCH);
#pragma unroll
    for (int i = 1; i < WTM; ++i) fa[f][i] = *(const u32x4 *)(base + fa_base + i * 32 * PITCH);
  };
  auto mfmas = [&](int f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j) acc[i][j] = mfma<KIND>(fa[f][i], fb[f][j], acc[i][j]);
  };
  // pins one k-step's order: NM slots of one MFMA followed by their share of
  // the NR fragment reads, XL loads and XW LDS writes
  auto pin = [&](auto XL, auto XW) __attribute__((always_inline)) {
    pin_slots<0, NM, NR, decltype(XL)::value, decltype(XW)::value>();
    __builtin_amdgcn_sched_barrier(0);
  };

  gload(0, 0, 0, PER_WAVE);
  gload(1, 1, 0, PER_WAVE);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_WAVE) : "memory");
  lwrite(0, 0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  read_frags(0, 0, 0);

  // Stage kt reads LDS buffer kt & 1.  Its first KS/2 k-steps issue the
  // loads of stage kt+2 into register set kt & 1; k-step KS-2 writes set
  // (kt+1) & 1 (stage kt+1, loaded during stage kt-1) to buffer (kt+1) & 1,
  // which every wave finished reading before the previous stage barrier;
  // the barrier sits before the last k-step.
  auto stage = [&](int kt, auto P) __attribute__((always_inline)) {
    constexpr int p = decltype(P)::value;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks < KS - 1) {
        read_frags(p, ks + 1, cur ^ 1);
        mfmas(cur);
        if (ks < LK) gload(p, kt + 2, ks * LPK, (ks + 1) * LPK);
        if (ks == WK) {
          // set p^1 was issued a stage before set p: only set p may be in flight
          asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_WAVE) : "memory");
          lwrite(p ^ 1, p ^ 1);
        }
        constexpr int zero = 0;
        (void)zero;
        if (ks < LK && ks == WK) {
          pin(std::integral_constant<int, LPK>{}, std::integral_constant<int, PER_WAVE>{});
        } else if (ks < LK) {
          pin(std::integral_constant<int, LPK>{}, std::integral_constant<int, 0>{});
        } else if (ks == WK) {
          pin(std::integral_constant<int, 0>{}, std::integral_constant<int, PER_WAVE>{});
        } else {
          pin(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
        }
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        read_frags(p ^ 1, 0, cur ^ 1);
        mfmas(cur);
        pin(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
      }
    }
  };
  for (int kt = 0; kt < nkt; kt += 2) {
    stage(kt, std::integral_constant<int, 0>{});
    stage(kt + 1, std::integral_constant<int, 1>{});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (SPLIT) {
    GemmArgs pa = args;
    pa.y = args.part + (size_t)split * args.m * args.n;
    gemm_store<KIND, BM, BN, OUT_F32, false, WM, WN, false>(pa, acc, m0, n0, nullptr);
  } else {
    gemm_store<KIND, BM, BN, OUT, false, WM, WN, STAGE>(args, acc, m0, n0, (char *)lds + wv * (BM / WM) * OC * 2);
  }
}

// 4-wave tiles (one wave per SIMD, the accumulators in AGPRs) with the K
// slices moved global -> LDS by buffer_load ... lds: no staging registers
// and no LDS write instructions, which the register-staged kernel above
// issues in bursts that fill the LDS data FIFO.  Stages of SB bytes of K per
// row (SB / 32 MFMA k-steps) in a ring of 128 KiB (two stages of 256 + 256
// rows at SB = 128, three of 128 + 192 rows).  One DMA instruction fills
// 1024 / SB rows: lane l writes chunk position l % (SB / 16) of its row, so
// it loads the global chunk that the swizzle maps there.  Chunk c of row r
// sits at position c ^ swz(r), swz a function of r % 16 ((r >> 2) & 3 for
// 64-byte rows, (r >> 1) & 7 for 128-byte rows): each fragment address is a
// per-lane base per k-step plus an immediate per 32-row tile, and the 16
// rows one LDS pass of a fragment read serves hit distinct 16-byte bank
// groups.  One barrier
// per stage, before its last k-step: it publishes stage kt+1 and frees
// stage kt's slot.  Each stage's moves go out in two halves spread over the
// MFMA slots of two k-steps (a burst of them fills the texture address
// FIFO): the first half in the last k-step of the stage whose slot it
// refills, the second in the next stage's first k-step.  K bytes a multiple
// of SB; full tiles only.
template <int KIND, int OUT, int BM, int BN, int SB = 64, int WM = 2, int WN = 2, bool SPLIT = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_nt_dma4_kernel(GemmArgs args) {
  static_assert(WM * WN == 4, "four waves");
  static_assert(SB == 64 || SB == 128, "64- or 128-byte stages");
  constexpr int ROWB = SB, CH = SB / 16, KS = SB / 32;      // bytes per row, chunks per row, k-steps per stage
  constexpr int STAGE_BYTES = (BM + BN) * ROWB;
  constexpr int NS = (128 * 1024) / STAGE_BYTES;            // ring of 128 KiB
  constexpr int RPI = 1024 / ROWB;                           // rows per 1 KiB DMA instruction
  constexpr int WTM = BM / WM / 32, WTN = BN / WN / 32;
  // each wave issues a quarter of the A instructions, then a quarter of the
  // Bt ones, so which operand an issue slot moves is known at compile time
  constexpr int A_INSTR = BM / RPI, B_INSTR = BN / RPI;
  constexpr int PA = A_INSTR / 4, PB = B_INSTR / 4, PER_WAVE = PA + PB;
  static_assert(NS >= 2 && A_INSTR % 4 == 0 && B_INSTR % 4 == 0,
                "two stages at least; DMA instructions split evenly over the waves");
  constexpr int OC = OUT == OUT_SWIGLU ? BN / WN / 2 : BN / WN;
  static_assert(4 * (BM / WM) * OC * 2 <= NS * STAGE_BYTES, "staging fits in the ring");
  __shared__ __align__(1024) uint8_t lds[NS * STAGE_BYTES];
  // split-K: workgroup ids [s tiles, (s + 1) tiles) take split s
  const int tiles = args.tiles_m * args.tiles_n;
  const int split = SPLIT ? (int)blockIdx.x / tiles : 0;
  int tm, tn;
  tile_coords(args, (int)blockIdx.x - split * tiles, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wv / WN, wn = wv % WN;
  const int l32 = lane & 31, g = lane >> 5;

  typename Acc<KIND>::T acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int kb = args.kbytes;
  const int kchunk = SPLIT ? kb / args.ksplit : kb;
  const int k0 = split * kchunk, nkt = kchunk / SB;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void *)(args.a + (size_t)m0 * kb + k0), 0, BM * kb - k0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void *)(args.bt + (size_t)n0 * kb + k0), 0, BN * kb - k0, 0x00020000);
  // the swizzle of row r: (r >> 2) & 3 for 64-byte rows, (r >> 1) & 7 for
  // 128-byte rows, a function of r % 16 either way.  The LDS serves a
  // fragment read 16 lanes (16 rows r0 .. r0 + 15, r0 % 16 == 0) at a time
  // over 64 banks, so a 16-byte chunk's bank group is (r * ROWB / 16 + chunk)
  // % 16; with these swizzles the 16 rows hit 16 distinct groups.  (r & 7
  // for 128-byte rows puts rows r and r + 8 on one group: every read took
  // two passes, half the LDS cycles counted as bank conflicts.)
  auto swz = [](int r) __attribute__((always_inline)) { return SB == 64 ? (r >> 2) & 3 : (r >> 1) & 7; };
  // DMA lane offset: row lane / CH of the instruction's RPI rows, global
  // chunk (lane % CH) ^ swz(row); at 128-byte rows an instruction covers 8
  // rows, so odd instructions (rows 8 .. 15 of a 16-row group) take voff1
  const int voff0 = (lane / CH) * kb + (((lane % CH) ^ swz(lane / CH)) << 4);
  const int voff1 = (lane / CH) * kb + (((lane % CH) ^ swz((RPI % 16) + lane / CH)) << 4);
  // instructions q0 .. q1-1 of this wave's PER_WAVE for stage kt into ring
  // slot kt % NS (past the last stage a clamped copy into a free slot, never
  // read)
  auto issue = [&](int kt, int q0, int q1) __attribute__((always_inline)) {
    const int koff = min(kt, nkt - 1) * SB;
    uint8_t *slot = lds + (kt % NS) * STAGE_BYTES;
#pragma unroll
    for (int q = q0; q < q1; ++q) {
      const bool is_a = q < PA;                                 // compile-time
      const int rel = is_a ? wv * PA + q : wv * PB + (q - PA);  // instruction within the operand
      const int ins = is_a ? rel : A_INSTR + rel;
      const int soff = __builtin_amdgcn_readfirstlane(rel * RPI * kb + koff);
      // (ins & 1 is known at compile time where the wave's share of the
      // operand's instructions is even)
      const int voff = RPI < 16 && (ins & 1) ? voff1 : voff0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? ra : rb,
                                               (__attribute__((address_space(3))) void *)(slot + ins * 1024), 16,
                                               voff, soff, 0, 0);
    }
  };
  // fragment offsets within a stage for k-step ks (chunk 2 ks + g):
  // A row wm * (BM / WM) + 32 i + l32, Bt row BM + wn * (BN / WN) + 32 j + l32
  // (32 i keeps the swizzle, so the tiles differ by immediates)
  const int sw = swz(l32);
  int fa_off[KS], fb_off[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    fa_off[ks] = (wm * (BM / WM) + l32) * ROWB + (((2 * ks + g) ^ sw) << 4);
    fb_off[ks] = (BM + wn * (BN / WN) + l32) * ROWB + (((2 * ks + g) ^ sw) << 4);
  }
  u32x4 fa[2][WTM], fb[2][WTN];
  constexpr int NM = WTM * WTN, NR = WTM + WTN;
  // fragment read r of a k-step, in the order its MFMAs (row-major over i,
  // j) consume them: A tile 0, the WTN Bt tiles, A tiles 1 ..
  auto read_frag = [&](int kt, int ks, int f, int r) __attribute__((always_inline)) {
    const uint8_t *base = lds + (kt % NS) * STAGE_BYTES;
    if (r == 0)
      fa[f][0] = *(const u32x4 *)(base + fa_off[ks]);
    else if (r <= WTN)
      fb[f][r - 1] = *(const u32x4 *)(base + fb_off[ks] + (r - 1) * 32 * ROWB);
    else
      fa[f][r - WTN] = *(const u32x4 *)(base + fa_off[ks] + (r - WTN) * 32 * ROWB);
  };
  auto read_frags = [&](int kt, int ks, int f) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < NR; ++r) read_frag(kt, ks, f, r);
  };
  // One k-step in NR slots, each fenced: NM / NR MFMAs of fragment set f,
  // one fragment read of the next k-step (set nf of stage nkt_, k-step nks)
  // and, for `moves` > 0, DMA instructions q0 .. q0 + moves - 1 of stage
  // `mkt` spread over the slots (a burst of DMA issues fills the texture
  // address FIFO and stalls the wave).
  auto kstep = [&](int f, int nkt_, int nks, int nf, int mkt, int q0, int moves) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
#pragma unroll
      for (int t = (r * NM) / NR; t < ((r + 1) * NM) / NR; ++t)
        acc[t / WTN][t % WTN] = mfma<KIND>(fa[f][t / WTN], fb[f][t % WTN], acc[t / WTN][t % WTN]);
      read_frag(nkt_, nks, nf, r);
      if (moves > 0) issue(mkt, q0 + (r * moves) / NR, q0 + ((r + 1) * moves) / NR);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // each stage's moves go out in two halves: the first in the last k-step
  // of the stage whose slot it refills (after that stage's barrier), the
  // second in the first k-step of the next stage
  constexpr int H1 = PER_WAVE / 2, H2 = PER_WAVE - H1;

#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue(s, 0, PER_WAVE);
  issue(NS - 1, 0, H1);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 2) * PER_WAVE + H1) : "memory");
  read_frags(0, 0, 0);
  for (int kt = 0; kt < nkt; ++kt) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks < KS - 1) {
        // this k-step's MFMAs with the next one's fragment reads between
        // them (and, in the first, the second half of stage kt+NS-1's moves)
        kstep(cur, kt, ks + 1, cur ^ 1, kt + NS - 1, H1, ks == 0 ? H2 : 0);
      } else {
        // stage kt+1 has landed for this wave (later stages may still fly)
        // and its reads of stage kt are done; after the barrier stage kt+1
        // is visible to every wave and slot kt % NS is free for stage kt+NS
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NS - 2) * PER_WAVE) : "memory");
        __builtin_amdgcn_sched_barrier(0);
        // the last k-step's MFMAs with stage kt+1's first fragment reads and
        // the first half of stage kt+NS's moves between them
        kstep(cur, kt + 1, 0, cur ^ 1, kt + NS, 0, H1);
      }
    }
  }
  // the clamped tail loads are still in flight: drain before the LDS is reused
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (SPLIT) {
    GemmArgs pa = args;
    pa.y = args.part + (size_t)split * args.m * args.n;
    gemm_store<KIND, BM, BN, OUT_F32, false, WM, WN, false>(pa, acc, m0, n0, nullptr);
  } else {
    gemm_store<KIND, BM, BN, OUT, false, WM, WN, true>(args, acc, m0, n0, (char *)lds + wv * (BM / WM) * OC * 2);
  }
}

// Split-K fold: y = epilogue(part[0] + part[1] + ... + part[S-1]) per
// element, the partial tiles added in split order; OUT_NARROW narrows to
// the input format, OUT_NARROW_RES adds the residual as the per-element
// epilogue does, OUT_F32 stores the sum.  8 elements per thread (M*N a
// multiple of 8).
template <int KIND, int OUT>
__global__ __launch_bounds__(256) void gemm_fold_kernel(const float *__restrict__ part, int ksplit,
                                                        const uint16_t *__restrict__ res, void *__restrict__ y,
                                                        int64_t count) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < count / 8; q += stride) {
    f32x4 lo = *(const f32x4 *)(part + 8 * q), hi = *(const f32x4 *)(part + 8 * q + 4);
    for (int s = 1; s < ksplit; ++s) {
      lo = lo + *(const f32x4 *)(part + (size_t)s * count + 8 * q);
      hi = hi + *(const f32x4 *)(part + (size_t)s * count + 8 * q + 4);
    }
    const float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    if constexpr (OUT == OUT_F32) {
      *(f32x4 *)((float *)y + 8 * q) = lo;
      *(f32x4 *)((float *)y + 8 * q + 4) = hi;
    } else {
      u32x4 rv = {0, 0, 0, 0};
      if constexpr (OUT == OUT_NARROW_RES) rv = *(const u32x4 *)(res + 8 * q);
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (KIND == KIND_F16) {
          uint32_t h[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            uint16_t n = narrow_f16(v[2 * e + t]);
            if constexpr (OUT == OUT_NARROW_RES) n = narrow_f16(widen_f16(n) + widen_f16((uint16_t)(rv[e] >> (16 * t))));
            h[t] = n;
          }
          o[e] = h[0] | (h[1] << 16);
        } else {
          uint32_t n = bf16x2_rne(v[2 * e], v[2 * e + 1]);
          if constexpr (OUT == OUT_NARROW_RES)
            n = bf16x2_rne(__uint_as_float(n << 16) + __uint_as_float(rv[e] << 16),
                           __uint_as_float(n & 0xffff0000u) + __uint_as_float(rv[e] & 0xffff0000u));
          o[e] = n;
        }
      }
      *(u32x4 *)((uint16_t *)y + 8 * q) = o;
    }
  }
}

// Re-layout of a normal rhs B [K, N] into Bt [N, K] (the NT operand form).

// int8, register only: each lane transposes a 16 (k) x 16 (n) byte block
// (16 row loads of 16 bytes, sixteen 4x4 byte transposes with v_perm, 16 row
// stores of 16 bytes) with no LDS and no barrier.  Lane l of a wave takes
// k block l % 8 and n block l / 8 of the wave's 128 x 128 tile, so each load
// instruction reads 8 whole 128-byte row segments and each store writes 8
// whole 128-byte segments of Bt.  K and N multiples of 128.  (8 x 16 blocks
// per lane, two waves per tile, measured slower: 8.8 against 8.2 us at 4096^2.)
__global__ __launch_bounds__(256) void transpose_i8_reg_kernel(const uint8_t *__restrict__ src,
                                                               uint8_t *__restrict__ dst, int K, int N) {
  const int lane = threadIdx.x & 63;
  const int tiles_n = N / 128;
  const long tiles = (long)(K / 128) * tiles_n;
  const long wstride = (long)gridDim.x * (blockDim.x / 64);
  for (long t = (long)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); t < tiles; t += wstride) {
    const int k0 = (int)(t / tiles_n) * 128 + (lane & 7) * 16;
    const int n0 = (int)(t % tiles_n) * 128 + (lane >> 3) * 16;
    u32x4 r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) r[i] = *(const u32x4 *)(src + (size_t)(k0 + i) * N + n0);
    u32x4 o[16];  // o[c]: column n0 + c, bytes k0 .. k0 + 15
#pragma unroll
    for (int j = 0; j < 4; ++j)    // rows 4 j .. 4 j + 3
#pragma unroll
      for (int w = 0; w < 4; ++w) {  // columns 4 w .. 4 w + 3
        const uint32_t a0 = r[4 * j][w], a1 = r[4 * j + 1][w], a2 = r[4 * j + 2][w], a3 = r[4 * j + 3][w];
        const uint32_t t01l = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
        const uint32_t t01h = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
        const uint32_t t23l = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
        const uint32_t t23h = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
        o[4 * w + 0][j] = __builtin_amdgcn_perm(t23l, t01l, 0x05040100u);
        o[4 * w + 1][j] = __builtin_amdgcn_perm(t23l, t01l, 0x07060302u);
        o[4 * w + 2][j] = __builtin_amdgcn_perm(t23h, t01h, 0x05040100u);
        o[4 * w + 3][j] = __builtin_amdgcn_perm(t23h, t01h, 0x07060302u);
      }
#pragma unroll
    for (int c = 0; c < 16; ++c) *(u32x4 *)(dst + (size_t)(n0 + c) * K + k0) = o[c];
  }
}

// 16-bit: a 128-thread block moves a 32 (k) x 64 (n) tile.  Thread (k2, n8)
// loads rows 2 k2, 2 k2 + 1 at elements 8 n8 .. +7; each output dword is the
// 2 k-elements of one column.
__global__ __launch_bounds__(128) void transpose_b16_kernel(const uint16_t *__restrict__ src,
                                                            uint16_t *__restrict__ dst, int K, int N) {
  __shared__ uint32_t T[64][17];  // [n][k / 2], padded
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 64;
  const int tid = threadIdx.x, k2 = tid & 15, n8 = tid >> 4;
  const u32x4 r0 = *(const u32x4 *)(src + (size_t)(k0 + 2 * k2) * N + n0 + 8 * n8);
  const u32x4 r1 = *(const u32x4 *)(src + (size_t)(k0 + 2 * k2 + 1) * N + n0 + 8 * n8);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int n = 8 * n8 + 2 * w;
    T[n + 0][k2] = __builtin_amdgcn_perm(r1[w], r0[w], 0x05040100u);
    T[n + 1][k2] = __builtin_amdgcn_perm(r1[w], r0[w], 0x07060302u);
  }
  __syncthreads();
  // thread tid writes half of row n0 + tid/2 of Bt: 32 bytes of k
  const int n = tid >> 1, q0 = (tid & 1) * 2;
  uint16_t *d = dst + (size_t)(n0 + n) * K + k0;
#pragma unroll
  for (int q = q0; q < q0 + 2; ++q) {
    u32x4 v;
    v[0] = T[n][4 * q + 0];
    v[1] = T[n][4 * q + 1];
    v[2] = T[n][4 * q + 2];
    v[3] = T[n][4 * q + 3];
    *(u32x4 *)(d + 8 * q) = v;
  }
}

// Re-layout for an N that the tiled kernels above do not divide (their
// 16-byte row loads also need N * element bytes to be a multiple of 16): a
// 32 x 32 element tile through LDS with every access bounds-checked.
template <typename T>
__global__ __launch_bounds__(256) void transpose_any_kernel(const T *__restrict__ src, T *__restrict__ dst,
                                                            int K, int N) {
  __shared__ T tile[32][33];
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
  for (int i = ty; i < 32; i += 8)
    if (k0 + i < K && n0 + tx < N) tile[i][tx] = src[(size_t)(k0 + i) * N + n0 + tx];
  __syncthreads();
#pragma unroll
  for (int i = ty; i < 32; i += 8)
    if (n0 + i < N && k0 + tx < K) dst[(size_t)(n0 + i) * K + k0 + tx] = tile[tx][i];
}

template <int KIND, int OUT, int SB>
int launch_gemm_tiles(hipStream_t st, GemmArgs args);

template <int KIND, int OUT, int SB>
int launch_gemm_sb(hipStream_t st, GemmArgs args) {
  if constexpr (OUT != OUT_SWIGLU) {
    return launch_gemm_tiles<KIND, OUT, SB>(st, args);
  } else {
    // 256x224 tiles (4 x 1 waves of 64 x 224, LDS-DMA staging) where their
    // rounds of 256 workgroups take less time than those of 256x256 tiles
    // (gate/up at n 28672: 512 tiles in two rounds of 7/8 the work, against
    // 448 tiles whose second round is three quarters full; 211 against
    // 217 us register-staged in the decoder layer)
    if constexpr (SB == 128) {
      if (args.m % 256 == 0 && args.n % 224 == 0 && args.kbytes % 256 == 0) {
        const long t224 = (long)(args.m / 256) * (args.n / 224), t256 = (long)(args.m / 256) * ((args.n + 255) / 256);
        if (7 * ((t224 + 255) / 256) < 8 * ((t256 + 255) / 256)) {
          args.tiles_m = args.m / 256;
          args.tiles_n = args.n / 224;
          hipLaunchKernelGGL((gemm_nt_dma4_kernel<KIND, OUT, 256, 224, 128, 4, 1>),
                             dim3(args.tiles_m * args.tiles_n), dim3(256), 0, st, args);
          return launch_status("gemm_nt_dma4_kernel");
        }
      }
    }
    args.tiles_m = (args.m + 255) / 256;
    args.tiles_n = (args.n + 255) / 256;
    const dim3 grid(args.tiles_m * args.tiles_n);
    if (args.m % 256 == 0 && args.n % 256 == 0 && args.kbytes % 256 == 0)
      hipLaunchKernelGGL((gemm_nt_rs_kernel<KIND, OUT, 256, 256, 128, false>), grid, dim3(256), 0, st, args);
    else if (args.m % 256 == 0 && args.n % 256 == 0)
      hipLaunchKernelGGL((gemm_nt_kernel<KIND, 256, 256, OUT, false, SB>), grid, dim3(512), 0, st, args);
    else
      hipLaunchKernelGGL((gemm_nt_kernel<KIND, 256, 256, OUT, true, SB>), grid, dim3(512), 0, st, args);
    return launch_status("gemm_nt_kernel");
  }
}

template <int KIND, int OUT, int SB>
int launch_gemm_tiles(hipStream_t st, GemmArgs args) {
  // split-K planned by the entry (plan_split, partial area in args.part), on
  // the LDS-DMA kernel (the decoder layer's down projection: 106 against
  // 115 us register-staged)
  if constexpr (KIND != KIND_I8 && SB == 128) {
    if (args.ksplit > 1) {
      args.tiles_m = args.m / 256;
      args.tiles_n = args.n / 256;
      hipLaunchKernelGGL((gemm_nt_dma4_kernel<KIND, OUT_F32, 256, 256, 128, 2, 2, true>),
                         dim3(args.tiles_m * args.tiles_n * args.ksplit), dim3(256), 0, st, args);
      WAFER_TRY(launch_status("gemm_nt_dma4_kernel"));
      const int64_t count = (int64_t)args.m * args.n;
      const unsigned grid = (unsigned)std::min<int64_t>((count / 8 + 255) / 256, 8192);
      hipLaunchKernelGGL((gemm_fold_kernel<KIND, OUT>), dim3(grid), dim3(256), 0, st, args.part, args.ksplit,
                         args.res, args.y, count);
      return launch_status("gemm_fold_kernel");
    }
  }
  // 256x256 tiles only where they divide the output and still fill the chip
  if (args.m % 256 == 0 && args.n % 256 == 0 && (args.m / 256) * (args.n / 256) >= 192) {
    args.tiles_m = args.m / 256;
    args.tiles_n = args.n / 256;
    // 16-bit operands with an even number of 128-byte K stages: 4 waves,
    // register-staged (int8 keeps 8 waves: its 4-wave dequant epilogue
    // spills; a residual keeps the 8-wave kernel's staged epilogue)
    if constexpr (KIND != KIND_I8 && OUT != OUT_NARROW_RES) {
      if (args.kbytes % 128 == 0) {
        // LDS-DMA staging (4096^3: 107 against 111 us register-staged)
        hipLaunchKernelGGL((gemm_nt_dma4_kernel<KIND, OUT, 256, 256, 128>), dim3(args.tiles_m * args.tiles_n),
                           dim3(256), 0, st, args);
        return launch_status("gemm_nt_dma4_kernel");
      }
    }
    hipLaunchKernelGGL((gemm_nt_kernel<KIND, 256, 256, OUT, false, SB>), dim3(args.tiles_m * args.tiles_n),
                       dim3(512), 0, st, args);
    return launch_status("gemm_nt_kernel");
  }
  // 128x192 tiles where they need fewer rounds of 256 workgroups for 1.5x
  // the work per tile (QKV at M = 1024: 256 tiles against 384 of 128x128)
  // (128-byte K stages only: 64-byte stages would not split 320 rows of DMA
  // evenly over 8 waves)
  const long t128 = (long)((args.m + 127) / 128) * ((args.n + 127) / 128);
  if (SB == 128 && args.m % 128 == 0 && args.n % 192 == 0) {
    const long t192 = (long)(args.m / 128) * (args.n / 192);
    if (3 * ((t192 + 255) / 256) < 2 * ((t128 + 255) / 256)) {
      args.tiles_m = args.m / 128;
      args.tiles_n = args.n / 192;
      if constexpr (SB == 128) {
        // 16-bit operands, plain outputs: the 4-wave kernel (QKV at M = 1024:
        // 53.3 against 55.4 us); a residual keeps the 8-wave kernel's staged
        // epilogue
        if constexpr (KIND != KIND_I8 && OUT != OUT_NARROW_RES) {
          if (args.kbytes % 128 == 0) {
            // LDS-DMA staging, three stages (QKV at M = 1024 in the decoder
            // layer: 52.5 against 59.4 us register-staged)
            hipLaunchKernelGGL((gemm_nt_dma4_kernel<KIND, OUT, 128, 192, 128>), dim3(args.tiles_m * args.tiles_n),
                               dim3(256), 0, st, args);
            return launch_status("gemm_nt_dma4_kernel");
          }
        }
        hipLaunchKernelGGL((gemm_nt_kernel<KIND, 128, 192, OUT, false, SB, 4, 2>),
                           dim3(args.tiles_m * args.tiles_n), dim3(512), 0, st, args);
        return launch_status("gemm_nt_kernel");
      }
    }
  }
  args.tiles_m = (args.m + 127) / 128;
  args.tiles_n = (args.n + 127) / 128;
  const dim3 grid(args.tiles_m * args.tiles_n);
  // full 16-bit tiles with plain outputs: the 4-wave LDS-DMA kernel, each
  // wave 64x64 (the decoder layer's O projection, 1024 x 4096 x 4096: 36.0
  // against 41.4 us on the 8-wave register-staged kernel)
  if constexpr (KIND != KIND_I8 && OUT != OUT_NARROW_RES && SB == 128) {
    if (args.m % 128 == 0 && args.n % 128 == 0) {
      hipLaunchKernelGGL((gemm_nt_dma4_kernel<KIND, OUT, 128, 128, 128>), grid, dim3(256), 0, st, args);
      return launch_status("gemm_nt_dma4_kernel");
    }
  }
  // ragged, int8, residual or 64-byte-stage GEMMs: 4 x 2 waves (each 32 x 64)
  // measured 2-3 % faster than 2 x 4 on 128x128 tiles
  if (args.m % 128 == 0 && args.n % 128 == 0)
    hipLaunchKernelGGL((gemm_nt_kernel<KIND, 128, 128, OUT, false, SB, 4, 2>), grid, dim3(512), 0, st, args);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<KIND, 128, 128, OUT, true, SB, 4, 2>), grid, dim3(512), 0, st, args);
  return launch_status("gemm_nt_kernel");
}

// Split-K plan for 16-bit GEMMs whose 128x128 grid is at most one round of
// workgroups and whose K is long: 256x256 tiles on the 4-wave kernel (half
// the operand bytes per FLOP of 128x128 tiles), each tile's K split over
// ksplit workgroups so that the grid still fills the CUs, plus a fold
// launch.  Returns 1 (no split) otherwise.  The decoder layer's down
// projection (1024 x 4096, K 14336, with the residual): 113.3 us + 14.2 us
// fold against 136.1 us on 128x128 tiles; 256x128 tiles with two splits
// (32 MiB of partials instead of 64) measured 138.3 + 9.3 us.
int plan_split(int m, int n, int kbytes, int cus) {
  if (m % 256 != 0 || n % 256 != 0 || kbytes < 16384) return 1;
  const long t2 = (long)(m / 256) * (n / 256), t128 = (long)(m / 128) * (n / 128);
  if (t128 > cus) return 1;
  for (int s = 4; s >= 2; --s)
    if (t2 * s <= cus && kbytes % (256 * s) == 0) return s;  // whole pairs of 128-byte stages per split
  return 1;
}

// Sets up args.ksplit / args.part for a 16-bit GEMM (growing the context's
// partial-tile area when a split is planned).
int prepare_split(wafer_hip_context *ctx, GemmArgs &args) {
  const int s = plan_split(args.m, args.n, args.kbytes, ctx->cu_count > 0 ? ctx->cu_count : 256);
  if (s < 2) return WAFER_HIP_OK;
  WAFER_TRY(ensure_workspace(ctx, &ctx->partials, &ctx->partials_bytes, (size_t)s * args.m * args.n * sizeof(float)));
  args.ksplit = s;
  args.part = (float *)ctx->partials;
  return WAFER_HIP_OK;
}

template <int KIND, int OUT>
int launch_gemm(hipStream_t st, GemmArgs args) {
  // 128-byte K stages where K allows (half the stage barriers per FLOP)
  return args.kbytes % 128 == 0 ? launch_gemm_sb<KIND, OUT, 128>(st, args) : launch_gemm_sb<KIND, OUT, 64>(st, args);
}

int relayout_rhs(wafer_hip_context *ctx, const void *rhs, uint32_t k, uint32_t n, int esize,
                 const uint8_t **bt) {
  const size_t need = (size_t)k * n * esize;
  // the transposes put K blocks of 32 or more on grid y (at most 65535)
  if ((k + 31) / 32 > 65535)
    return fail(WAFER_HIP_E_INVALID_FIELD, "gemm: k above 2097120 with a [K,N] rhs; pass the [N,K] form");
  WAFER_TRY(ensure_workspace(ctx, &ctx->relayout, &ctx->relayout_bytes, need));
  // check_shape guarantees k a multiple of 64 (int8) or 32 (16-bit); the
  // tiled kernels need n a multiple of their 128 / 64 columns and (int8) k a
  // multiple of 128
  const bool tiled = esize == 1 ? (n % 128 == 0 && k % 128 == 0) : n % 64 == 0;
  if (!tiled) {
    const dim3 grid((n + 31) / 32, (k + 31) / 32);
    if (esize == 1)
      hipLaunchKernelGGL(transpose_any_kernel<uint8_t>, grid, dim3(256), 0, ctx->stream, (const uint8_t *)rhs,
                         (uint8_t *)ctx->relayout, (int)k, (int)n);
    else
      hipLaunchKernelGGL(transpose_any_kernel<uint16_t>, grid, dim3(256), 0, ctx->stream, (const uint16_t *)rhs,
                         (uint16_t *)ctx->relayout, (int)k, (int)n);
  } else if (esize == 1) {
    const long tiles = (long)(k / 128) * (n / 128);  // one wave each
    hipLaunchKernelGGL(transpose_i8_reg_kernel, dim3((unsigned)std::min<long>((tiles + 3) / 4, 65536)), dim3(256),
                       0, ctx->stream, (const uint8_t *)rhs, (uint8_t *)ctx->relayout, (int)k, (int)n);
  }
  else
    hipLaunchKernelGGL(transpose_b16_kernel, dim3(n / 64, k / 32), dim3(128), 0, ctx->stream,
                       (const uint16_t *)rhs, (uint16_t *)ctx->relayout, (int)k, (int)n);
  WAFER_TRY(launch_status("transpose kernel"));
  *bt = (const uint8_t *)ctx->relayout;
  return WAFER_HIP_OK;
}

int check_shape(uint32_t m, uint32_t k, uint32_t n, int esize, const char *what) {
  if (m == 0 || k == 0 || n == 0) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(what) + ": empty dimension");
  if (((uint64_t)k * esize) % BKB)
    return fail(WAFER_HIP_E_UNSUPPORTED, std::string(what) + ": needs k*elem_bytes a multiple of 64");
  // m, n are kernel ints; the grid is one dimension of 128x128 tiles
  if (m > 0x7fffffffu || n > 0x7fffffffu || (uint64_t)((m + 127) / 128) * ((n + 127) / 128) > 0x7fffffffull)
    return fail(WAFER_HIP_E_INVALID_FIELD, std::string(what) + ": output too large");
  // in-tile offsets (row * k * esize over 256 rows) are 32-bit
  if ((uint64_t)m * k * esize > 0x7fffffffffull || (uint64_t)k * esize >= (1u << 24))
    return fail(WAFER_HIP_E_INVALID_FIELD, std::string(what) + ": operand too large (k * element bytes must be below 16 MiB)");
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
  GemmArgs args{(const uint8_t *)lhs, bt, dst, nullptr, nullptr, (int)m, (int)n, (int)(k * 2), 0, 0};
  WAFER_TRY(prepare_split(ctx, args));
  const bool f32 = out_format == WAFER_FMT_F32;
  if (in_format == WAFER_FMT_BF16)
    return f32 ? launch_gemm<KIND_BF16, OUT_F32>(ctx->stream, args)
               : launch_gemm<KIND_BF16, OUT_NARROW>(ctx->stream, args);
  return f32 ? launch_gemm<KIND_F16, OUT_F32>(ctx->stream, args)
             : launch_gemm<KIND_F16, OUT_NARROW>(ctx->stream, args);
}

extern "C" int wafer_hip_gemm_mfma_residual(wafer_hip_context *ctx, const void *lhs, const void *rhs,
                                            const void *residual, void *dst, uint32_t m, uint32_t k, uint32_t n,
                                            uint32_t in_format, uint32_t rhs_orientation) {
  WAFER_CHECK_CTX(ctx);
  if (in_format != WAFER_FMT_BF16 && in_format != WAFER_FMT_F16)
    return fail(WAFER_HIP_E_UNSUPPORTED, "gemm_mfma_residual: input format must be BF16 or F16");
  if (rhs_orientation > 1) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_mfma_residual: bad orientation");
  if (!lhs || !rhs || !residual || !dst) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_mfma_residual: null tensor");
  WAFER_TRY(check_shape(m, k, n, 2, "gemm_mfma_residual"));
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const uint8_t *bt = (const uint8_t *)rhs;
  if (rhs_orientation == WAFER_GEMM_NORMAL) WAFER_TRY(relayout_rhs(ctx, rhs, k, n, 2, &bt));
  GemmArgs args{(const uint8_t *)lhs, bt, dst, nullptr, nullptr, (int)m, (int)n, (int)(k * 2), 0, 0,
                (const uint16_t *)residual};
  WAFER_TRY(prepare_split(ctx, args));
  return in_format == WAFER_FMT_BF16 ? launch_gemm<KIND_BF16, OUT_NARROW_RES>(ctx->stream, args)
                                     : launch_gemm<KIND_F16, OUT_NARROW_RES>(ctx->stream, args);
}

extern "C" int wafer_hip_gemm_mfma_swiglu(wafer_hip_context *ctx, const void *lhs, const void *rhs_gu,
                                          void *dst, uint32_t m, uint32_t k, uint32_t features,
                                          uint32_t in_format) {
  WAFER_CHECK_CTX(ctx);
  if (in_format != WAFER_FMT_BF16 && in_format != WAFER_FMT_F16)
    return fail(WAFER_HIP_E_UNSUPPORTED, "gemm_mfma_swiglu: input format must be BF16 or F16");
  if (!lhs || !rhs_gu || !dst) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_mfma_swiglu: null tensor");
  if (features == 0 || features % 16)
    return fail(WAFER_HIP_E_UNSUPPORTED, "gemm_mfma_swiglu: features must be a positive multiple of 16");
  if (features > 0x3fffffffu) return fail(WAFER_HIP_E_INVALID_FIELD, "gemm_mfma_swiglu: output too large");
  WAFER_TRY(check_shape(m, k, 2 * features, 2, "gemm_mfma_swiglu"));
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  GemmArgs args{(const uint8_t *)lhs, (const uint8_t *)rhs_gu, dst, nullptr, nullptr, (int)m,
                (int)(2 * features), (int)(k * 2), 0, 0};
  return in_format == WAFER_FMT_BF16 ? launch_gemm<KIND_BF16, OUT_SWIGLU>(ctx->stream, args)
                                     : launch_gemm<KIND_F16, OUT_SWIGLU>(ctx->stream, args);
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
  // a [K, N] rhs on whole 256x256 tiles that fill the chip: read in place
  // (K * N below 2^31: the kernel's buffer offsets are 32-bit)
  if (rhs_orientation == WAFER_GEMM_NORMAL && m % 256 == 0 && n % 256 == 0 && k % 128 == 0 &&
      (m / 256) * (n / 256) >= 192 && (uint64_t)k * n < (1ull << 31)) {
    GemmArgs args{(const uint8_t *)a, bt, y, acc_out, scale, (int)m, (int)n, (int)k, 0, 0};
    args.tiles_m = (int)(m / 256);
    args.tiles_n = (int)(n / 256);
    hipLaunchKernelGGL((gemm_nt_kernel<KIND_I8, 256, 256, OUT_I8_DEQUANT, false, 128, 2, 4, true>),
                       dim3(args.tiles_m * args.tiles_n), dim3(512), 0, ctx->stream, args);
    return launch_status("gemm_nt_kernel");
  }
  if (rhs_orientation == WAFER_GEMM_NORMAL) WAFER_TRY(relayout_rhs(ctx, b, k, n, 1, &bt));
  GemmArgs args{(const uint8_t *)a, bt, y, acc_out, scale, (int)m, (int)n, (int)k, 0, 0};
  return launch_gemm<KIND_I8, OUT_I8_DEQUANT>(ctx->stream, args);
}
