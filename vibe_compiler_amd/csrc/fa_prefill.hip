// fa_prefill.hip -- FA flash-attention prefill for gfx950.
//
// Semantics: the compiler's online-attention decomposition
// (lib/Wafer/Transforms/Linalg/OnlineAttentionDecomposition.cpp:568-597; QK
// :242-277, score region :279-426, PV :509-566; finalize
// lib/Wafer/Transforms/Linalg/OnlineAttentionMaterialization.cpp:197-262):
//   per KV block: S = q.k (f32 accumulate), S = S*scale (+0/-inf causal bias),
//   m' = max(m, rowmax S), alpha = ExpLp(m - m'), P = ExpLp(S - m'),
//   l = l*alpha + rowsum(P) (unrounded P), acc = acc*alpha + T(P).V,
//   out = T(acc * (1/l)), 0 for a row with l == 0; T the storage format
//   (bf16 or f16, both RNE).
// The two partial states of interleaved key sets combine with the state
// merge of OnlineAttentionMaterialization.cpp:264-373: m = max(mL, mR),
// sL = ExpLp(mL - m), sR = ExpLp(mR - m), l = lL sL + lR sR,
// acc = accL sL + accR sR.
//
// Mapping onto CDNA4:
//  * a workgroup (8 waves) serves two 64-query blocks of one (batch, head),
//    block n-1-i (late) and block i (early) of the causal triangle, side by
//    side: every workgroup does the same amount of work (n-i + i+1 key
//    blocks) and one launch of heads*ceil(n/2) workgroups fills the CUs
//    evenly with no cross-workgroup merge (an odd n leaves the middle block
//    alone in its workgroup).  Partial last blocks: padding queries load a
//    clamped row and are not stored; keys past kv_len read as zero (each
//    block's buffer resource is sized to its rows) and are masked;
//  * both blocks read the same two-block stages (their key ranges start at
//    0; the early block's is a prefix of the late one's).  Waves 0-3 take
//    the late block: query tile w & 1 (32 queries) and key half w >> 1 (the
//    even or the odd 64-key blocks); the two halves of a tile merge through
//    LDS at the end.  Waves 4-7 take the early block: 16 queries each over
//    every key block (both blocks of each stage), so they need no merge.
//    Waves w and w + 4 share a SIMD, so each SIMD carries one wave of each
//    block and all SIMDs do the same work;
//  * scores are computed transposed, S^T = K . Q^T (A = keys x d from LDS,
//    B = Q^T kept in VGPRs): the late waves on v_mfma_f32_32x32x16 (each
//    lane holds 32 scores of one query, the 2 lanes of a query combine with
//    a permlane32 swap; every K and V fragment read feeds 32 queries), the
//    early waves on v_mfma_f32_16x16x32 (16 scores per lane, the 4 lanes of
//    a query combine with permlane16/permlane32 swaps);
//  * the output is accumulated transposed as well, O^T = V^T . P^T: P^T feeds
//    the MFMA B operand straight from the score registers after RNE narrowing
//    (v_cvt_pk_{bf16,f16}_f32), and the V^T operand comes from row-major V in LDS
//    through the transposing read ds_read_b64_tr_b16 (within each 16-lane
//    group, lane i receives element i%4 of the 4-element vectors at the
//    addresses of lanes 4e + i/4, e = 0..3);
//  * K and V blocks move global -> LDS by buffer_load ... lds (no staging
//    registers): two stages, the next blocks' DMA overlapping the current
//    blocks' compute.  Rows are 256 bytes (one line of the 64 LDS banks)
//    with 16-byte chunks XOR-swizzled: K by row & 15, so the 16 rows one
//    LDS pass of a ds_read_b128 fragment read serves hit 16 distinct bank
//    groups (measured: no conflicts on K), V by 2 (row & 7) for the
//    transposed ds_read_b64_tr_b16 reads;
//  * lazy rescale: the exponentials are taken against a per-query reference
//    max that moves only when a score exceeds it by more than 2^8 in the
//    log2 domain; the common path computes no block max at all (a lane sum
//    of P above 2^8 detects every such block);
//  * consecutive workgroup ids walk (batch*head), so each head's workgroups
//    land on one XCD (ids are dealt round-robin over the 8 XCDs) and share
//    its L2.
//
// Arithmetic note: ExpLp(S*scale - m) is evaluated as
// exp2(fma(s_raw, scale*log2e, -m_ref*scale*log2e)) (one rounding fewer than
// the reference's mul, sub, mul chain); the difference is below 1 ulp of the
// f32 argument and far inside the attention tolerance.  With the lazy
// reference P <= 2^8 and its rounding point in T differs from the
// reference's, with the same relative bound (2^8 is far inside f16's range).
#include "common.h"

#include <type_traits>

namespace wafer {
namespace {

constexpr int D = 128;
constexpr int QB = 64;            // queries per query block
constexpr int BK = 64;            // keys per KV block
constexpr int THREADS = 512;

// Lazy rescaling: the exponentials use a reference max that moves only when
// some query's max exceeds it by more than 2^RESCALE_LOG2 (P <= 2^8).
constexpr float RESCALE_LOG2 = 8.0f;
constexpr float RESCALE_BOUND = 256.0f;  // 2^RESCALE_LOG2
// __builtin_amdgcn_sched_group_barrier instruction classes
constexpr int SG_MFMA = 0x008, SG_VMEM = 0x010, SG_DS_READ = 0x100;
// "no reference yet": the lowest finite float, so exp2(fma(s, c, -NOREF)) is
// +inf (or at least 1) for a visible score and 0 for a masked one (never
// NaN), exp2(NOREF - x) == 0 for x above NOREF + 150, and any visible score,
// however negative, becomes a valid reference
constexpr float NOREF = -0x1.fffffep127f;

// x combined with the value of lane ^ 32 (v_permlane32_swap exchanges the
// upper half of one register with the lower half of the other)
__device__ inline float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ inline float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 16x16x32 MFMA on 8-element fragments of the storage type T
template <typename T>
__device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (std::is_same_v<T, __bf16>)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}
// output narrowing: bf16 by the reference's codec (canonical NaN 0x7fc0);
// f16 by v_cvt_f16_f32 (RNE, gradual underflow, overflow to inf), a NaN to
// the canonical 0x7e00
template <typename T>
__device__ inline uint32_t narrow_pair(float lo, float hi) {
  if constexpr (std::is_same_v<T, __bf16>) {
    return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
  } else {
    lo = f32_rounded(lo);
    hi = f32_rounded(hi);
    const uint32_t l = lo != lo ? 0x7e00u : __builtin_bit_cast(uint16_t, (_Float16)lo);
    const uint32_t h = hi != hi ? 0x7e00u : __builtin_bit_cast(uint16_t, (_Float16)hi);
    return l | (h << 16);
  }
}

// Element strides (batch, head, row) of Q, K, V and O for the STRIDED
// instantiation; the other reads the dense [B, H, S, 128] layout.
struct FaStrides {
  int64_t q[3], k[3], v[3], o[3];
};

// 32x32x16 MFMA on 8-element fragments of the storage type T
template <typename T>
__device__ inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (std::is_same_v<T, __bf16>)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

template <typename T, bool CAUSAL, bool STRIDED = false>
__global__ __launch_bounds__(THREADS) void fa_prefill_d128(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K,
    const uint16_t *__restrict__ V, uint16_t *__restrict__ O, int q_heads, int kv_heads,
    int q_len, int kv_len, float c, int bh_count, int n_qblocks, const FaStrides st = FaStrides{}) {
  // two stages of [K block 2t | K block 2t+1 | V block 2t | V block 2t+1],
  // 16 KiB each: rows of 256 bytes (64 keys x 128 d), 16-byte chunk ch of
  // row r stored at chunk position ch ^ 2 (r & 7)
  __shared__ __align__(1024) uint16_t sbuf[2][4][BK * D];

  const int bid = blockIdx.x;
  const int pair = bid / bh_count;
  const int bh = bid - pair * bh_count;
  const int b = bh / q_heads;
  const int h = bh - b * q_heads;
  const int kvh = h / (q_heads / kv_heads);
  const uint16_t *Qp = STRIDED ? Q + b * st.q[0] + h * st.q[1] : Q + ((size_t)bh * q_len) * D;
  const uint16_t *Kp = STRIDED ? K + b * st.k[0] + kvh * st.k[1] : K + ((size_t)(b * kv_heads + kvh) * kv_len) * D;
  const uint16_t *Vp = STRIDED ? V + b * st.v[0] + kvh * st.v[1] : V + ((size_t)(b * kv_heads + kvh) * kv_len) * D;
  uint16_t *Op = STRIDED ? O + b * st.o[0] + h * st.o[1] : O + ((size_t)bh * q_len) * D;
  // row strides in elements (D in the dense layout)
  const int64_t q_rs = STRIDED ? st.q[2] : D, k_rs = STRIDED ? st.k[2] : D, v_rs = STRIDED ? st.v[2] : D;
  const int64_t o_rs = STRIDED ? st.o[2] : D;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the late query block n-1-pair (waves 0-3) and the early block `pair`
  // (waves 4-7; none when they coincide: the middle block of an odd count)
  // run side by side.  The last query block and the last key block may be
  // partial.
  const int qb_a = n_qblocks - 1 - pair;
  const int qb_b = pair;
  const int kv_blocks = (kv_len + BK - 1) / BK;
  const int nk_a = CAUSAL ? min(kv_blocks, qb_a + 1) : kv_blocks;
  const int nk_b = qb_b < qb_a ? (CAUSAL ? min(kv_blocks, qb_b + 1) : kv_blocks) : 0;
  const int niter = (nk_a + 1) / 2;  // iteration t works on key blocks 2t and 2t + 1
  const int nite = (nk_b + 1) / 2;   // iterations in which the early block has keys

  // global -> LDS by buffer_load ... lds: wave w moves rows
  // 16 (w >> 1) + 4 j + lane / 16 (j = 0..3) of the K and V blocks of key
  // half w & 1 (block 2t + (w & 1)), 4 + 4 instructions of 1 KiB per wave
  // and iteration.  Lane l writes chunk position l % 16, so it loads global
  // chunk (l % 16) ^ swz(row): for K swz(row) = row & 15 = 4 j + (l >> 4),
  // which keeps the K fragment reads (ds_read_b128, 16 rows per LDS pass)
  // free of bank conflicts; for V swz(row) = 2 (row & 7) = 8 (j & 1) +
  // 2 (l >> 4), for the transposed reads (ds_read_b64_tr_b16).  One buffer resource
  // per block, based at the block and sized to its rows (the hardware range
  // check covers the lane offset, not the scalar one), so rows of a partial
  // last block past kv_len read as zero.
  const int dq = wave >> 1, dh = wave & 1;
  auto block_rsrc = [&](const uint16_t *base, int64_t rs, int kb) __attribute__((always_inline)) {
    const int rows = min(BK, kv_len - kb * BK);
    return __builtin_amdgcn_make_buffer_rsrc((void *)(base + (size_t)kb * BK * rs), 0,
                                             (int)(((int64_t)(rows - 1) * rs + D) * 2), 0x00020000);
  };
  uint32_t dma_off_k[4], dma_off_v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 16 * dq + 4 * j + (lane >> 4);
    const uint32_t chunk_k = (uint32_t)(((lane & 15) ^ (4 * j + (lane >> 4))) << 4);  // row & 15
    const uint32_t chunk_v = (uint32_t)(((lane & 15) ^ (8 * (j & 1) + 2 * (lane >> 4))) << 4);  // 2 (row & 7)
    dma_off_k[j] = (uint32_t)(row * k_rs * 2) + chunk_k;
    dma_off_v[j] = (uint32_t)(row * v_rs * 2) + chunk_v;
  }
  // this wave's share of iteration t's blocks (t clamped to the last
  // iteration, the block to the late block's last: loads past the end are
  // harmless)
  auto dma_k = [&](int t, int buf) __attribute__((always_inline)) {
    const int kb = min(2 * min(t, niter - 1) + dh, nk_a - 1);
    const __amdgpu_buffer_rsrc_t rsrc = block_rsrc(Kp, k_rs, __builtin_amdgcn_readfirstlane(kb));
    uint16_t *dk = sbuf[buf][dh] + dq * 4 * 512;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(dk + j * 512), 16,
                                               dma_off_k[j], 0, 0, 0);
  };
  auto dma_v = [&](int t, int buf) __attribute__((always_inline)) {
    const int kb = min(2 * min(t, niter - 1) + dh, nk_a - 1);
    const __amdgpu_buffer_rsrc_t rsrc = block_rsrc(Vp, v_rs, __builtin_amdgcn_readfirstlane(kb));
    uint16_t *dv = sbuf[buf][2 + dh] + dq * 4 * 512;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(dv + j * 512), 16,
                                               dma_off_v[j], 0, 0, 0);
  };
  auto lds_barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // LDS only: stores stay in flight
  };

  // Iteration t computes from stage t % 2 while every wave moves its share
  // of iteration t+1's blocks into stage (t+1) % 2 (read last in iteration
  // t-1, before the barrier that ended it), then waits for its own moves and
  // meets the other waves at one barrier.  Both roles run the same loop and
  // the same barriers.
  auto run = [&](auto &&body) __attribute__((always_inline)) {
    dma_k(0, 0);
    dma_v(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // Q and the first blocks
    __syncthreads();
    auto step = [&](int t, auto slot) __attribute__((always_inline)) {
      constexpr int P = decltype(slot)::value;  // == t % 2
      // the next blocks' moves (after the last iteration a clamped, unused
      // block: unconditional, so they can sit between the MFMAs)
      auto kdma = [&]() __attribute__((always_inline)) { dma_k(t + 1, P ^ 1); };
      auto vdma = [&]() __attribute__((always_inline)) { dma_v(t + 1, P ^ 1); };
      body(t, slot, kdma, vdma);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    };
    for (int t = 0; t < niter; t += 2) {
      step(t, std::integral_constant<int, 0>{});
      if (t + 1 < niter) step(t + 1, std::integral_constant<int, 1>{});
    }
  };

  if (wave < 4) {
    // ---- late block: wave w takes queries 32 (w & 1) + [0,32) and the key
    // blocks of half w >> 1; the halves merge at the end.
    // S^T = K.Q^T on v_mfma_f32_32x32x16 (A = 32 keys x 16 d from LDS,
    // B = Q^T in VGPRs): each lane holds 32 scores of query l32 (keys
    // 32 kt + 8 (r / 4) + 4 g2 + r % 4 of tile kt, register r), the
    // other 32 sit in lane ^ 32.  O^T = V^T.P^T: P^T straight from the
    // score registers (k-step ks = 2 kt + kk takes registers 8 kk .. 8 kk + 7
    // of tile kt), V^T through ds_read_b64_tr_b16 in the same key order.
    // Every K and V fragment feeds 32 queries.
    const int lt = wave & 1, hh = wave >> 1;
    const int l32 = lane & 31, g2 = lane >> 5;
    const int q0 = qb_a * QB + 32 * lt;
    // Q^T as the B operand: query l32, d = 16 s + 8 g2 + [0,8) (rows past
    // q_len load the last row and are never stored)
    u32x4 qr[8];
    {
      const int row = min(q0 + l32, q_len - 1);
#pragma unroll
      for (int s = 0; s < 8; ++s) qr[s] = *(const u32x4 *)(Qp + (size_t)row * q_rs + s * 16 + g2 * 8);
    }
    // LDS byte offsets within a 16 KiB block:
    //  K (d-step s, key tile kt): row 32 kt + l32, chunk 2 s + g2,
    //    swz = l32 & 15  ->  ko[s] + kt * 8192
    //  V^T (d tile dt, k-step ks, half hi): in 16-lane group q16 = lane / 16
    //    lane i reads row 16 ks + 8 hi + 4 g2 + i / 4, d 32 dt + 16 (q16 % 2)
    //    + 4 (i % 4) and receives d 32 dt + l32 at keys 16 ks + 8 hi + 4 g2
    //    + [0,4)  ->  vo[dt] + (16 ks + 8 hi) * 256
    uint32_t ko[8], vo[4];
#pragma unroll
    for (int s = 0; s < 8; ++s) ko[s] = (uint32_t)(l32 * 256 + (((2 * s + g2) ^ (l32 & 15)) << 4));
    {
      const int q16 = lane >> 4, i16 = lane & 15;
      const int vrow = 4 * g2 + (i16 >> 2);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        vo[dt] = (uint32_t)(vrow * 256 + (((4 * dt + 2 * (q16 & 1) + ((i16 >> 1) & 1)) ^ (2 * (vrow & 7))) << 4) +
                            8 * (i16 & 1));
    }
    float mref = NOREF;  // scaled reference max of query l32 (shared with lane ^ 32)
    float lsum = 0.0f;   // this lane's partial sum of P
    f32x16 oacc[4];      // O^T d tile dt: d 32 dt + 8 (r / 4) + 4 g2 + r % 4, query l32
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.0f;

    auto compute = [&](int kb, const char *sk, const char *sv, auto &&kdma, auto &&vdma)
                       __attribute__((always_inline)) {
      f32x16 sc[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[kt][r] = 0.0f;
      // K fragments two d-steps ahead of their MFMAs; then the V fragments
      // of k-steps 0 and 1, which land during the softmax
      u32x4 kf[8][2];
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) kf[s][kt] = *(const u32x4 *)(sk + ko[s] + kt * 8192);
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) sc[kt] = mfma32<T>(kf[s][kt], qr[s], sc[kt]);
      u32x4 vf[4][4];
      auto read_v = [&](int ks) __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(sv + vo[dt] + (16 * ks) * 256));
          const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(sv + vo[dt] + (16 * ks + 8) * 256));
          vf[ks][dt] = __builtin_bit_cast(u32x4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      };
      read_v(0);
      read_v(1);
      kdma();
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 4, 0);
#pragma unroll
      for (int s = 0; s < 6; ++s) {
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 4, 0);
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 16, 0);
      __builtin_amdgcn_sched_group_barrier(SG_VMEM, 4, 0);
      // key kb*BK + 32 kt + 8 (r / 4) + 4 g2 + r % 4 is visible to query
      // q0 + l32 iff it is below kv_len and (causal) not past the query
      if ((CAUSAL && kb * BK + BK - 1 > q0) || kb * BK + BK > kv_len) {
        const int lim = CAUSAL ? min(q0 + l32, kv_len - 1) : kv_len - 1;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (kb * BK + 32 * kt + 8 * (r >> 2) + 4 * g2 + (r & 3) > lim) sc[kt][r] = -__builtin_inff();
      }
      f32x16 p[2];
      float rsum;
      auto expo = [&]() __attribute__((always_inline)) {
        float rs[8];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              p[kt][4 * r4 + j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][4 * r4 + j], c, -mref));
            rs[4 * kt + r4] = (p[kt][4 * r4] + p[kt][4 * r4 + 1]) + (p[kt][4 * r4 + 2] + p[kt][4 * r4 + 3]);
          }
        rsum = ((rs[0] + rs[1]) + (rs[2] + rs[3])) + ((rs[4] + rs[5]) + (rs[6] + rs[7]));
      };
      expo();
      if (__builtin_expect(__any(rsum > RESCALE_BOUND), 0)) {
        float mx = -__builtin_inff();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[kt][r]);
        mx = xor32_max(mx);
        const float mc_new = mx * c;
        if (mx != -__builtin_inff() && mc_new > mref + RESCALE_LOG2) {
          const float alpha = __builtin_amdgcn_exp2f(mref - mc_new);  // 0 from NOREF
          lsum *= alpha;
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
          mref = mc_new;
        }
        expo();
      }
      lsum += rsum;
      typedef T t8 __attribute__((ext_vector_type(8)));
      u32x4 pb[4];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          t8 x;
#pragma unroll
          for (int j = 0; j < 8; ++j) x[j] = (T)p[kt][8 * kk + j];
          pb[2 * kt + kk] = __builtin_bit_cast(u32x4, x);
        }
      // V fragments of k-steps 2 and 3 while those of 0 and 1 feed the MFMAs
      read_v(2);
      read_v(3);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) oacc[dt] = mfma32<T>(vf[ks][dt], pb[ks], oacc[dt]);
      vdma();
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 8, 1);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 4, 1);
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 8, 1);
      __builtin_amdgcn_sched_group_barrier(SG_VMEM, 1, 1);
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 4, 1);
        __builtin_amdgcn_sched_group_barrier(SG_VMEM, 1, 1);
      }
    };

    run([&](int t, auto slot, auto &&kdma, auto &&vdma) __attribute__((always_inline)) {
      constexpr int P = decltype(slot)::value;
      const int kb = 2 * t + hh;
      if (kb < nk_a) {
        compute(kb, (const char *)sbuf[P][hh], (const char *)sbuf[P][2 + hh], kdma, vdma);
      } else {
        asm volatile("" ::: "memory");  // keeps the moves from being hoisted out of compute
        kdma();
        vdma();
      }
    });

    // The two key halves of a query tile merge by a reduce-scatter through
    // LDS (free after the loop's last barrier): half H keeps d tiles 2 H and
    // 2 H + 1, hands the other two to its partner, merges the partner's two
    // into its own, normalises and writes them.  Exchange layout: 16-byte
    // vectors [lt][writer half][tile][r / 4][lane], then the (reference max,
    // lane sum) pairs.  Each state is (acc, l) relative to its scaled
    // reference max; a state that saw no visible key (NOREF) has l == 0 and
    // acc == 0 (state merge of OnlineAttentionMaterialization.cpp:264-373,
    // finalize :197-262).
    auto merge_h = [&](auto half_c) __attribute__((always_inline)) {
      constexpr int H = decltype(half_c)::value;  // == hh, so every tile index is static
      f32x4 *xacc = (f32x4 *)&sbuf[0][0][0];      // 32 KiB
      float *xml = (float *)(xacc + 2 * 2 * 2 * 4 * 64);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x16 &a = oacc[2 * (1 - H) + i];
          xacc[(((lt * 2 + H) * 2 + i) * 4 + rq) * 64 + lane] =
              f32x4{a[4 * rq], a[4 * rq + 1], a[4 * rq + 2], a[4 * rq + 3]};
        }
      xml[((lt * 2 + H) * 2 + 0) * 64 + lane] = mref;
      xml[((lt * 2 + H) * 2 + 1) * 64 + lane] = lsum;
      lds_barrier();
      const float m1 = xml[((lt * 2 + (1 - H)) * 2 + 0) * 64 + lane];
      const float l1 = xml[((lt * 2 + (1 - H)) * 2 + 1) * 64 + lane];
      const float e = fmaxf(mref, m1);
      const float s0 = __builtin_amdgcn_exp2f(mref - e);
      const float s1 = __builtin_amdgcn_exp2f(m1 - e);
      const float l = xor32_sum(lsum * s0 + l1 * s1);
      // finalize: coefficient = Recip(l) (0 for an empty row), out = T(acc * coef)
      const float coef = (l == 0.0f) ? 0.0f : 1.0f / l;
      uint16_t *orow = Op + (int64_t)(q0 + l32) * o_rs + 4 * g2;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int dt = 2 * H + i;
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 o = xacc[(((lt * 2 + (1 - H)) * 2 + i) * 4 + rq) * 64 + lane];
          f32x4 r;
#pragma unroll
          for (int j = 0; j < 4; ++j) r[j] = (oacc[dt][4 * rq + j] * s0 + o[j] * s1) * coef;
          u32x2 packed;
          packed[0] = narrow_pair<T>(r[0], r[1]);
          packed[1] = narrow_pair<T>(r[2], r[3]);
          if (q0 + l32 < q_len) *(u32x2 *)(orow + dt * 32 + rq * 8) = packed;
        }
      }
      // a distinct marker per half: keeps the two copies from being merged
      // into one tail that would index oacc at run time (and spill it)
      asm volatile("; fa merge tail %0" ::"n"(H));
    };
    if (hh == 0)  // wave-uniform
      merge_h(std::integral_constant<int, 0>{});
    else
      merge_h(std::integral_constant<int, 1>{});
  } else {
    // ---- early block: wave 4 + e takes queries 16 e + [0,16) over every
    // key block (both blocks of each stage), so it needs no merge.
    // S^T = K.Q^T on v_mfma_f32_16x16x32 (A = 16 keys x 32 d from LDS,
    // B = Q^T in VGPRs): each lane holds 16 scores of query l16, the 4 lanes
    // of a query combine with permlane16/permlane32 swaps.  O^T = V^T.P^T
    // with P^T from the score registers and V^T through ds_read_b64_tr_b16
    // (within each 16-lane group, lane i receives element i%4 of the
    // 4-element vectors at the addresses of lanes 4e + i/4, e = 0..3).
    const int l16 = lane & 15, g = lane >> 4;
    const int q0 = qb_b * QB + (wave - 4) * 16;
    // Q^T as the MFMA B operand: lane holds query l16, d = 32 s + 8 g + [0,8)
    u32x4 qreg[4];
    {
      const int row = min(q0 + l16, q_len - 1);
#pragma unroll
      for (int s = 0; s < 4; ++s) qreg[s] = *(const u32x4 *)(Qp + (size_t)row * q_rs + s * 32 + g * 8);
    }
    // LDS read offsets (bytes within a 16 KiB block), per lane:
    //  K (A operand, k-step s, key tile kt): row kt*16 + l16, chunk 4 s + g,
    //    swz = l16  ->  k_off[s] + kt * 4096
    //  V^T (A operand via ds_read_b64_tr_b16, k-step s, key half hx, d tile
    //    dt): lane reads row 32 s + 16 hx + 4 g + l16/4, d 16 dt + 4 (l16 % 4)
    //    (chunk 2 dt + (l16/2) % 2, byte 8 (l16 % 2));
    //    swz = 8 (g % 2) + 2 (l16 / 4)  ->  v_off[dt] + (32 s + 16 hx) * 256
    uint32_t k_off[4], v_off[8];
#pragma unroll
    for (int s = 0; s < 4; ++s) k_off[s] = (uint32_t)(l16 * 256 + (((4 * s + g) ^ l16) << 4));
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      v_off[dt] = (uint32_t)((4 * g + (l16 >> 2)) * 256 +
                             (((2 * dt + ((l16 >> 1) & 1)) ^ (8 * (g & 1) + 2 * (l16 >> 2))) << 4) + 8 * (l16 & 1));
    float mc_ref = NOREF;  // scaled reference max of query l16 (shared by its 4 lanes)
    float l_part = 0.0f;   // this lane's partial sum of P
    f32x4 acc_o[8];        // O^T rows dt*16 + 4 g + [0,4), column query l16
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc_o[dt][j] = 0.0f;

    auto compute = [&](int kb, const char *sk, const char *sv, auto &&kdma, auto &&vdma)
                       __attribute__((always_inline)) {
      f32x4 sacc[4];  // S^T rows kt*16 + 4 g + [0,4)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j) sacc[kt][j] = 0.0f;
      u32x4 kf[4][4], vf[2][8];
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) kf[s][kt] = *(const u32x4 *)(sk + k_off[s] + kt * 4096);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) sacc[kt] = mfma16<T>(kf[s][kt], qreg[s], sacc[kt]);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(sv + v_off[dt] + (32 * s) * 256));
          const v4i16 hi =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(sv + v_off[dt] + (32 * s + 16) * 256));
          vf[s][dt] = __builtin_bit_cast(u32x4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      kdma();
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 16, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 16, 0);
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 32, 0);
      __builtin_amdgcn_sched_group_barrier(SG_VMEM, 4, 0);
      // key kb*BK + kt*16 + 4 g + j is visible to query q0 + l16 iff it is
      // below kv_len and (causal) not past the query
      if ((CAUSAL && kb * BK + BK - 1 > q0) || kb * BK + BK > kv_len) {
        const int lim = CAUSAL ? min(q0 + l16, kv_len - 1) : kv_len - 1;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (kb * BK + kt * 16 + 4 * g + j > lim) sacc[kt][j] = -__builtin_inff();
      }
      f32x4 p[4];
      float rs[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) p[kt][j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][j], c, -mc_ref));
        rs[kt] = (p[kt][0] + p[kt][1]) + (p[kt][2] + p[kt][3]);
      }
      float rsum = (rs[0] + rs[1]) + (rs[2] + rs[3]);
      if (__builtin_expect(__any(rsum > RESCALE_BOUND), 0)) {
        float mx = -__builtin_inff();
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          mx = fmaxf(mx, fmaxf(fmaxf(sacc[kt][0], sacc[kt][1]), fmaxf(sacc[kt][2], sacc[kt][3])));
        mx = xor16_max(xor32_max(mx));
        const float mc_new = mx * c;
        if (mx != -__builtin_inff() && mc_new > mc_ref + RESCALE_LOG2) {
          const float alpha = __builtin_amdgcn_exp2f(mc_ref - mc_new);  // 0 from NOREF
          l_part *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc_o[dt][j] *= alpha;
          mc_ref = mc_new;
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
          for (int j = 0; j < 4; ++j) p[kt][j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][j], c, -mc_ref));
          rs[kt] = (p[kt][0] + p[kt][1]) + (p[kt][2] + p[kt][3]);
        }
        rsum = (rs[0] + rs[1]) + (rs[2] + rs[3]);
      }
      l_part += rsum;
      // P^T operand of k-step s: slots 8 g + [0,4) are keys 32 s + 4 g + [0,4)
      // (tile 2 s), slots 8 g + [4,8) keys 32 s + 16 + 4 g + [0,4) (tile 2 s + 1)
      typedef T t8 __attribute__((ext_vector_type(8)));
      u32x4 pb[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        t8 x;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = (T)p[2 * s][j];
          x[4 + j] = (T)p[2 * s + 1][j];
        }
        pb[s] = __builtin_bit_cast(u32x4, x);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc_o[dt] = mfma16<T>(vf[s][dt], pb[s], acc_o[dt]);
      vdma();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 4, 1);
        __builtin_amdgcn_sched_group_barrier(SG_VMEM, 1, 1);
      }
    };
    auto nop = [&]() __attribute__((always_inline)) {};

    run([&](int t, auto slot, auto &&kdma, auto &&vdma) __attribute__((always_inline)) {
      constexpr int P = decltype(slot)::value;
      if (t < nite) {
        compute(2 * t, (const char *)sbuf[P][0], (const char *)sbuf[P][2], kdma, vdma);
        if (2 * t + 1 < nk_b) compute(2 * t + 1, (const char *)sbuf[P][1], (const char *)sbuf[P][3], nop, nop);
        if (t == nite - 1) {
          // finalize: coefficient = Recip(l) (0 for an empty row), out = T(acc * coef)
          const float l = xor16_sum(xor32_sum(l_part));
          const float coef = (l == 0.0f) ? 0.0f : 1.0f / l;
          uint16_t *orow = Op + (int64_t)(q0 + l16) * o_rs + 4 * g;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) {
            u32x2 packed;
            packed[0] = narrow_pair<T>(acc_o[dt][0] * coef, acc_o[dt][1] * coef);
            packed[1] = narrow_pair<T>(acc_o[dt][2] * coef, acc_o[dt][3] * coef);
            if (q0 + l16 < q_len) *(u32x2 *)(orow + dt * 16) = packed;
          }
        }
      } else {
        asm volatile("" ::: "memory");
        kdma();
        vdma();
      }
    });
    lds_barrier();  // the late waves' merge barrier
  }
}

// one launch of the kernel for the storage format (BF16 or F16)
template <bool STRIDED>
int launch_fa(wafer_hip_context *ctx, uint32_t format, bool causal, const void *q, const void *k, const void *v,
              void *o, uint32_t q_heads, uint32_t kv_heads, uint32_t q_len, uint32_t kv_len, float c, int bh_count,
              int n_qblocks, const FaStrides &st) {
  dim3 grid((unsigned)(bh_count * ((n_qblocks + 1) / 2)));  // one workgroup per pair of query blocks
#define FA_GO(T, CZ)                                                                                           \
  hipLaunchKernelGGL((fa_prefill_d128<T, CZ, STRIDED>), grid, dim3(THREADS), 0, ctx->stream, (const uint16_t *)q, \
                     (const uint16_t *)k, (const uint16_t *)v, (uint16_t *)o, (int)q_heads, (int)kv_heads,      \
                     (int)q_len, (int)kv_len, c, bh_count, n_qblocks, st)
  if (format == WAFER_FMT_BF16) {
    if (causal) FA_GO(__bf16, true);
    else FA_GO(__bf16, false);
  } else {
    if (causal) FA_GO(_Float16, true);
    else FA_GO(_Float16, false);
  }
#undef FA_GO
  return launch_status("fa_prefill_d128");
}

}  // namespace
}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_attention_prefill(wafer_hip_context *ctx, uint32_t format,
                                           const void *q, const void *k, const void *v,
                                           void *o, uint32_t batch, uint32_t q_heads,
                                           uint32_t kv_heads, uint32_t q_len,
                                           uint32_t kv_len, uint32_t head_dim,
                                           float scale, uint32_t causal) {
  WAFER_CHECK_CTX(ctx);
  if ((format != WAFER_FMT_BF16 && format != WAFER_FMT_F16) || head_dim != D) {
    wafer_hip_attention_mask mask{};
    mask.flags = causal ? WAFER_HIP_ATT_CAUSAL : 0u;
    return attention_prefill_masked(ctx, format, q, k, v, o, batch, q_heads, kv_heads, q_len, kv_len, head_dim,
                                    scale, &mask);
  }
  if (!q || !k || !v || !o) return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: null tensor");
  if (batch == 0 || q_heads == 0 || kv_heads == 0 || q_len == 0 || kv_len == 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: empty dimension");
  if (q_heads % kv_heads != 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: q_heads % kv_heads != 0");
  if (!(scale > 0.0f)) return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: scale must be positive");
  if ((uint64_t)kv_len * D * 2 > 0x7fffffffull)  // 32-bit buffer offsets of one head's K/V
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_prefill: kv_len too large (max 8388607)");
  const uint64_t n_qblocks64 = (q_len + QB - 1) / QB;
  if ((uint64_t)batch * q_heads * ((n_qblocks64 + 1) / 2) > 0x7fffffffull)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: grid too large");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const int n_qblocks = (int)n_qblocks64;
  const int bh_count = (int)(batch * q_heads);
  const float c = scale * 0x1.715476p+0f;
  return launch_fa<false>(ctx, format, causal != 0, q, k, v, o, q_heads, kv_heads, q_len, kv_len, c, bh_count,
                          n_qblocks, FaStrides{});
}

extern "C" int wafer_hip_attention_prefill_strided(wafer_hip_context *ctx, uint32_t format, const void *q,
                                                   const void *k, const void *v, void *o, uint32_t batch,
                                                   uint32_t q_heads, uint32_t kv_heads, uint32_t q_len,
                                                   uint32_t kv_len, uint32_t head_dim, float scale,
                                                   uint32_t causal, const wafer_hip_attention_strides *strides) {
  WAFER_CHECK_CTX(ctx);
  if ((format != WAFER_FMT_BF16 && format != WAFER_FMT_F16) || head_dim != D)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_prefill_strided: BF16 or F16 with head_dim 128 only");
  if (!q || !k || !v || !o || !strides) return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill_strided: null tensor");
  if (batch == 0 || q_heads == 0 || kv_heads == 0 || q_len == 0 || kv_len == 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill_strided: empty dimension");
  if (q_heads % kv_heads != 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill_strided: q_heads % kv_heads != 0");
  if (!(scale > 0.0f)) return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill_strided: scale must be positive");
  const int64_t *all[4] = {strides->q, strides->k, strides->v, strides->o};
  for (const int64_t *t : all)
    for (int i = 0; i < 3; ++i)
      if (t[i] < 0 || t[i] % 8) return fail(WAFER_HIP_E_INVALID_FIELD,
                                            "attention_prefill_strided: strides must be non-negative multiples of 8");
  if (strides->q[2] < D || strides->k[2] < D || strides->v[2] < D || strides->o[2] < D)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill_strided: row strides below head_dim");
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) & 15)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill_strided: tensors must be 16-byte aligned");
  // one key block's buffer range and the DMA lane offsets are 32-bit
  if (((int64_t)(BK - 1) * std::max(strides->k[2], strides->v[2]) + D) * 2 > 0x7fffffffll)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_prefill_strided: key row stride too large");
  const uint64_t n_qblocks64 = (q_len + QB - 1) / QB;
  if ((uint64_t)batch * q_heads * ((n_qblocks64 + 1) / 2) > 0x7fffffffull)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill_strided: grid too large");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  FaStrides st{};
  for (int i = 0; i < 3; ++i) {
    st.q[i] = strides->q[i];
    st.k[i] = strides->k[i];
    st.v[i] = strides->v[i];
    st.o[i] = strides->o[i];
  }
  const int n_qblocks = (int)n_qblocks64;
  const int bh_count = (int)(batch * q_heads);
  const float c = scale * 0x1.715476p+0f;
  return launch_fa<true>(ctx, format, causal != 0, q, k, v, o, q_heads, kv_heads, q_len, kv_len, c, bh_count,
                         n_qblocks, st);
}
