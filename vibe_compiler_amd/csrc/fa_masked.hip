// fa_masked.hip -- FA prefill with masks, FP16 storage and head_dim 64 (and
// a small-head_dim lane) for gfx950.
//
// Semantics: the compiler's online-attention decomposition
// (lib/Wafer/Transforms/Linalg/OnlineAttentionDecomposition.cpp:568-597) with
// its score region and position bias (applyScoreRegion :279-426): per
// element s = q.k (f32), t = s*scale, optionally narrowed to the storage
// type, + an additive F32 mask value (optionally narrowed again), and -inf
// where the key is invisible (boolean mask false, beyond the causal diagonal
// or the window, or at or past kv_len, the valid prefix of :185-210).  Then
// m' = max(m, rowmax t), P = ExpLp(t - m'), l = l*alpha + rowsum(P),
// acc = acc*alpha + narrow(P).V, out = narrow(acc * (1/l)), exactly 0 for a
// row that saw no visible key (zero_fully_masked,
// OnlineAttentionMaterialization.cpp:229-242).
//
// Two kernels:
//  * fa_fwd<T, D, MASK> (D = 64 or 128, BF16 or F16): a workgroup of 4 waves
//    serves two 64-query blocks of one (batch, head) (the late block of the
//    causal triangle, then the early one, so every workgroup carries the
//    same work); wave w owns query tile w & 1 (32 queries) and key half
//    w >> 1 (the even or the odd 64-key blocks); the two halves merge through
//    LDS with the state merge of OnlineAttentionMaterialization.cpp:264-373.
//    One wave per SIMD with the full 512-entry register file.
//    - S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_{bf16,f16}: Q
//      stays in VGPRs, K fragments are ds_read_b128 from LDS, V^T fragments
//      come from row-major V through ds_read_b64_tr_b16, P^T feeds the B
//      operand straight from the score registers after RNE narrowing;
//    - K / V blocks move global -> LDS by buffer_load ... lds, double
//      buffered; each iteration is one hand-pipelined sequence of slots
//      (QK of block u+1, exponentials of block u, PV of block u-1, the LDS
//      fragment reads two slots ahead and this iteration's DMA issues), with
//      scheduling fences between slots;
//    - lazy rescale: exponentials are taken against a per-query reference
//      that moves only when a block's max exceeds it by more than 2^8 (log2
//      domain); a lane sum of P above 2^8 detects every such block, and the
//      exact update (block max, state rescale, exponentials again) runs
//      then.  P <= 2^8 and its narrowing point differs from the
//      reference's with the same relative bound;
//    - MASK_CAUSAL masks by position only (no mask operands, no rounding);
//      MASK_GENERAL evaluates the whole score region per element in the
//      natural-log domain and hands u = t*log2(e) to the exponentials.
//  * fa_small<T> (head_dim <= 64 other than 64): one thread per query row,
//    K / V blocks of 64 keys staged as f32 in LDS, the reference's block
//    update evaluated per row in its own order (dot products as fma chains
//    from +0, row sums and PV sums left to right).
#include "common.h"

#include <type_traits>

namespace wafer {
namespace {

constexpr int QB = 64;        // queries per query block (two 32-query wave tiles)
constexpr int BK = 64;        // keys per KV block
constexpr int THREADS = 256;  // 4 waves: (tile, key half)
constexpr float RESCALE_LOG2 = 8.0f;
constexpr float RESCALE_BOUND = 256.0f;
// "no reference yet": the lowest finite float, so exp2(u - NOREF) is +inf
// (or at least 1) for a visible score and 0 for a masked one (never NaN),
// exp2(NOREF - x) == 0 for any score x above NOREF + 150, and every finite
// visible score is a valid reference (P relative to NOREF stays below 2^8
// until a score exceeds NOREF + 8, which sends the wave to the exact update).
constexpr float NOREF = -0x1.fffffep127f;
constexpr float LOG2E = 0x1.715476p+0f;

enum { MASK_CAUSAL = 1, MASK_GENERAL = 2 };
constexpr uint32_t F_CAUSAL = WAFER_HIP_ATT_CAUSAL, F_WINDOW = WAFER_HIP_ATT_WINDOW,
                   F_ROUND_SCALED = WAFER_HIP_ATT_ROUND_SCALED, F_ROUND_BIASED = WAFER_HIP_ATT_ROUND_BIASED;

struct FaArgs {
  const uint16_t *q, *k, *v;
  uint16_t *o;
  int q_heads, kv_heads, q_len, kv_len, kv_cap;
  float c;      // scale * log2(e)
  float scale;
  int bh_count, n_qblocks;
  uint32_t flags;
  int diag;     // CAUSAL: key j visible to query i only if j <= i + diag
  int lo_off;   // WINDOW: and j >= i + lo_off (lo_off = diag - window + 1)
  const float *bias;
  long long bias_sb, bias_sh, bias_sq;
  const uint8_t *keep;
  long long keep_sb, keep_sh, keep_sq;
};

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

template <typename T>
__device__ inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (std::is_same_v<T, __bf16>)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// two f32 rounded to the storage format (RNE), packed low / high
template <typename T>
__device__ inline uint32_t pack2(float lo, float hi) {
  typedef T t2 __attribute__((ext_vector_type(2)));
  const t2 v = {(T)f32_rounded(lo), (T)f32_rounded(hi)};
  return __builtin_bit_cast(uint32_t, v);
}
template <typename T>
__device__ inline float round_to(float x) {
  return (float)(T)f32_rounded(x);
}
template <typename T>
__device__ inline float load_elem(const uint16_t *p) {
  return (float)__builtin_bit_cast(T, *p);
}

// x combined with the value of lane ^ 32.  v_permlane32_swap exchanges the
// upper half of its first operand with the lower half of its second, so with
// both operands x the two results hold {own, partner} in some order per lane.
__device__ inline float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// One score through the score region and the masks: visible -> u = t*log2(e)
// (a finite t whose u overflows is clamped to the lowest finite float),
// invisible -> -inf, whatever t is (an invisible key is excluded).
template <typename T>
__device__ inline float general_score(float s, float scale, uint32_t flags, const float *brow,
                                      const uint8_t *krow, int key, bool vis) {
  float t = s * scale;
  if (flags & F_ROUND_SCALED) t = round_to<T>(t);
  if (vis && brow) {
    t = t + brow[key];
    if (flags & F_ROUND_BIASED) t = round_to<T>(t);
  }
  if (vis && krow) vis = krow[key] != 0;
  if (!vis || t == -__builtin_inff()) return -__builtin_inff();
  const float u = t * LOG2E;
  return u == u ? fmaxf(u, NOREF) : u;  // NaN passes through
}

// LDS swizzles (16-byte chunk index XOR): K rows are read 32 rows x one
// chunk (ds_read_b128), V rows 4 rows x 64 bytes (ds_read_b64_tr_b16).
template <int D>
__device__ inline int swz_k(int row) {
  return D == 128 ? (row & 15) : ((row >> 1) & 7);
}
template <int D>
__device__ inline int swz_v(int row) {
  return D == 128 ? 4 * (row & 3) : 4 * ((row >> 1) & 1);
}

template <typename T, int D, int MASK>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void fa_fwd(const FaArgs a) {
  constexpr int ROWB = 2 * D;            // bytes per K / V row
  constexpr int CH = ROWB / 16;          // 16-byte chunks per row
  constexpr int RPI = 64 / CH;           // rows per 1 KiB DMA instruction
  constexpr int NDMA = 32 / RPI;         // DMA instructions per wave per block (32 rows)
  constexpr int BLK = BK * ROWB;         // bytes per K / V block
  constexpr int KS = D / 16;             // QK k-steps
  constexpr int DT = D / 32;             // O^T d tiles
  // four distinct arrays (K slot 0/1, V slot 0/1, each [half][block]), so
  // that the compiler can tell a slot being filled by DMA from the slot being
  // read and waits for the moves only at the iteration's barrier
  __shared__ __align__(1024) char sk0[2 * BLK], sk1[2 * BLK], sv0[2 * BLK], sv1[2 * BLK];
  __shared__ float sml[4][2][64];

  const int bid = blockIdx.x;
  const int pair = bid / a.bh_count;
  const int bh = bid - pair * a.bh_count;
  const int b = bh / a.q_heads;
  const int h = bh - b * a.q_heads;
  const int kvh = h / (a.q_heads / a.kv_heads);
  const uint16_t *Qp = a.q + (size_t)bh * a.q_len * D;
  const uint16_t *Kp = a.k + (size_t)(b * a.kv_heads + kvh) * a.kv_cap * D;
  const uint16_t *Vp = a.v + (size_t)(b * a.kv_heads + kvh) * a.kv_cap * D;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = wave & 1, half = wave >> 1;
  const int l32 = lane & 31, g = lane >> 5;

  // ---- phases: late query block then early one (causal balance)
  const int qb_a = a.n_qblocks - 1 - pair, qb_b = pair;
  // key blocks [lo, lo + n) that meet a query block's visible key range
  auto key_range = [&](int qb, int &lo, int &n) __attribute__((always_inline)) {
    int klo = 0, khi = a.kv_len - 1;
    if (a.flags & F_CAUSAL) khi = min(khi, qb * QB + QB - 1 + a.diag);
    if (MASK == MASK_GENERAL && (a.flags & F_WINDOW)) klo = max(0, qb * QB + a.lo_off);
    if (khi < klo) { lo = 0; n = 0; return; }
    lo = klo / BK;
    n = khi / BK - lo + 1;
  };
  int lo_a, nk_a, lo_b, nk_b;
  key_range(qb_a, lo_a, nk_a);
  if (qb_b < qb_a) key_range(qb_b, lo_b, nk_b); else { lo_b = 0; nk_b = 0; }
  const bool has_b = qb_b < qb_a;
  const int ta = (nk_a + 1) / 2, tb = (nk_b + 1) / 2;
  const int niter = ta + tb;
  // this half's block count per phase
  const int na_h = (nk_a + 1 - half) / 2, nb_h = (nk_b + 1 - half) / 2;

  // key block of global iteration x for this half (clamped: loads of blocks
  // that no iteration uses are harmless)
  auto block_of = [&](int x) __attribute__((always_inline)) {
    const bool in_a = x < ta || tb == 0;
    const int u = in_a ? min(x, ta - 1) : min(x - ta, tb - 1);
    return in_a ? lo_a + min(2 * u + half, nk_a - 1) : lo_b + min(2 * u + half, nk_b - 1);
  };

  // ---- DMA: wave `tile` of half h moves rows [32 tile, 32 tile + 32) of
  // half h's K and V blocks; instruction j fills 1 KiB (RPI rows); lane i
  // writes chunk position i % CH of row i / CH and loads the logical chunk
  // the swizzle puts there.  The K swizzle repeats every PK instructions and
  // the V swizzle every one, so lane offsets are kept for the first PK (one)
  // instructions and the rest add a wave-uniform row step.
  constexpr int PK = D == 128 ? 4 : 2;
  uint32_t dk_base[PK], dv_base;
#pragma unroll
  for (int j = 0; j < PK; ++j) {
    const int row = tile * 32 + j * RPI + lane / CH, pos = lane % CH;
    dk_base[j] = (uint32_t)(row * ROWB + ((pos ^ swz_k<D>(row)) << 4));
  }
  {
    const int row = tile * 32 + lane / CH, pos = lane % CH;
    dv_base = (uint32_t)(row * ROWB + ((pos ^ swz_v<D>(row)) << 4));
  }
  auto dma_voff = [&](bool is_k, int j) __attribute__((always_inline)) { return is_k ? dk_base[j % PK] : dv_base; };
  auto dma_soff = [&](bool is_k, int j) __attribute__((always_inline)) {
    return is_k ? (j / PK) * (PK * 1024) : j * 1024;
  };
  // a block's buffer resource covers its valid rows only: rows past kv_len
  // read as zero
  auto rsrc_of = [&](const uint16_t *base, int kb) __attribute__((always_inline)) {
    const int rows = min(BK, a.kv_len - kb * BK);
    return __builtin_amdgcn_make_buffer_rsrc((void *)(base + (size_t)kb * BK * D), 0, rows * ROWB, 0x00020000);
  };
  // (values are copied to locals first: a dependent-array element passed
  // straight to the builtin makes the host compile drop the kernel)
  auto dma_one = [&](__amdgpu_buffer_rsrc_t r, char *d, bool is_k, int j) __attribute__((always_inline)) {
    const uint32_t vo = dma_voff(is_k, j);
    const int so = dma_soff(is_k, j);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)(d + j * 1024), 16, vo, so,
                                             0, 0);
  };
  auto dma = [&](const uint16_t *base, int kb, char *dst, bool is_k) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t r = rsrc_of(base, __builtin_amdgcn_readfirstlane(kb));
    char *d = dst + tile * 32 * ROWB;
#pragma unroll
    for (int j = 0; j < NDMA; ++j) dma_one(r, d, is_k, j);
  };
  auto kslot = [&](int slot) __attribute__((always_inline)) { return (slot ? sk1 : sk0) + half * BLK; };
  auto vslot = [&](int slot) __attribute__((always_inline)) { return (slot ? sv1 : sv0) + half * BLK; };

  // ---- LDS fragment offsets
  // K (A operand of S^T = K Q^T, k-step s, key tile kt): row kt*32 + l32,
  // logical chunk 2 s + g
  uint32_t k_off[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) k_off[s] = (uint32_t)(l32 * ROWB + (((2 * s + g) ^ swz_k<D>(l32)) << 4));
  // V^T (A operand of O^T = V^T P^T via ds_read_b64_tr_b16): 16-lane group G
  // covers d = dt*32 + 16 (G & 1) + [0,16) and keys kbase + 8 p + 4 (G >> 1) + [0,4);
  // lane i of the group supplies the address of row + (i >> 2), d + 4 (i & 3)
  const int G = lane >> 4, gi = lane & 15, e = gi >> 2, qq = gi & 3;
  uint32_t v_off[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int row = 4 * (G >> 1) + e;  // + kbase + 8 p (multiples of 4: the swizzle is fixed)
    const int lc = dt * 4 + 2 * (G & 1) + (qq >> 1);
    v_off[dt] = (uint32_t)(row * ROWB + ((lc ^ swz_v<D>(row)) << 4) + 8 * (qq & 1));
  }

  // ---- per-wave state
  u32x4 qf[KS];
  int q0 = 0;
  auto load_q = [&](int qb) __attribute__((always_inline)) {
    q0 = qb * QB + tile * 32;
    const int row = min(q0 + l32, a.q_len - 1);
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = *(const u32x4 *)(Qp + (size_t)row * D + 16 * s + 8 * g);
  };
  f32x16 acc[DT];
  float m_ref = NOREF, l_part = 0.0f;
  auto reset = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[dt][r] = 0.0f;
    m_ref = NOREF;
    l_part = 0.0f;
  };

  // scores of block kb -> the operand of the exponentials (MASK_GENERAL
  // rewrites S into u = t * log2(e) and uses c_eff = 1)
  auto mask_scores = [&](int kb, f32x16 (&s)[2]) __attribute__((always_inline)) {
    const int qi = q0 + l32;
    if constexpr (MASK == MASK_GENERAL) {
      const int qc = min(qi, a.q_len - 1);
      const float *brow = a.bias ? a.bias + b * a.bias_sb + h * a.bias_sh + qc * a.bias_sq : nullptr;
      const uint8_t *krow = a.keep ? a.keep + b * a.keep_sb + h * a.keep_sh + qc * a.keep_sq : nullptr;
      const int hi_k = (a.flags & F_CAUSAL) ? min(qi + a.diag, a.kv_len - 1) : a.kv_len - 1;
      const int lo_k = (a.flags & F_WINDOW) ? qi + a.lo_off : 0;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * BK + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          s[kt][r] = general_score<T>(s[kt][r], a.scale, a.flags, brow, krow, key, key <= hi_k && key >= lo_k);
        }
    } else {
      const bool need = ((a.flags & F_CAUSAL) && kb * BK + BK - 1 > q0 + a.diag) || kb * BK + BK > a.kv_len;
      if (need) {
        const int lim = (a.flags & F_CAUSAL) ? min(qi + a.diag, a.kv_len - 1) : a.kv_len - 1;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (kb * BK + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3) > lim) s[kt][r] = -__builtin_inff();
      }
    }
  };
  const float c_eff = MASK == MASK_GENERAL ? 1.0f : a.c;

  // The exact update, taken when some lane's sum of P crossed the bound
  // (rare: the first visible block of a query and a later one whose max
  // exceeds the reference by 2^8): block max, reference moved with the state
  // rescaled when the max exceeds it by more than 2^8, then the
  // exponentials and the lane sum again.  Fenced in small pieces so that it
  // adds no register pressure to the pipelined iteration around it.
  auto exact = [&](const f32x16 (&s)[2], u32x4 (&p)[4]) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    float mx = -__builtin_inff();
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kt][r]);
    mx = xor32_max(mx);
    const float mc = mx * c_eff;
    if (mx != -__builtin_inff() && mc > m_ref + RESCALE_LOG2) {
      const float alpha = __builtin_amdgcn_exp2f(m_ref - mc);
      l_part *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
        __builtin_amdgcn_sched_barrier(0);
      }
      m_ref = mc;
    }
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {  // pair q: scores 2q, 2q + 1 of tile q / 8
      const int kt = q / 8, j = 2 * (q % 8);
      const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][j], c_eff, -m_ref));
      const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][j + 1], c_eff, -m_ref));
      p[2 * kt + j / 8][(j % 8) / 2] = pack2<T>(e0, e1);
      sum += e0 + e1;
      if (q % 4 == 3) __builtin_amdgcn_sched_barrier(0);
    }
    return sum;
  };

  // ---- merge of the two key halves of a query tile (reduce-scatter) and
  // finalize: out = narrow(acc * Recip(l)), 0 for a row that saw no key
  auto finish_h = [&](char *xch, auto half_c) __attribute__((always_inline)) {
    constexpr int H = decltype(half_c)::value;  // == half: every acc index stays static
    const float l_full = xor32_sum(l_part);
    sml[wave][0][lane] = m_ref;
    sml[wave][1][lane] = l_full;
    // hand the partner the d tiles it keeps: half h keeps [h DT/2, (h+1) DT/2)
    f32x4 *x = (f32x4 *)(xch + wave * (DT / 2) * 16 * 64 * 4);
#pragma unroll
    for (int i = 0; i < DT / 2; ++i) {
      const int dt = (1 - H) * (DT / 2) + i;
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        f32x4 v = {acc[dt][4 * r4], acc[dt][4 * r4 + 1], acc[dt][4 * r4 + 2], acc[dt][4 * r4 + 3]};
        x[(i * 4 + r4) * 64 + lane] = v;
      }
    }
    __syncthreads();
    const int pw = wave ^ 2;
    const float m1 = sml[pw][0][lane], l1 = sml[pw][1][lane];
    const float em = fmaxf(m_ref, m1);
    const float s0 = __builtin_amdgcn_exp2f(m_ref - em), s1 = __builtin_amdgcn_exp2f(m1 - em);
    const float l = l_full * s0 + l1 * s1;
    const float coef = l == 0.0f ? 0.0f : 1.0f / l;
    const f32x4 *px = (const f32x4 *)(xch + pw * (DT / 2) * 16 * 64 * 4);
    const int qi = q0 + l32;
    uint16_t *orow = a.o + ((size_t)bh * a.q_len + min(qi, a.q_len - 1)) * D;
#pragma unroll
    for (int i = 0; i < DT / 2; ++i) {
      const int dt = H * (DT / 2) + i;
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f32x4 o1 = px[(i * 4 + r4) * 64 + lane];
        float r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = (acc[dt][4 * r4 + j] * s0 + o1[j] * s1) * coef;
        u32x2 w;
        w[0] = pack2<T>(r[0], r[1]);
        w[1] = pack2<T>(r[2], r[3]);
        if (qi < a.q_len) *(u32x2 *)(orow + dt * 32 + 8 * r4 + 4 * g) = w;
      }
    }
    __syncthreads();  // exchange reads done before the slot is reused
    asm volatile("; fa merge tail %0" ::"n"(H));  // keeps the two copies apart
  };
  auto finish = [&](char *xch) __attribute__((always_inline)) {
    if (half == 0)
      finish_h(xch, std::integral_constant<int, 0>{});
    else
      finish_h(xch, std::integral_constant<int, 1>{});
  };

  // ---- the pipeline.  Global iteration t (phase A: t < ta, then phase B)
  // works on block u = t - t0 of this half: softmax(S_u), PV(u-1), QK(u+1);
  // it moves K(t+2) into K slot t%2 and V(t) into V slot t%2.  A phase starts
  // with QK(0) (prologue) and ends with PV(last) and the merge.  S and P are
  // double-buffered by iteration parity, so no registers are copied.
  f32x16 sA[2], sB[2];
  u32x4 pA[4], pB[4];
  using T1 = std::true_type;
  using F0 = std::false_type;

  // One iteration's work as a hand-pipelined sequence of NSLOT slots.  Slot
  // i issues QK MFMA i and PV MFMA i, the LDS fragment reads of slot i + PF,
  // its share of the softmax VALU work (exponentials, storage rounding, row
  // sum) and its share of the K/V moves; sched_barrier fences keep each
  // slot's instructions together (the compiler reorders within a slot only).
  // Flags: SOFT (exponentials of s_cur into p_cur; returns the lane sum), PV
  // (acc += V^T P^T from vb), QK (s_nxt = K Q^T from kb), MV (moves into kd,
  // vd).  QK MFMA i is k-step i / 2 of key tile i % 2; PV MFMA i is k-step
  // i / DT of d tile i % DT.
  constexpr int NQK = 2 * KS, NPV = 4 * DT, NSLOT = NQK > NPV ? NQK : NPV, PF = 2;
  constexpr int SPS = 32 / NSLOT;                      // scores per slot
  constexpr int DPS = (2 * NDMA + NSLOT - 1) / NSLOT;  // moves per slot
  auto body = [&](auto soft_c, auto pv_c, auto qk_c, auto mv_c, const char *kb, const char *vb, char *kd, char *vd,
                  __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, f32x16 (&s_cur)[2], f32x16 (&s_nxt)[2],
                  const u32x4 (&p_prev)[4], u32x4 (&p_cur)[4]) __attribute__((always_inline)) {
    constexpr bool SOFT = decltype(soft_c)::value, PV = decltype(pv_c)::value, QK = decltype(qk_c)::value,
                   MV = decltype(mv_c)::value;
    u32x4 kf[NQK], vf[NPV];
    auto read_k = [&](int i) __attribute__((always_inline)) {
      kf[i] = *(const u32x4 *)(kb + k_off[i / 2] + (i % 2) * 32 * ROWB);
    };
    auto read_v = [&](int i) __attribute__((always_inline)) {
      const int s4 = i / DT, dt = i % DT;
      const int kbase = (s4 >> 1) * 32 + 16 * (s4 & 1);
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(vb + v_off[dt] + kbase * ROWB));
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(vb + v_off[dt] + (kbase + 8) * ROWB));
      vf[i] = __builtin_bit_cast(u32x4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    auto move = [&](int m) __attribute__((always_inline)) {  // K moves first, then V
      const bool is_k = m < NDMA;
      dma_one(is_k ? rk : rv, is_k ? kd : vd, is_k, is_k ? m : m - NDMA);
    };
    float e[32], part[4];
    auto score = [&](int r) __attribute__((always_inline)) {  // score r = 16 kt + j
      e[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[r / 16][r % 16], c_eff, -m_ref));
    };
    auto finish_pair = [&](int r) __attribute__((always_inline)) {  // scores r, r + 1 done (r even)
      const int kt = r / 16, j = r % 16;
      p_cur[2 * kt + j / 8][(j % 8) / 2] = pack2<T>(e[r], e[r + 1]);
      const float ps = e[r] + e[r + 1];
      const int pi = (r / 2) % 4;
      part[pi] = r < 8 ? ps : part[pi] + ps;
    };
    if constexpr (QK) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) s_nxt[kt][r] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      if (QK && i < NQK) read_k(i);
      if (PV && i < NPV) read_v(i);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) {
      if (QK && i < NQK) s_nxt[i % 2] = mfma32<T>(kf[i], qf[i / 2], s_nxt[i % 2]);
      if (QK && i + PF < NQK) read_k(i + PF);
      if (PV && i + PF < NPV) read_v(i + PF);
      if constexpr (SOFT) {
#pragma unroll
        for (int r = i * SPS; r < i * SPS + SPS / 2; ++r) score(r);
      }
      if (PV && i < NPV) acc[i % DT] = mfma32<T>(vf[i], p_prev[i / DT], acc[i % DT]);
      if constexpr (SOFT) {
#pragma unroll
        for (int r = i * SPS + SPS / 2; r < (i + 1) * SPS; ++r) score(r);
#pragma unroll
        for (int r = i * SPS; r < (i + 1) * SPS; r += 2) finish_pair(r);
      }
      if constexpr (MV) {
#pragma unroll
        for (int m = i * DPS; m < (i + 1) * DPS && m < 2 * NDMA; ++m) move(m);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    return SOFT ? (part[0] + part[1]) + (part[2] + part[3]) : 0.0f;
  };
  // after the softmax of a block: the exact update if a lane sum crossed the
  // bound, then the row sum
  auto settle = [&](float rs, f32x16 (&s_cur)[2], u32x4 (&p_cur)[4]) __attribute__((always_inline)) {
    if (__builtin_expect(__any(rs > RESCALE_BOUND), 0)) rs = exact(s_cur, p_cur);
    l_part += rs;
  };
  auto end_iteration = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };

  // One iteration of the phase loop for block u of this half (slot parity
  // P = t & 1): the score mask where the block needs it (every score of a
  // block the half does not have), then the pipelined body, the settle and
  // the barrier.  FIRST: no PV yet.
  auto iter = [&](auto parity, auto first_c, int t, int u, int nh, int lo, f32x16 (&s_cur)[2], f32x16 (&s_nxt)[2],
                  const u32x4 (&p_prev)[4], u32x4 (&p_cur)[4]) __attribute__((always_inline)) {
    constexpr int P = decltype(parity)::value;
    constexpr bool FIRST = decltype(first_c)::value;
    if (u >= nh) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) s_cur[kt][r] = -__builtin_inff();
    } else {
      mask_scores(lo + 2 * u + half, s_cur);
    }
    const float rs = body(T1{}, std::integral_constant<bool, !FIRST>{}, T1{}, T1{}, (P ? sk0 : sk1) + half * BLK,
                          (P ? sv0 : sv1) + half * BLK, (P ? sk1 : sk0) + half * BLK + tile * 32 * ROWB,
                          (P ? sv1 : sv0) + half * BLK + tile * 32 * ROWB, rsrc_of(Kp, block_of(t + 2)),
                          rsrc_of(Vp, block_of(t)), s_cur, s_nxt, p_prev, p_cur);
    settle(rs, s_cur, p_cur);
    end_iteration();
  };
  // One phase: query block qb, key blocks lo + 2u + half for u < nh, over
  // tn iterations (the half with one block fewer idles through its last
  // iteration: all its scores masked, P = 0), then PV of the last P (zero
  // for that half) and the merge.
  auto run_phase = [&](int qb, int lo, int tn, int nh, int &t) __attribute__((always_inline)) {
    load_q(qb);
    reset();
    if (tn > 0) {
      {  // prologue: S_0 = QK(0) (K(t) moved two iterations ago)
        const char *kb = kslot(t & 1);
        body(F0{}, F0{}, T1{}, F0{}, kb, kb, nullptr, nullptr, rsrc_of(Kp, 0), rsrc_of(Vp, 0), sB, sA, pA, pB);
      }
      __syncthreads();
      auto run = [&](auto p0) __attribute__((always_inline)) {
        constexpr int P0 = decltype(p0)::value, P1 = P0 ^ 1;
        using IP0 = std::integral_constant<int, P0>;
        using IP1 = std::integral_constant<int, P1>;
        iter(IP0{}, T1{}, t, 0, nh, lo, sA, sB, pB, pA);
        int u = 1;
        for (; u + 1 < tn; u += 2) {
          iter(IP1{}, F0{}, t + u, u, nh, lo, sB, sA, pA, pB);
          iter(IP0{}, F0{}, t + u + 1, u + 1, nh, lo, sA, sB, pB, pA);
        }
        if (u < tn) iter(IP1{}, F0{}, t + u, u, nh, lo, sB, sA, pA, pB);
        t += tn;
        // epilogue: PV of the last block (P of iteration tn - 1; its V moved then)
        const char *vb = vslot((t - 1) & 1);
        if (tn & 1)
          body(F0{}, T1{}, F0{}, F0{}, vb, vb, nullptr, nullptr, rsrc_of(Kp, 0), rsrc_of(Vp, 0), sA, sB, pA, pB);
        else
          body(F0{}, T1{}, F0{}, F0{}, vb, vb, nullptr, nullptr, rsrc_of(Kp, 0), rsrc_of(Vp, 0), sA, sB, pB, pA);
      };
      if (t & 1)
        run(std::integral_constant<int, 1>{});
      else
        run(std::integral_constant<int, 0>{});
    }
    finish((t & 1) ? sv1 : sv0);  // both halves of the free V slot
  };

  if (niter > 0) {
    dma(Kp, block_of(0), kslot(0), true);
    dma(Kp, block_of(1), kslot(1), true);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  int t = 0;
  run_phase(qb_a, lo_a, ta, na_h, t);
  if (has_b) run_phase(qb_b, lo_b, tb, nb_h, t);
}

// ---- the small-head_dim lane: one thread per query row
constexpr int SMALL_D = 64;        // largest head_dim served
constexpr int SMALL_ROWS = 256;    // query rows per workgroup
constexpr int SMALL_BK = 64;       // keys per block (the reference's block walk)

template <typename T>
__global__ __launch_bounds__(SMALL_ROWS) void fa_small(const FaArgs a, int D, int row_blocks) {
  __shared__ float sk[SMALL_BK][SMALL_D + 1], sv[SMALL_BK][SMALL_D + 1], ss[SMALL_BK][SMALL_ROWS];
  const int bh = blockIdx.x / row_blocks;
  const int rb = blockIdx.x - bh * row_blocks;
  const int b = bh / a.q_heads;
  const int h = bh - b * a.q_heads;
  const int kvh = h / (a.q_heads / a.kv_heads);
  const uint16_t *Kp = a.k + (size_t)(b * a.kv_heads + kvh) * a.kv_cap * D;
  const uint16_t *Vp = a.v + (size_t)(b * a.kv_heads + kvh) * a.kv_cap * D;
  const int i0 = rb * SMALL_ROWS, i = i0 + (int)threadIdx.x;
  const bool live = i < a.q_len;
  const int ic = min(i, a.q_len - 1);

  float q[SMALL_D], acc[SMALL_D];
  const uint16_t *qrow = a.q + ((size_t)bh * a.q_len + ic) * D;
#pragma unroll
  for (int d = 0; d < SMALL_D; ++d) {
    q[d] = d < D ? load_elem<T>(qrow + d) : 0.0f;
    acc[d] = 0.0f;
  }
  // visible key positions of a row
  auto lo_of = [&](int r) { return (a.flags & F_WINDOW) ? max(0, r + a.lo_off) : 0; };
  auto hi_of = [&](int r) { return (a.flags & F_CAUSAL) ? min(a.kv_len - 1, r + a.diag) : a.kv_len - 1; };
  const int lo = lo_of(ic), hi = hi_of(ic);
  // the workgroup walks the union of its rows' ranges (both bounds grow with
  // the row), starting at a block boundary as the reference's walk does
  const int last = min(i0 + SMALL_ROWS, a.q_len) - 1;
  const int wlo = lo_of(i0), whi = hi_of(last);
  const float *brow = a.bias ? a.bias + b * a.bias_sb + h * a.bias_sh + ic * a.bias_sq : nullptr;
  const uint8_t *krow = a.keep ? a.keep + b * a.keep_sb + h * a.keep_sh + ic * a.keep_sq : nullptr;
  float m = -__builtin_inff(), l = 0.0f;

  for (int j0 = wlo / SMALL_BK * SMALL_BK; j0 <= whi; j0 += SMALL_BK) {
    const int n = min(SMALL_BK, a.kv_len - j0);
    __syncthreads();
    for (int x = threadIdx.x; x < SMALL_BK * D; x += SMALL_ROWS) {
      const int r = x / D, d = x - r * D;
      sk[r][d] = r < n ? load_elem<T>(Kp + (size_t)(j0 + r) * D + d) : 0.0f;
      sv[r][d] = r < n ? load_elem<T>(Vp + (size_t)(j0 + r) * D + d) : 0.0f;
    }
    __syncthreads();
    // a block that meets none of this row's visible keys changes nothing
    // (alpha = 1, P = 0; or m stays -inf with l = acc = 0)
    if (!live || lo > hi || j0 > hi || j0 + SMALL_BK - 1 < lo) continue;
    // scores and then P of this row live in LDS column threadIdx.x (a
    // register array indexed by the key loop would go to scratch)
    float rowmax = -__builtin_inff();
#pragma unroll 1
    for (int j = 0; j < SMALL_BK; ++j) {
      float t = -__builtin_inff();
      if (j < n) {
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < SMALL_D; ++d)
          if (d < D) dot = __builtin_fmaf(q[d], sk[j][d], dot);
        const int key = j0 + j;
        t = dot * a.scale;
        if (a.flags & F_ROUND_SCALED) t = round_to<T>(t);
        if (brow) {
          t = t + brow[key];
          if (a.flags & F_ROUND_BIASED) t = round_to<T>(t);
        }
        if (key < lo || key > hi || (krow && krow[key] == 0)) t = -__builtin_inff();  // excluded
      }
      ss[j][threadIdx.x] = t;
      rowmax = (t != t || rowmax != rowmax) ? __builtin_nanf("") : fmaxf(rowmax, t);
    }
    const float mnew = (m != m || rowmax != rowmax) ? __builtin_nanf("") : fmaxf(m, rowmax);
    const float ref = mnew == -__builtin_inff() ? 0.0f : mnew;
    const float alpha = exp2f((m - ref) * LOG2E);
    l = l * alpha;
#pragma unroll 1
    for (int j = 0; j < n; ++j) {
      const float p = exp2f((ss[j][threadIdx.x] - ref) * LOG2E);
      l = l + p;
      ss[j][threadIdx.x] = round_to<T>(p);  // P narrowed to V's storage type for PV
    }
#pragma unroll
    for (int d = 0; d < SMALL_D; ++d) {
      if (d >= D) continue;
      float pv = 0.0f;
#pragma unroll 1
      for (int j = 0; j < n; ++j) pv = __builtin_fmaf(ss[j][threadIdx.x], sv[j][d], pv);
      acc[d] = acc[d] * alpha + pv;
    }
    m = mnew;
  }
  if (!live) return;
  const float coef = l == 0.0f ? 0.0f : 1.0f / l;
  uint16_t *orow = a.o + ((size_t)bh * a.q_len + i) * D;
#pragma unroll
  for (int d = 0; d < SMALL_D; ++d)
    if (d < D) orow[d] = __builtin_bit_cast(uint16_t, (T)f32_rounded(acc[d] * coef));
}

}  // namespace

// Shared by wafer_hip_attention_prefill (every case its BF16 / head_dim 128
// kernel does not serve) and wafer_hip_attention_prefill_masked.
int attention_prefill_masked(wafer_hip_context *ctx, uint32_t format, const void *q, const void *k, const void *v,
                             void *o, uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t q_len,
                             uint32_t kv_len, uint32_t head_dim, float scale, const wafer_hip_attention_mask *mask) {
  WAFER_CHECK_CTX(ctx);
  const char *W = "attention_prefill_masked: ";
  if (format != WAFER_FMT_BF16 && format != WAFER_FMT_F16)
    return fail(WAFER_HIP_E_UNSUPPORTED, std::string(W) + "storage must be BF16 or F16");
  if (!(head_dim == 128 || (head_dim >= 1 && head_dim <= 64)))
    return fail(WAFER_HIP_E_UNSUPPORTED, std::string(W) + "head_dim must be 128 or in [1, 64]");
  if (!q || !k || !v || !o) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(W) + "null tensor");
  if (batch == 0 || q_heads == 0 || kv_heads == 0 || q_len == 0 || kv_len == 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, std::string(W) + "empty dimension");
  if (q_heads % kv_heads != 0) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(W) + "q_heads % kv_heads != 0");
  if (!(scale > 0.0f) || scale == __builtin_inff())
    return fail(WAFER_HIP_E_INVALID_FIELD, std::string(W) + "scale must be positive and finite");
  const wafer_hip_attention_mask none{};
  const wafer_hip_attention_mask &m = mask ? *mask : none;
  const uint32_t known = WAFER_HIP_ATT_CAUSAL | WAFER_HIP_ATT_WINDOW | WAFER_HIP_ATT_ROUND_SCALED |
                         WAFER_HIP_ATT_ROUND_BIASED;
  if (m.flags & ~known) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(W) + "unknown flag bits");
  const uint32_t cap = m.kv_capacity ? m.kv_capacity : kv_len;
  if (cap < kv_len) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(W) + "kv_capacity < kv_len");
  if (cap > 0x7fffffffu) return fail(WAFER_HIP_E_UNSUPPORTED, std::string(W) + "kv_capacity too large");
  if ((m.flags & WAFER_HIP_ATT_WINDOW) && m.window < 1)
    return fail(WAFER_HIP_E_INVALID_FIELD, std::string(W) + "window must be >= 1");
  for (int s = 0; s < 3; ++s)
    if (m.bias_strides[s] < 0 || m.keep_strides[s] < 0)
      return fail(WAFER_HIP_E_INVALID_FIELD, std::string(W) + "mask strides must be >= 0");
  const uint64_t n_qblocks64 = (q_len + QB - 1) / QB;
  const uint64_t rows64 = (uint64_t)batch * q_heads;
  if (rows64 * ((n_qblocks64 + 1) / 2) > 0x7fffffffull || rows64 * ((q_len + SMALL_ROWS - 1) / SMALL_ROWS) > 0x7fffffffull)
    return fail(WAFER_HIP_E_INVALID_FIELD, std::string(W) + "grid too large");

  FaArgs args{};
  args.q = (const uint16_t *)q;
  args.k = (const uint16_t *)k;
  args.v = (const uint16_t *)v;
  args.o = (uint16_t *)o;
  args.q_heads = (int)q_heads;
  args.kv_heads = (int)kv_heads;
  args.q_len = (int)q_len;
  args.kv_len = (int)kv_len;
  args.kv_cap = (int)cap;
  args.c = scale * LOG2E;
  args.scale = scale;
  args.bh_count = (int)rows64;
  args.n_qblocks = (int)n_qblocks64;
  args.flags = m.flags;
  // The two key bounds j <= i + diag and j >= i + lo_off, each clamped to
  // [-(q_len + 1), kv_len + 1], which keeps its meaning for every row (an
  // offset at either end shows every key or none) and fits the kernels' int
  // arithmetic.
  const __int128 omin = -(__int128)q_len - 1, omax = (__int128)kv_len + 1;
  auto clamp_off = [&](__int128 x) { return (int)(x < omin ? omin : (x > omax ? omax : x)); };
  args.diag = clamp_off(m.causal_diagonal);
  if (m.flags & WAFER_HIP_ATT_WINDOW) args.lo_off = clamp_off((__int128)m.causal_diagonal - m.window + 1);
  args.bias = m.bias;
  args.bias_sb = m.bias_strides[0];
  args.bias_sh = m.bias_strides[1];
  args.bias_sq = m.bias_strides[2];
  args.keep = m.keep;
  args.keep_sb = m.keep_strides[0];
  args.keep_sh = m.keep_strides[1];
  args.keep_sq = m.keep_strides[2];
  const bool general = m.bias || m.keep || (m.flags & (WAFER_HIP_ATT_WINDOW | WAFER_HIP_ATT_ROUND_SCALED));
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const bool bf = format == WAFER_FMT_BF16;
  if (head_dim == 128 || head_dim == 64) {
    const dim3 grid((unsigned)(args.bh_count * ((args.n_qblocks + 1) / 2)));
#define FA_LAUNCH(TT, DD)                                                                              \
  do {                                                                                                 \
    if (general)                                                                                       \
      hipLaunchKernelGGL((fa_fwd<TT, DD, MASK_GENERAL>), grid, dim3(THREADS), 0, ctx->stream, args);   \
    else                                                                                               \
      hipLaunchKernelGGL((fa_fwd<TT, DD, MASK_CAUSAL>), grid, dim3(THREADS), 0, ctx->stream, args);    \
  } while (0)
    if (bf && head_dim == 128) FA_LAUNCH(__bf16, 128);
    else if (bf) FA_LAUNCH(__bf16, 64);
    else if (head_dim == 128) FA_LAUNCH(_Float16, 128);
    else FA_LAUNCH(_Float16, 64);
#undef FA_LAUNCH
    return launch_status("fa_fwd");
  }
  const int row_blocks = (int)((q_len + SMALL_ROWS - 1) / SMALL_ROWS);
  const dim3 grid((unsigned)(args.bh_count * row_blocks));
  if (bf)
    hipLaunchKernelGGL(fa_small<__bf16>, grid, dim3(SMALL_ROWS), 0, ctx->stream, args, (int)head_dim, row_blocks);
  else
    hipLaunchKernelGGL(fa_small<_Float16>, grid, dim3(SMALL_ROWS), 0, ctx->stream, args, (int)head_dim, row_blocks);
  return launch_status("fa_small");
}

}  // namespace wafer

extern "C" int wafer_hip_attention_prefill_masked(wafer_hip_context *ctx, uint32_t format, const void *q,
                                                  const void *k, const void *v, void *o, uint32_t batch,
                                                  uint32_t q_heads, uint32_t kv_heads, uint32_t q_len,
                                                  uint32_t kv_len, uint32_t head_dim, float scale,
                                                  const wafer_hip_attention_mask *mask) {
  return wafer::attention_prefill_masked(ctx, format, q, k, v, o, batch, q_heads, kv_heads, q_len, kv_len, head_dim,
                                         scale, mask);
}
