// fa_prefill.hip -- FA flash-attention prefill for gfx950.
//
// Semantics: the compiler's online-attention decomposition
// (lib/Wafer/Transforms/Linalg/OnlineAttentionDecomposition.cpp:568-597; QK
// :242-277, score region :279-426, PV :509-566; finalize
// lib/Wafer/Transforms/Linalg/OnlineAttentionMaterialization.cpp:197-262):
//   per KV block: S = q.k (f32 accumulate), S = S*scale (+0/-inf causal bias),
//   m' = max(m, rowmax S), alpha = ExpLp(m - m'), P = ExpLp(S - m'),
//   l = l*alpha + rowsum(P) (unrounded P), acc = acc*alpha + bf16(P).V,
//   out = bf16(acc * (1/l)), 0 for a row with l == 0.
// The two partial states of interleaved key sets combine with the state
// merge of OnlineAttentionMaterialization.cpp:264-373: m = max(mL, mR),
// sL = ExpLp(mL - m), sR = ExpLp(mR - m), l = lL sL + lR sR,
// acc = accL sL + accR sR.
//
// Mapping onto CDNA4:
//  * a workgroup (8 waves) serves two 64-query blocks of one (batch, head):
//    block i and block n-1-i of the causal triangle, so every workgroup does
//    the same amount of work (i+1 + n-i key blocks) and one launch of
//    heads*n/2 workgroups fills the CUs evenly with no cross-workgroup merge;
//  * wave w: group g = w>>2 (0: the late block, 1: the early block), query
//    tile w&1 (32 queries), key half (w>>1)&1.  The two key halves sweep the
//    even and the odd 64-key blocks; each SIMD holds one late-block and one
//    early-block wave, so all SIMDs carry equal work and one wave's softmax
//    VALU work overlaps the other's MFMAs;
//  * scores are computed transposed, S^T = K . Q^T, on
//    v_mfma_f32_32x32x16_bf16 (A = 32 keys x 16 d from LDS, B = Q^T kept in
//    VGPRs), so each lane's accumulator column is one query: row max / sum /
//    alpha are lane-local plus one xor-32 exchange;
//  * the output is accumulated transposed as well, O^T = V^T . P^T: the
//    rescale by alpha is lane-local and P^T feeds the MFMA B operand from the
//    score registers after RNE narrowing (v_cvt_pk_bf16_f32).  The rescale is
//    skipped when alpha == 1 for the whole wave (x * 1 == x exactly);
//  * K tiles sit row-major in LDS, V tiles transposed (d-major) with keys
//    permuted inside every 16-key group so the 8 keys one lane needs for one
//    MFMA are contiguous (one ds_read_b128); per key half double-buffered in
//    LDS and staged global -> VGPR two iterations ahead; both query blocks of a
//    workgroup read the same tiles for their common key prefix;
//  * consecutive workgroup ids walk (batch*head), so each head's workgroups
//    land on one XCD (ids are dealt round-robin over the 8 XCDs) and share
//    its L2.
//
// Arithmetic note: ExpLp(S*scale - m) is evaluated as
// exp2(fma(s_raw, scale*log2e, -m_raw*scale*log2e)) (one rounding fewer than
// the reference's mul, sub, mul chain); the difference is below 1 ulp of the
// f32 argument and far inside the attention tolerance.
#include "common.h"

#include <type_traits>

namespace wafer {
namespace {

constexpr int D = 128;
constexpr int QB = 64;            // queries per query block
constexpr int BK = 64;            // keys per KV block
constexpr int KPITCH = D + 8;     // LDS row pitch of K tiles (elements): 272 B
constexpr int VPITCH = BK + 8;    // LDS row pitch of V^T tiles (elements): 144 B
constexpr int THREADS = 512;

// Lazy rescaling: the exponentials use a reference max that moves only when
// some row's running max exceeds it by more than 2^RESCALE_LOG2 (P <= 2^8).
constexpr float RESCALE_LOG2 = 8.0f;

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

// V^T LDS column p of a 64-key block holds key swap23(p): bits 2 and 3 of
// the key index swapped, so the 8 keys one lane feeds into one PV MFMA are
// contiguous (the 32x32 accumulator layout puts rows 8(r/4) + 4g + r%4 in a
// lane) and one ds_read_b128 fetches them.
__device__ inline int swap23(int p) { return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1); }

template <bool CAUSAL>
__global__ __launch_bounds__(THREADS) void fa_prefill_bf16_d128(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K,
    const uint16_t *__restrict__ V, uint16_t *__restrict__ O, int q_heads, int kv_heads,
    int q_len, int kv_len, float c, int bh_count, int n_qblocks) {
  __shared__ __align__(16) uint16_t sK[2][2][BK * KPITCH];  // [half][buf]
  __shared__ __align__(16) uint16_t sV[2][2][D * VPITCH];

  const int bid = blockIdx.x;
  const int pair = bid / bh_count;
  const int bh = bid - pair * bh_count;
  const int b = bh / q_heads;
  const int h = bh - b * q_heads;
  const int kvh = h / (q_heads / kv_heads);
  const uint16_t *Qp = Q + ((size_t)bh * q_len) * D;
  const uint16_t *Kp = K + ((size_t)(b * kv_heads + kvh) * kv_len) * D;
  const uint16_t *Vp = V + ((size_t)(b * kv_heads + kvh) * kv_len) * D;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = wave >> 2, tile = wave & 1, half = (wave >> 1) & 1;
  const int l32 = lane & 31, g = lane >> 5;
  // causal: pair the early block `pair` with the late block n-1-pair
  const int qb_lo = CAUSAL ? pair : 2 * pair;
  const int qb_hi = CAUSAL ? n_qblocks - 1 - pair : 2 * pair + 1;
  const int qb = grp == 0 ? qb_hi : qb_lo;
  const int q0 = qb * QB + tile * 32;
  const int my_q = q0 + l32;
  const int kv_blocks = kv_len / BK;
  const int nk_hi = CAUSAL ? min(kv_blocks, qb_hi + 1) : kv_blocks;
  const int nk_mine = CAUSAL ? min(kv_blocks, qb + 1) : kv_blocks;

  // Q^T as the MFMA B operand: lane holds query l32, d = s*16 + g*8 + [0,8).
  bf16x8 qreg[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
    qreg[s] = *(const bf16x8 *)(Qp + (size_t)my_q * D + s * 16 + g * 8);
  // (the Q loads are drained in the prologue below, together with the first
  // K/V block: without an explicit drain the waitcnt pass ties Q's registers
  // to the in-loop prefetch loads and stalls every iteration on them)

  // global -> VGPR staging: the 4 waves of a key half load that half's
  // block (K: 16 lanes per 256-byte key row; V: 4 consecutive keys per lane,
  // so the V^T stores of 16 lanes fill one 128-byte LDS row segment without
  // bank conflicts).  Two register slots keep the loads two iterations ahead
  // of their use.
  const int ltid = (((wave & 1) | ((wave >> 2) << 1)) << 6) | lane;  // 0..255 within the half
  const int k_row = ltid >> 4, k_col = (ltid & 15) * 8;               // rows k_row + 16 i
  const int v_kg = ltid & 15, v_dc = ltid >> 4;                       // keys 4 v_kg + i, d 8 v_dc
  const int v_pos = swap23(4 * v_kg);
  u32x4 kst[2][4], vst[2][4];
  auto gload = [&](int kb, auto slot) __attribute__((always_inline)) {
    const uint16_t *kp = Kp + (size_t)(kb * BK) * D;
    const uint16_t *vp = Vp + (size_t)(kb * BK) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      kst[slot][i] = *(const u32x4 *)(kp + (size_t)(k_row + 16 * i) * D + k_col);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vst[slot][i] = *(const u32x4 *)(vp + (size_t)(4 * v_kg + i) * D + 8 * v_dc);
  };
  auto sstore = [&](int buf, auto slot) __attribute__((always_inline)) {
    uint16_t *sk = sK[half][buf];
    uint16_t *sv = sV[half][buf];
#pragma unroll
    for (int i = 0; i < 4; ++i) *(u32x4 *)&sk[(k_row + 16 * i) * KPITCH + k_col] = kst[slot][i];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t a0 = vst[slot][0][w], a1 = vst[slot][1][w], a2 = vst[slot][2][w], a3 = vst[slot][3][w];
      u32x2 lo, hi;
      lo[0] = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
      lo[1] = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
      hi[0] = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
      hi[1] = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
      *(u32x2 *)&sv[(8 * v_dc + 2 * w) * VPITCH + v_pos] = lo;
      *(u32x2 *)&sv[(8 * v_dc + 2 * w + 1) * VPITCH + v_pos] = hi;
    }
  };

  // running max of the raw scores, the reference max the exponentials use
  // (and its scaled value, 0 while the reference is -inf), and the sum of P
  float m_run = -__builtin_inff(), m_ref = -__builtin_inff(), mc_ref = 0.0f;
  float l_sum = 0.0f;
  f32x16 acc_o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[dt][r] = 0.0f;

  // one 64-key block: S^T = K.Q^T, online-softmax update, O^T += V^T.P^T
  auto compute = [&](int kb, const uint16_t *sk, const uint16_t *sv) __attribute__((always_inline)) {
    f32x16 sacc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[t][r] = 0.0f;
    // the two key tiles alternate so consecutive MFMAs are independent
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8 a = *(const bf16x8 *)&sk[(t * 32 + l32) * KPITCH + s * 16 + g * 8];
        sacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[s], sacc[t], 0, 0, 0);
      }
    if (CAUSAL && kb * BK + BK - 1 > q0) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * BK + t * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key > my_q) sacc[t][r] = -__builtin_inff();
        }
    }
    float mx = sacc[0][0];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[t][r]);
    mx = xor32_max(mx);
    const float m_new = fmaxf(m_run, mx);
    m_run = m_new;
    // move the reference max (and rescale acc and l by alpha) only when a
    // row's running max has grown by more than 2^RESCALE_LOG2 over it
    const bool grow = m_new != -__builtin_inff() &&
                      (m_ref == -__builtin_inff() || m_new * c > mc_ref + RESCALE_LOG2);
    if (__any(grow)) {
      const float mc = (m_new == -__builtin_inff()) ? 0.0f : m_new * c;
      const float alpha = (m_ref == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(mc_ref - mc);
      l_sum *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha;
      m_ref = m_new;
      mc_ref = mc;
    }
    float rs = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[t][r], c, -mc_ref));
        sacc[t][r] = p;
        rs += p;
      }
    l_sum += xor32_sum(rs);
    // P^T operands: (t, hf) covers S^T rows t*32 + hf*16 + [0,16); the
    // lane's 8 values are accumulator rows hf*8 + [0,8) of tile t.
    bf16x8 pb[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[t][hf][e] = (__bf16)sacc[t][hf * 8 + e];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const bf16x8 va = *(const bf16x8 *)&sv[(dt * 32 + l32) * VPITCH + t * 32 + hf * 16 + g * 8];
          acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[t][hf], acc_o[dt], 0, 0, 0);
        }
  };

  // Pipeline (per key half; iteration i works on block 2 i + half):
  //   LDS buffer i%2 holds iteration i's block; register slot (i+1)%2 holds
  //   iteration i+1's block, loaded one iteration earlier; iteration i loads
  //   iteration i+2's block into slot i%2, computes, stores slot (i+1)%2 into
  //   LDS buffer (i+1)%2, and meets the other waves at one barrier.  Loads
  //   and stores are unconditional (block index clamped to the last block)
  //   so the waitcnt pass counts them exactly and waits only for the older
  //   slot.
  const int niter = (nk_hi + 1) / 2;
  const int last = nk_hi - 1;
  gload(min(half, last), std::integral_constant<int, 0>{});
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): Q and the first block
  sstore(0, std::integral_constant<int, 0>{});
  gload(min(half + 2, last), std::integral_constant<int, 1>{});
  __syncthreads();

  auto step = [&](int i, auto slot) __attribute__((always_inline)) {
    constexpr int P = decltype(slot)::value;  // == i % 2
    const int kb = 2 * i + half;
    gload(min(kb + 4, last), std::integral_constant<int, P>{});
    const bool active = (kb < nk_mine) && (!CAUSAL || kb * BK <= q0 + 31);
    if (active) compute(kb, sK[half][P], sV[half][P]);
    if (i + 1 < niter) {
      sstore(P ^ 1, std::integral_constant<int, P ^ 1>{});
      __syncthreads();
    }
  };
  for (int i = 0; i < niter; i += 2) {
    step(i, std::integral_constant<int, 0>{});
    if (i + 1 < niter) step(i + 1, std::integral_constant<int, 1>{});
  }

  // ---- merge the odd-block half into the even-block half through LDS ----
  __syncthreads();
  float *xacc = (float *)&sK[0][0][0];  // [grp*2+tile][dt][r][lane], 64 KiB
  float *xml = (float *)&sV[0][0][0];   // m [slot][lane], l [slot][lane]
  const int slot = grp * 2 + tile;
  if (half == 1) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) xacc[((slot * 4 + dt) * 16 + r) * 64 + lane] = acc_o[dt][r];
    xml[slot * 64 + lane] = m_ref;
    xml[256 + slot * 64 + lane] = l_sum;
  }
  __syncthreads();
  if (half == 1) return;
  {
    // each state is (acc, l) relative to its reference max
    const float m1 = xml[slot * 64 + lane], l1 = xml[256 + slot * 64 + lane];
    const float m = fmaxf(m_ref, m1);
    const float e = (m == -__builtin_inff()) ? 0.0f : m * c;
    const float s0 = (m_ref == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(m_ref * c - e);
    const float s1 = (m1 == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(m1 * c - e);
    l_sum = l_sum * s0 + l1 * s1;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc_o[dt][r] = acc_o[dt][r] * s0 + xacc[((slot * 4 + dt) * 16 + r) * 64 + lane] * s1;
  }

  // finalize: coefficient = Recip(l) (0 for an empty row), out = bf16(acc * coef)
  const float coef = (l_sum == 0.0f) ? 0.0f : 1.0f / l_sum;
  uint16_t *orow = O + ((size_t)bh * q_len + my_q) * D;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      u32x2 packed;
      packed[0] = (uint32_t)f32_to_bf16(acc_o[dt][4 * rq + 0] * coef) |
                  ((uint32_t)f32_to_bf16(acc_o[dt][4 * rq + 1] * coef) << 16);
      packed[1] = (uint32_t)f32_to_bf16(acc_o[dt][4 * rq + 2] * coef) |
                  ((uint32_t)f32_to_bf16(acc_o[dt][4 * rq + 3] * coef) << 16);
      *(u32x2 *)(orow + dt * 32 + 8 * rq + 4 * g) = packed;
    }
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
  if (format != WAFER_FMT_BF16)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_prefill: only BF16 storage is served");
  if (head_dim != D)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_prefill: head_dim must be 128");
  if (!q || !k || !v || !o) return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: null tensor");
  if (batch == 0 || q_heads == 0 || kv_heads == 0 || q_len == 0 || kv_len == 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: empty dimension");
  if (q_heads % kv_heads != 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: q_heads % kv_heads != 0");
  if (q_len % (2 * QB) != 0 || kv_len % BK != 0)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_prefill: q_len must be a multiple of 128 and kv_len of 64");
  if (causal && kv_len < q_len)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_prefill: causal needs kv_len >= q_len");
  if (!(scale > 0.0f)) return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: scale must be positive");
  if ((uint64_t)batch * q_heads * (q_len / (2 * QB)) > 0x7fffffffull)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: grid too large");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const int n_qblocks = (int)(q_len / QB);
  const int bh_count = (int)(batch * q_heads);
  const float c = scale * 0x1.715476p+0f;
  dim3 grid((unsigned)(bh_count * (n_qblocks / 2)));
  if (causal)
    hipLaunchKernelGGL(fa_prefill_bf16_d128<true>, grid, dim3(THREADS), 0, ctx->stream,
                       (const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)v, (uint16_t *)o,
                       (int)q_heads, (int)kv_heads, (int)q_len, (int)kv_len, c, bh_count, n_qblocks);
  else
    hipLaunchKernelGGL(fa_prefill_bf16_d128<false>, grid, dim3(THREADS), 0, ctx->stream,
                       (const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)v, (uint16_t *)o,
                       (int)q_heads, (int)kv_heads, (int)q_len, (int)kv_len, c, bh_count, n_qblocks);
  return launch_status("fa_prefill_bf16_d128");
}
