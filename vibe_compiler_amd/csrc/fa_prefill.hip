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
//
// Mapping onto CDNA4:
//  * one workgroup = 4 waves = 128 queries of one (batch, head); each wave owns
//    32 queries for the whole KV sweep;
//  * scores are computed transposed, S^T = K . Q^T with
//    v_mfma_f32_32x32x16_bf16 (A = 32 keys x 16 d from LDS, B = Q^T held in
//    VGPRs for the whole sweep), so each lane's accumulator column is one
//    query: row max / row sum / alpha are lane-local plus one xor-32 exchange;
//  * the output is accumulated transposed too, O^T = V^T . P^T, so the
//    rescale by alpha is lane-local and P^T feeds the MFMA B operand straight
//    from the score registers (after RNE narrowing to bf16);
//  * K tiles sit row-major in LDS, V tiles transposed (d-major) with keys
//    permuted inside every 16-key group so that the 8 keys one lane needs for
//    one MFMA are contiguous (one ds_read_b128); both are double-buffered and
//    staged global -> VGPR -> LDS one block ahead;
//  * causal: blocks past a wave's last query are skipped, diagonal blocks are
//    masked; workgroups are issued longest-first, and consecutive workgroup
//    ids walk (batch, head) so each head's blocks land on one XCD (ids are
//    dealt round-robin over the 8 XCDs) and share that XCD's L2.
//
// Arithmetic note: ExpLp(S*scale - m) is evaluated as
// exp2(fma(s_raw, scale*log2e, -m_raw*scale*log2e)) (one rounding fewer than
// the reference's mul, sub, mul chain); the difference is below 1 ulp of the
// f32 argument and far inside the attention tolerance.
#include "common.h"

namespace wafer {
namespace {

constexpr int D = 128;
constexpr int BQ = 128;           // queries per workgroup
constexpr int BK = 64;            // keys per pipeline stage
constexpr int KPITCH = D + 8;     // LDS row pitch of K tiles (elements): 272 B
constexpr int VPITCH = BK + 8;    // LDS row pitch of V^T tiles (elements): 144 B

__device__ inline int permute_key(int key) {
  // swap bits 2 and 3 of the key index inside its 16-key group
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

template <bool CAUSAL>
__global__ __launch_bounds__(256) void fa_prefill_bf16_d128(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K,
    const uint16_t *__restrict__ V, uint16_t *__restrict__ O, int q_heads,
    int kv_heads, int q_len, int kv_len, float scale_log2e, int n_qblocks,
    int bh_count) {
  __shared__ __align__(16) uint16_t sK[2][BK * KPITCH];
  __shared__ __align__(16) uint16_t sV[2][D * VPITCH];

  const int bid = blockIdx.x;
  const int rank = bid / bh_count;
  const int bh = bid - rank * bh_count;
  const int qb = CAUSAL ? (n_qblocks - 1 - rank) : rank;
  const int b = bh / q_heads;
  const int h = bh - b * q_heads;
  const int kvh = h / (q_heads / kv_heads);

  const uint16_t *Qp = Q + ((size_t)(b * q_heads + h) * q_len) * D;
  const uint16_t *Kp = K + ((size_t)(b * kv_heads + kvh) * kv_len) * D;
  const uint16_t *Vp = V + ((size_t)(b * kv_heads + kvh) * kv_len) * D;
  uint16_t *Op = O + ((size_t)(b * q_heads + h) * q_len) * D;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int q0 = qb * BQ + wave * 32;
  const int my_q = q0 + l32;

  // Q^T as the MFMA B operand: lane holds query l32, d = s*16 + g*8 + [0,8).
  bf16x8 qreg[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
    qreg[s] = *(const bf16x8 *)(Qp + (size_t)my_q * D + s * 16 + g * 8);

  int kv_end = kv_len;
  if (CAUSAL) kv_end = min(kv_len, (qb + 1) * BQ);
  const int nkb = (kv_end + BK - 1) / BK;

  // global -> VGPR staging coordinates
  const int k_row = tid >> 4, k_col = (tid & 15) * 8;   // rows k_row + 16 i
  const int v_kg = tid & 15, v_dc = tid >> 4;           // keys 4 v_kg + i, d 8 v_dc
  const int v_pos = permute_key(4 * v_kg);
  u32x4 kst[4], vst[4];

  auto gload = [&](int kb) {
    const uint16_t *kp = Kp + (size_t)(kb * BK) * D;
    const uint16_t *vp = Vp + (size_t)(kb * BK) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      kst[i] = *(const u32x4 *)(kp + (size_t)(k_row + 16 * i) * D + k_col);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vst[i] = *(const u32x4 *)(vp + (size_t)(4 * v_kg + i) * D + 8 * v_dc);
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *(u32x4 *)&sK[buf][(k_row + 16 * i) * KPITCH + k_col] = kst[i];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t a0 = vst[0][w], a1 = vst[1][w], a2 = vst[2][w], a3 = vst[3][w];
      u32x2 lo, hi;
      lo[0] = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
      lo[1] = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
      hi[0] = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
      hi[1] = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
      *(u32x2 *)&sV[buf][(8 * v_dc + 2 * w) * VPITCH + v_pos] = lo;
      *(u32x2 *)&sV[buf][(8 * v_dc + 2 * w + 1) * VPITCH + v_pos] = hi;
    }
  };

  float m_raw = -__builtin_inff();
  float l_sum = 0.0f;
  f32x16 acc_o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[dt][r] = 0.0f;

  gload(0);
  sstore(0);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nkb) gload(kb + 1);
    const bool active = !CAUSAL || (kb * BK <= q0 + 31);
    if (active) {
      f32x16 sacc[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[t][r] = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const bf16x8 a = *(const bf16x8 *)&sK[buf][(t * 32 + l32) * KPITCH + s * 16 + g * 8];
          sacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[s], sacc[t], 0, 0, 0);
        }
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
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_raw, mx);
      const float mc = (m_new == -__builtin_inff()) ? 0.0f : m_new * scale_log2e;
      const float alpha = __builtin_amdgcn_exp2f(m_raw * scale_log2e - mc);
      float rs = 0.0f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[t][r], scale_log2e, -mc));
          sacc[t][r] = p;
          rs += p;
        }
      rs += __shfl_xor(rs, 32);
      l_sum = l_sum * alpha + rs;
      m_raw = m_new;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha;
      // P^T operands: (t, half) covers keys t*32 + half*16 + [0,16); lane's 8
      // keys are accumulator rows half*8 + [0,8) of tile t.
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
            const bf16x8 va = *(const bf16x8 *)&sV[buf][(dt * 32 + l32) * VPITCH + t * 32 + hf * 16 + g * 8];
            acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[t][hf], acc_o[dt], 0, 0, 0);
          }
    }
    if (kb + 1 < nkb) {
      sstore(buf ^ 1);
      __syncthreads();
    }
  }

  // finalize: coefficient = Recip(l) (0 for an empty row), out = bf16(acc * coef)
  const float coef = (l_sum == 0.0f) ? 0.0f : 1.0f / l_sum;
  uint16_t *orow = Op + (size_t)my_q * D;
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
  if (q_len % BQ != 0 || kv_len % BK != 0)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_prefill: q_len must be a multiple of 128 and kv_len of 64");
  if (causal && kv_len < q_len)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_prefill: causal needs kv_len >= q_len");
  if (!(scale > 0.0f)) return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: scale must be positive");
  if ((uint64_t)batch * q_heads * (q_len / BQ) > 0x7fffffffull)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_prefill: grid too large");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const int n_qblocks = (int)(q_len / BQ);
  const int bh_count = (int)(batch * q_heads);
  const float c = scale * 0x1.715476p+0f;
  dim3 grid((unsigned)(n_qblocks * bh_count));
  if (causal)
    hipLaunchKernelGGL(fa_prefill_bf16_d128<true>, grid, dim3(256), 0, ctx->stream,
                       (const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)v,
                       (uint16_t *)o, (int)q_heads, (int)kv_heads, (int)q_len, (int)kv_len,
                       c, n_qblocks, bh_count);
  else
    hipLaunchKernelGGL(fa_prefill_bf16_d128<false>, grid, dim3(256), 0, ctx->stream,
                       (const uint16_t *)q, (const uint16_t *)k, (const uint16_t *)v,
                       (uint16_t *)o, (int)q_heads, (int)kv_heads, (int)q_len, (int)kv_len,
                       c, n_qblocks, bh_count);
  return launch_status("fa_prefill_bf16_d128");
}
