// fd_decode.hip -- FD flash-decoding for gfx950.
//
// Semantics: every KV chunk gets its own online-softmax state (the FA block
// update of OnlineAttentionDecomposition.cpp:568-597), the chunk states are
// folded left to right in contribution order
// (lib/Wafer/Transforms/Linalg/SpatialRegionMaterialization.cpp:2391-2430)
// with materializeOnlineAttentionStateMerge
// (lib/Wafer/Transforms/Linalg/OnlineAttentionMaterialization.cpp:264-373):
//   m = max(mL, mR), sL = ExpLp(mL - m), sR = ExpLp(mR - m),
//   l = lL*sL + lR*sR, acc = accL*sL + accR*sR,
// then finalised as FA: out = bf16(acc * (1/l)).  GQA: q head h reads kv
// head h / (q_heads / kv_heads).
//
// Mapping onto CDNA4 (the kernel is HBM-bound: every KV byte is read once):
//  * pass 1, grid (chunk, kv_head, batch), 4 waves per workgroup; each wave
//    sweeps a quarter of the chunk in 64-key blocks and serves all G query
//    heads of the GQA group from one read of K and V;
//  * Q.K^T on v_mfma_f32_16x16x32_bf16 with A = 16 keys x 32 d (each lane
//    loads 16 B; 4 lanes cover 64 contiguous bytes of a key row) and
//    B = Q^T padded to 16 head columns;
//  * P.V on the VALU with fully coalesced 128-bit V loads (16 lanes read one
//    256-byte key row), P broadcast through LDS, lane partials folded with
//    xor shuffles at the end of the sweep;
//  * the 4 wave states merge in key order through LDS into one chunk state
//    (acc[128], m, l per head) written to the context workspace;
//  * pass 2, one workgroup per (batch, q_head), folds the chunk states left to
//    right and writes the bf16 output.
// Scores are tracked in the log2 domain (m2 = m * scale * log2e) so every
// ExpLp becomes one exp2 of an fma; see fa_prefill.hip for the rounding note.
#include "common.h"

namespace wafer {
namespace {

constexpr int D = 128;
constexpr int WAVES = 4;
constexpr int BLK = 64;

struct ChunkState {  // per (batch, q_head, chunk), f32
  float acc[D];
  float m2;
  float l;
  float pad[2];
};

template <int G>
__global__ __launch_bounds__(256) void fd_chunk_bf16_d128(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ Kc,
    const uint16_t *__restrict__ Vc, ChunkState *__restrict__ part, int q_heads,
    int kv_heads, int kv_len, int cap, int chunk_len, int chunks,
    float scale_log2e) {
  __shared__ float sP[WAVES][BLK][G];
  __shared__ float sAlpha[WAVES][G];
  __shared__ float sAcc[WAVES][G][D];
  __shared__ float sM[WAVES][G], sL[WAVES][G];

  const int c = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane & 15, grp = lane >> 4;

  const int c0 = c * chunk_len;
  const int c1 = min(c0 + chunk_len, kv_len);
  const int n = max(c1 - c0, 0);
  const int per = ((n + WAVES * 16 - 1) / (WAVES * 16)) * 16;  // keys per wave
  const int w0 = c0 + wave * per;
  const int w1 = min(w0 + per, c1);
  const int nblk = (per + BLK - 1) / BLK;  // uniform over the workgroup

  const uint16_t *Kp = Kc + ((size_t)(b * kv_heads + kvh) * cap) * D;
  const uint16_t *Vp = Vc + ((size_t)(b * kv_heads + kvh) * cap) * D;

  // Q^T as MFMA B operand: column = head hl, d = s*32 + grp*8 + [0,8)
  bf16x8 qreg[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (hl < G)
      qreg[s] = *(const bf16x8 *)(Q + ((size_t)(b * q_heads + kvh * G + hl)) * D + s * 32 + grp * 8);
    else
      for (int e = 0; e < 8; ++e) qreg[s][e] = (__bf16)0.0f;
  }

  float m2 = -__builtin_inff();  // running max (log2 domain) for head hl
  float lsum = 0.0f;
  float acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;

  for (int blk = 0; blk < nblk; ++blk) {
    const int kbase = w0 + blk * BLK;
    // K: 4 groups of 16 keys; lane loads key kbase + gi*16 + hl, 4 x 16 B
    bf16x8 kreg[4][4];
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int key = kbase + gi * 16 + hl;
      const bool ok = key < w1;
      const uint16_t *kr = Kp + (size_t)(ok ? key : 0) * D + grp * 8;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        kreg[gi][s] = *(const bf16x8 *)(kr + s * 32);
        if (!ok)
          for (int e = 0; e < 8; ++e) kreg[gi][s][e] = (__bf16)0.0f;
      }
    }
    // V: lane loads keys kbase + grp + 4 i, d = hl*8 + [0,8)
    u32x4 vreg[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kbase + grp + 4 * i;
      const bool ok = key < w1;
      vreg[i] = *(const u32x4 *)(Vp + (size_t)(ok ? key : 0) * D + hl * 8);
      if (!ok) vreg[i] = u32x4{0u, 0u, 0u, 0u};
    }
    // S^T = K . Q^T : lane holds head hl, keys gi*16 + 4 grp + r
    f32x4 sacc[4];
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      sacc[gi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        sacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kreg[gi][s], qreg[s], sacc[gi], 0, 0, 0);
    }
    float mx = -__builtin_inff();
#pragma unroll
    for (int gi = 0; gi < 4; ++gi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kbase + gi * 16 + 4 * grp + r;
        if (key >= w1) sacc[gi][r] = -__builtin_inff();
        mx = fmaxf(mx, sacc[gi][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mx2 = (mx == -__builtin_inff()) ? mx : mx * scale_log2e;
    const float m2_new = fmaxf(m2, mx2);
    const float e2 = (m2_new == -__builtin_inff()) ? 0.0f : m2_new;
    const float alpha = __builtin_amdgcn_exp2f(m2 - e2);
    float rs = 0.0f;
#pragma unroll
    for (int gi = 0; gi < 4; ++gi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[gi][r], scale_log2e, -e2));
        rs += p;
        if (hl < G) sP[wave][gi * 16 + 4 * grp + r][hl] = (float)(__bf16)p;
      }
    rs += __shfl_xor(rs, 16);
    rs += __shfl_xor(rs, 32);
    lsum = lsum * alpha + rs;
    m2 = m2_new;
    if (grp == 0 && hl < G) sAlpha[wave][hl] = alpha;
    __syncthreads();
    float al[G];
#pragma unroll
    for (int h = 0; h < G; ++h) al[h] = sAlpha[wave][h];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] *= al[h];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float p[G];
#pragma unroll
      for (int h = 0; h < G; ++h) p[h] = sP[wave][grp + 4 * i][h];
      float vf[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        vf[2 * w] = u2f(vreg[i][w] << 16);
        vf[2 * w + 1] = u2f(vreg[i][w] & 0xffff0000u);
      }
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = __builtin_fmaf(p[h], vf[e], acc[h][e]);
    }
    __syncthreads();
  }

  // fold the four key-residue lane groups: lanes hl, hl+16, hl+32, hl+48
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[h][e];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[h][e] = v;
    }
  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) sAcc[wave][h][hl * 8 + e] = acc[h][e];
    if (hl < G) {
      sM[wave][hl] = m2;
      sL[wave][hl] = lsum;
    }
  }
  __syncthreads();

  // merge the wave states in key order; thread t handles (head t/D.., d t%D)
  for (int idx = tid; idx < G * D; idx += 256) {
    const int h = idx / D, d = idx % D;
    float sm = sM[0][h], sl = sL[0][h], sa = sAcc[0][h][d];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      const float mr = sM[w][h];
      const float m = fmaxf(sm, mr);
      const float e = (m == -__builtin_inff()) ? 0.0f : m;
      const float s_l = __builtin_amdgcn_exp2f(sm - e);
      const float s_r = __builtin_amdgcn_exp2f(mr - e);
      sl = sl * s_l + sL[w][h] * s_r;
      sa = sa * s_l + sAcc[w][h][d] * s_r;
      sm = m;
    }
    ChunkState &cs = part[((size_t)(b * q_heads + kvh * G + h)) * chunks + c];
    cs.acc[d] = sa;
    if (d == 0) {
      cs.m2 = sm;
      cs.l = sl;
    }
  }
}

// Left fold over the chunk states of one (batch, q_head), then finalize.
__global__ __launch_bounds__(128) void fd_combine_bf16_d128(const ChunkState *__restrict__ part,
                                                            uint16_t *__restrict__ O, int chunks) {
  const int bh = blockIdx.x, d = threadIdx.x;
  const ChunkState *ps = part + (size_t)bh * chunks;
  float m = ps[0].m2, l = ps[0].l, a = ps[0].acc[d];
  for (int c = 1; c < chunks; ++c) {
    const float mr = ps[c].m2;
    const float mm = fmaxf(m, mr);
    const float e = (mm == -__builtin_inff()) ? 0.0f : mm;
    const float sl = __builtin_amdgcn_exp2f(m - e);
    const float sr = __builtin_amdgcn_exp2f(mr - e);
    l = l * sl + ps[c].l * sr;
    a = a * sl + ps[c].acc[d] * sr;
    m = mm;
  }
  const float coef = (l == 0.0f) ? 0.0f : 1.0f / l;
  O[(size_t)bh * D + d] = f32_to_bf16(a * coef);
}

}  // namespace
}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_attention_decode(wafer_hip_context *ctx, uint32_t format,
                                          const void *q, const void *k_cache,
                                          const void *v_cache, void *o, uint32_t batch,
                                          uint32_t q_heads, uint32_t kv_heads,
                                          uint32_t kv_len, uint32_t kv_capacity,
                                          uint32_t head_dim, float scale, uint32_t chunks) {
  WAFER_CHECK_CTX(ctx);
  if (format != WAFER_FMT_BF16)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_decode: only BF16 storage is served");
  if (head_dim != D) return fail(WAFER_HIP_E_UNSUPPORTED, "attention_decode: head_dim must be 128");
  if (!q || !k_cache || !v_cache || !o)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode: null tensor");
  if (batch == 0 || q_heads == 0 || kv_heads == 0 || kv_len == 0 || chunks == 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode: empty dimension");
  if (q_heads % kv_heads != 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode: q_heads % kv_heads != 0");
  if (kv_len > kv_capacity)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode: kv_len > kv_capacity");
  if (chunks > 65535 || kv_heads > 65535 || batch > 65535)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode: grid dimension above 65535");
  if (!(scale > 0.0f)) return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode: scale must be positive");
  const uint32_t G = q_heads / kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_decode: q_heads/kv_heads must be 1, 2, 4 or 8");
  // The reference needs at least two K2 pieces for FD
  // (lib/Wafer/IR/LinalgExt/AttentionOps.cpp:439-450); one chunk is the FA
  // state and is served as well.
  const int chunk_len = (int)((kv_len + chunks - 1) / chunks);
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const size_t need = (size_t)batch * q_heads * chunks * sizeof(ChunkState);
  WAFER_TRY(ensure_workspace(ctx, &ctx->workspace, &ctx->workspace_bytes, need));
  auto *part = (ChunkState *)ctx->workspace;
  const float c = scale * 0x1.715476p+0f;
  dim3 grid(chunks, kv_heads, batch);
#define FD_LAUNCH(GV)                                                                          \
  hipLaunchKernelGGL(fd_chunk_bf16_d128<GV>, grid, dim3(256), 0, ctx->stream,                \
                     (const uint16_t *)q, (const uint16_t *)k_cache, (const uint16_t *)v_cache, \
                     part, (int)q_heads, (int)kv_heads, (int)kv_len, (int)kv_capacity,       \
                     chunk_len, (int)chunks, c)
  switch (G) {
  case 1: FD_LAUNCH(1); break;
  case 2: FD_LAUNCH(2); break;
  case 4: FD_LAUNCH(4); break;
  default: FD_LAUNCH(8); break;
  }
#undef FD_LAUNCH
  WAFER_TRY(launch_status("fd_chunk_bf16_d128"));
  hipLaunchKernelGGL(fd_combine_bf16_d128, dim3(batch * q_heads), dim3(D), 0, ctx->stream,
                     part, (uint16_t *)o, (int)chunks);
  return launch_status("fd_combine_bf16_d128");
}
