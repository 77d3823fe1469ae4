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
// then finalised as FA: out = narrow(acc * (1/l)) to the BF16 or F16 storage.  GQA: q head h reads kv
// head h / (q_heads / kv_heads).
//
// The kernel is HBM-bound (every KV byte is read once, 4 B of traffic per
// 4 FLOP), so the design goal is coalesced 128-bit streaming with enough
// bytes in flight, and a GQA group's query heads served from one read:
//  * Q.K^T on v_mfma_f32_16x16x32_{bf16,f16} with A = 16 keys x 32 d (each lane
//    loads 16 B; 4 lanes cover 64 contiguous bytes of a key row) and
//    B = Q^T padded to 16 head columns; scores land one head per lane column;
//  * P.V on the VALU with fully coalesced 128-bit V loads (16 lanes read one
//    256-byte key row), P passed through a wave-private LDS slice, alpha
//    broadcast with v_readlane, lane partials folded with xor shuffles at the
//    end of the sweep;
//  * large batches (batch*kv_heads >= 3/4 of the CUs, chunks <= 16, GQA
//    group <= 4): one
//    workgroup of 16 waves per (batch, kv_head); the chunks are split over
//    the waves (one wave per chunk at 16 chunks) and the wave states are
//    folded left to right through LDS, so there is a single launch and no
//    cross-workgroup traffic;
//  * small batches: a grid of (chunk, kv_head, batch) workgroups writes chunk
//    states to the context workspace and a second launch folds them.
// Scores are tracked in the log2 domain (m2 = m * scale * log2e) so every
// ExpLp becomes one exp2 of an fma; see fa_prefill.hip for the rounding note.
#include "common.h"

#include <mutex>
#include <type_traits>

namespace wafer {
namespace {

constexpr int D = 128;
constexpr int BLK = 32;  // keys per wave step

// storage type T (__bf16 or _Float16): 8-element operand vectors, the
// 16x16x32 MFMA, RNE narrowing and the widening of 8 packed values
template <typename T>
using v8 = std::conditional_t<std::is_same_v<T, __bf16>, bf16x8, f16x8>;
template <typename T>
__device__ inline f32x4 mfma16(v8<T> a, v8<T> b, f32x4 c) {
  if constexpr (std::is_same_v<T, __bf16>)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
template <typename T>
__device__ inline uint16_t narrow(float x) {
  return __builtin_bit_cast(uint16_t, (T)f32_rounded(x));
}
// element e of 8 packed storage values, widened (exact); for F16 the
// conversion folds into v_fma_mix_f32 at its use.  (The F16 half is taken
// by shift and mask: an extract from a bit-cast <2 x half> of one vector
// element was folded onto element 0 of the vector for every e.)
template <typename T>
__device__ inline float elem8(u32x4 w, int e) {
  const uint32_t x = w[e >> 1];
  if constexpr (std::is_same_v<T, __bf16>) {
    return (e & 1) ? u2f(x & 0xffff0000u) : u2f(x << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)((e & 1) ? (x >> 16) : (x & 0xffffu)));
  }
}

struct ChunkState {  // per (batch, q_head, chunk), f32
  float acc[D];
  float m2;
  float l;
  float pad[2];
};

__device__ inline void wave_lds_order() {
  // orders this wave's LDS writes before its later LDS reads (and back)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Online state of one wave over keys [k0, k1), for the G query heads of a
// GQA group.  On return, lanes with grp == 0 hold acc[h][hl*8 + e]; every
// lane holds m2 / l of head (lane & 15) (meaningful for heads < G).
template <typename T, int G>
struct WaveSweep {
  float m2, lsum;
  float acc[G][8];

  __device__ void run(const uint16_t *__restrict__ Kp, const uint16_t *__restrict__ Vp,
                      const v8<T> (&qreg)[4], int k0, int k1, int nblk, float c,
                      float (*sP)[G]) {
    const int lane = threadIdx.x & 63, hl = lane & 15, grp = lane >> 4;
    m2 = -__builtin_inff();
    lsum = 0.0f;
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
    for (int blk = 0; blk < nblk; ++blk) {
      const int kbase = k0 + blk * BLK;
      // K: 2 groups of 16 keys; lane loads key kbase + gi*16 + hl, 4 x 16 B.
      // The cache is read once, so its loads are non-temporal (no L2
      // allocation for data nothing reads again: config 2 183.7 -> 167.9 us,
      // 73 -> 80 % of HBM peak)
      v8<T> kreg[2][4];
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const int key = kbase + gi * 16 + hl;
        const bool ok = key < k1;
        const uint16_t *kr = Kp + (size_t)(ok ? key : 0) * D + grp * 8;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          kreg[gi][s] = __builtin_nontemporal_load((const v8<T> *)(kr + s * 32));
          if (!ok)
            for (int e = 0; e < 8; ++e) kreg[gi][s][e] = (T)0.0f;
        }
      }
      // V: lane loads keys kbase + grp + 4 i, d = hl*8 + [0,8)
      u32x4 vreg[BLK / 4];
#pragma unroll
      for (int i = 0; i < BLK / 4; ++i) {
        const int key = kbase + grp + 4 * i;
        const bool ok = key < k1;
        vreg[i] = __builtin_nontemporal_load((const u32x4 *)(Vp + (size_t)(ok ? key : 0) * D + hl * 8));
        if (!ok) vreg[i] = u32x4{0u, 0u, 0u, 0u};
      }
      // S^T = K . Q^T : lane holds head hl, keys gi*16 + 4 grp + r
      f32x4 sacc[2];
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        sacc[gi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
          sacc[gi] = mfma16<T>(kreg[gi][s], qreg[s], sacc[gi]);
      }
      float mx = -__builtin_inff();
#pragma unroll
      for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kbase + gi * 16 + 4 * grp + r;
          if (key >= k1) sacc[gi][r] = -__builtin_inff();
          mx = fmaxf(mx, sacc[gi][r]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mx2 = (mx == -__builtin_inff()) ? mx : mx * c;
      const float m2_new = fmaxf(m2, mx2);
      const float e2 = (m2_new == -__builtin_inff()) ? 0.0f : m2_new;
      const float alpha = __builtin_amdgcn_exp2f(m2 - e2);
      float rs = 0.0f;
#pragma unroll
      for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[gi][r], c, -e2));
          rs += p;
          if (hl < G) sP[gi * 16 + 4 * grp + r][hl] = (float)(T)f32_rounded(p);
        }
      rs += __shfl_xor(rs, 16);
      rs += __shfl_xor(rs, 32);
      lsum = lsum * alpha + rs;
      m2 = m2_new;
      wave_lds_order();
      float al[G];
#pragma unroll
      for (int h = 0; h < G; ++h)
        al[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), h));
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] *= al[h];
#pragma unroll
      for (int i = 0; i < BLK / 4; ++i) {
        float p[G];
#pragma unroll
        for (int h = 0; h < G; ++h) p[h] = sP[grp + 4 * i][h];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] = __builtin_fmaf(p[h], elem8<T>(vreg[i], e), acc[h][e]);
      }
      wave_lds_order();  // the next block's writes to sP follow these reads
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
  }
};

__device__ inline void merge(float &m, float &l, float &a, float mr, float lr, float ar) {
  const float mm = fmaxf(m, mr);
  const float e = (mm == -__builtin_inff()) ? 0.0f : mm;
  const float sl = __builtin_amdgcn_exp2f(m - e);
  const float sr = __builtin_amdgcn_exp2f(mr - e);
  l = l * sl + lr * sr;
  a = a * sl + ar * sr;
  m = mm;
}

template <typename T>
__device__ inline void load_q(const uint16_t *__restrict__ Q, int row_base, int G, v8<T> (&qreg)[4]) {
  const int lane = threadIdx.x & 63, hl = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (hl < G)
      qreg[s] = *(const v8<T> *)(Q + ((size_t)(row_base + hl)) * D + s * 32 + grp * 8);
    else
      for (int e = 0; e < 8; ++e) qreg[s][e] = (T)0.0f;
  }
}

template <typename T, int G>
__device__ inline void publish_state(const WaveSweep<T, G> &st, int wave, float (*sAcc)[G][D],
                                     float (*sM)[G], float (*sL)[G]) {
  const int lane = threadIdx.x & 63, hl = lane & 15, grp = lane >> 4;
  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) sAcc[wave][h][hl * 8 + e] = st.acc[h][e];
    if (hl < G) {
      sM[wave][hl] = st.m2;
      sL[wave][hl] = st.lsum;
    }
  }
}

// ---- one workgroup (16 waves) per (batch, kv_head) ----------------------------
constexpr int WG_WAVES = 16;

template <typename T, int G>
__global__ __launch_bounds__(1024) void fd_group_d128(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ Kc,
    const uint16_t *__restrict__ Vc, uint16_t *__restrict__ O, int q_heads, int kv_heads,
    int kv_len, int cap, int chunks, int chunk_len, int sub, float c) {
  __shared__ float sP[WG_WAVES][BLK][G];
  __shared__ float sAcc[WG_WAVES][G][D];
  __shared__ float sM[WG_WAVES][G], sL[WG_WAVES][G];

  const int kvh = blockIdx.x, b = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const uint16_t *Kp = Kc + ((size_t)(b * kv_heads + kvh) * cap) * D;
  const uint16_t *Vp = Vc + ((size_t)(b * kv_heads + kvh) * cap) * D;
  const int row_base = b * q_heads + kvh * G;

  // wave -> (chunk, contiguous part of the chunk); waves past chunks*sub idle
  const int chunk = wave / sub, part = wave - chunk * sub;
  const int per = (((chunk_len + sub - 1) / sub) + 15) / 16 * 16;
  const int cend = min(chunk * chunk_len + chunk_len, kv_len);
  int k0 = chunk * chunk_len + part * per;
  int k1 = min(k0 + per, cend);
  if (chunk >= chunks || k1 < k0) k0 = k1 = 0;

  v8<T> qreg[4];
  load_q<T>(Q, row_base, G, qreg);
  WaveSweep<T, G> st;
  st.run(Kp, Vp, qreg, k0, k1, (k1 - k0 + BLK - 1) / BLK, c, sP[wave]);
  publish_state<T, G>(st, wave, sAcc, sM, sL);
  __syncthreads();
  // left fold over the wave states in key order (= chunk order), finalize
  const int used = min(WG_WAVES, chunks * sub);
  for (int idx = threadIdx.x; idx < G * D; idx += 1024) {
    const int h = idx / D, d = idx % D;
    float m = sM[0][h], l = sL[0][h], a = sAcc[0][h][d];
    for (int w = 1; w < used; ++w) merge(m, l, a, sM[w][h], sL[w][h], sAcc[w][h][d]);
    const float coef = (l == 0.0f) ? 0.0f : 1.0f / l;
    O[(size_t)(row_base + h) * D + d] = narrow<T>(a * coef);
  }
}

// ---- chunk grid + separate fold (small batches) --------------------------------
template <typename T, int G>
__global__ __launch_bounds__(256) void fd_chunk_d128(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ Kc,
    const uint16_t *__restrict__ Vc, ChunkState *__restrict__ part, int q_heads, int kv_heads,
    int kv_len, int cap, int chunk_len, int chunks, float c) {
  __shared__ float sP[4][BLK][G];
  __shared__ float sAcc[4][G][D];
  __shared__ float sM[4][G], sL[4][G];

  const int ch = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int wave = threadIdx.x >> 6;
  const uint16_t *Kp = Kc + ((size_t)(b * kv_heads + kvh) * cap) * D;
  const uint16_t *Vp = Vc + ((size_t)(b * kv_heads + kvh) * cap) * D;
  const int row_base = b * q_heads + kvh * G;

  const int c0 = ch * chunk_len;
  const int c1 = min(c0 + chunk_len, kv_len);
  const int n = max(c1 - c0, 0);
  const int per = ((n + 4 * 16 - 1) / (4 * 16)) * 16;
  int k0 = c0 + wave * per;
  int k1 = min(k0 + per, c1);
  if (k1 < k0) k0 = k1 = 0;

  v8<T> qreg[4];
  load_q<T>(Q, row_base, G, qreg);
  WaveSweep<T, G> st;
  st.run(Kp, Vp, qreg, k0, k1, (k1 - k0 + BLK - 1) / BLK, c, sP[wave]);
  publish_state<T, G>(st, wave, sAcc, sM, sL);
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * D; idx += 256) {
    const int h = idx / D, d = idx % D;
    float m = sM[0][h], l = sL[0][h], a = sAcc[0][h][d];
#pragma unroll
    for (int w = 1; w < 4; ++w) merge(m, l, a, sM[w][h], sL[w][h], sAcc[w][h][d]);
    ChunkState &cs = part[(size_t)(row_base + h) * chunks + ch];
    cs.acc[d] = a;
    if (d == 0) {
      cs.m2 = m;
      cs.l = l;
    }
  }
}

// Left fold over the chunk states of one (batch, q_head), then finalize.
template <typename T>
__global__ __launch_bounds__(128) void fd_fold_d128(const ChunkState *__restrict__ part, uint16_t *__restrict__ O,
                                                    int chunks) {
  const int bh = blockIdx.x, d = threadIdx.x;
  const ChunkState *ps = part + (size_t)bh * chunks;
  float m = ps[0].m2, l = ps[0].l, a = ps[0].acc[d];
  for (int cc = 1; cc < chunks; ++cc) merge(m, l, a, ps[cc].m2, ps[cc].l, ps[cc].acc[d]);
  const float coef = (l == 0.0f) ? 0.0f : 1.0f / l;
  O[(size_t)bh * D + d] = narrow<T>(a * coef);
}

// ---- the no-allocation variant's scratch -------------------------------------
// File-scope device array for the chunk states of the chunk-grid path, for
// callers that cannot allocate.  Each GPU holds its own copy at its own
// address, looked up once per device with hipGetSymbolAddress (the array's
// name is only a host-side stand-in and is never passed to a kernel).
constexpr size_t SCRATCH_STATES = 8192;  // 8192 x 528 B = 4.125 MiB per GPU
static __device__ __align__(256) ChunkState scratch[SCRATCH_STATES];
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
ChunkState *g_scratch[MAX_DEVICES] = {};

int scratch_for(int device, ChunkState **out) {
  if (device < 0 || device >= MAX_DEVICES)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_decode_noalloc: device index above 63");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[device]) {
    void *ptr = nullptr;  // the device is current (set by the caller)
    WAFER_TRY(check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
    g_scratch[device] = (ChunkState *)ptr;
  }
  *out = g_scratch[device];
  return WAFER_HIP_OK;
}

// Shared by both entries: validation, then the group path (no workspace) or
// the chunk grid plus fold, whose states go to `part` when given, else to
// the context's workspace (grown on demand).
int decode(wafer_hip_context *ctx, uint32_t format, const void *q, const void *k_cache, const void *v_cache, void *o,
           uint32_t batch, uint32_t q_heads, uint32_t kv_heads, uint32_t kv_len, uint32_t kv_capacity,
           uint32_t head_dim, float scale, uint32_t chunks, bool noalloc) {
  WAFER_CHECK_CTX(ctx);
  if (format != WAFER_FMT_BF16 && format != WAFER_FMT_F16)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_decode: storage must be BF16 or F16");
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
  const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  // (the F16 group kernel for G = 4 would spill at the 128 VGPRs of a
  // 16-wave workgroup: F16 groups of 4 take the chunk grid)
  const uint32_t gmax = format == WAFER_FMT_BF16 ? 4u : 2u;
  const bool group = G <= gmax && chunks <= (uint32_t)WG_WAVES && (uint64_t)batch * kv_heads * 4 >= (uint64_t)cus * 3;
  const size_t states = (size_t)batch * q_heads * chunks;
  if (noalloc && !group && states > SCRATCH_STATES)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_decode_noalloc: batch * q_heads * chunks = " +
                                             std::to_string(states) + " chunk states exceed the scratch maximum of " +
                                             std::to_string(SCRATCH_STATES));
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const float c = scale * 0x1.715476p+0f;

  // (G = 8 needs more than the 128 VGPRs a 16-wave workgroup allows)
  if (group) {
    const int sub = WG_WAVES / (int)chunks;
    dim3 grid(kv_heads, batch);
#define FD_GROUP(TT, GV)                                                                          \
  hipLaunchKernelGGL((fd_group_d128<TT, GV>), grid, dim3(1024), 0, ctx->stream, (const uint16_t *)q, \
                     (const uint16_t *)k_cache, (const uint16_t *)v_cache, (uint16_t *)o,        \
                     (int)q_heads, (int)kv_heads, (int)kv_len, (int)kv_capacity, (int)chunks,    \
                     chunk_len, sub, c)
    if (format == WAFER_FMT_BF16) {
      switch (G) {
      case 1: FD_GROUP(__bf16, 1); break;
      case 2: FD_GROUP(__bf16, 2); break;
      default: FD_GROUP(__bf16, 4); break;
      }
    } else {
      switch (G) {
      case 1: FD_GROUP(_Float16, 1); break;
      default: FD_GROUP(_Float16, 2); break;
      }
    }
#undef FD_GROUP
    return launch_status("fd_group_d128");
  }

  ChunkState *part = nullptr;
  if (noalloc) {
    WAFER_TRY(scratch_for(ctx->device, &part));
  } else {
    WAFER_TRY(ensure_workspace(ctx, &ctx->workspace, &ctx->workspace_bytes, states * sizeof(ChunkState)));
    part = (ChunkState *)ctx->workspace;
  }
  dim3 grid(chunks, kv_heads, batch);
#define FD_CHUNK(TT, GV)                                                                          \
  hipLaunchKernelGGL((fd_chunk_d128<TT, GV>), grid, dim3(256), 0, ctx->stream, (const uint16_t *)q, \
                     (const uint16_t *)k_cache, (const uint16_t *)v_cache, part, (int)q_heads,    \
                     (int)kv_heads, (int)kv_len, (int)kv_capacity, chunk_len, (int)chunks, c)
  if (format == WAFER_FMT_BF16) {
    switch (G) {
    case 1: FD_CHUNK(__bf16, 1); break;
    case 2: FD_CHUNK(__bf16, 2); break;
    case 4: FD_CHUNK(__bf16, 4); break;
    default: FD_CHUNK(__bf16, 8); break;
    }
  } else {
    switch (G) {
    case 1: FD_CHUNK(_Float16, 1); break;
    case 2: FD_CHUNK(_Float16, 2); break;
    case 4: FD_CHUNK(_Float16, 4); break;
    default: FD_CHUNK(_Float16, 8); break;
    }
  }
#undef FD_CHUNK
  WAFER_TRY(launch_status("fd_chunk_d128"));
  if (format == WAFER_FMT_BF16)
    hipLaunchKernelGGL(fd_fold_d128<__bf16>, dim3(batch * q_heads), dim3(D), 0, ctx->stream, part, (uint16_t *)o,
                       (int)chunks);
  else
    hipLaunchKernelGGL(fd_fold_d128<_Float16>, dim3(batch * q_heads), dim3(D), 0, ctx->stream, part, (uint16_t *)o,
                       (int)chunks);
  return launch_status("fd_fold_d128");
}

// The functional KV-cache append of a decode step: rows
// [past_len, past_len + tokens) of every (batch, kv head) of both caches take
// the new tokens' K / V rows, byte for byte; the rows before past_len are not
// touched.  One thread per 16-byte piece when rows are whole 16-byte vectors
// (VEC), else per element.
template <bool VEC>
__global__ __launch_bounds__(256) void kv_append_kernel(const uint16_t *__restrict__ k_new,
                                                        const uint16_t *__restrict__ v_new, uint16_t *k_cache,
                                                        uint16_t *v_cache, int64_t pieces, int piece_elems,
                                                        int row_pieces, int tokens, int past_len, int capacity) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= pieces) return;
  // piece i of the new tensors [bh][token][row_pieces]
  const int64_t row = i / row_pieces;          // bh * tokens + token
  const int64_t bh = row / tokens;
  const int64_t tok = row - bh * tokens;
  const int64_t within = i - row * row_pieces;  // piece within the row
  const int64_t dst = ((bh * capacity + past_len + tok) * row_pieces + within) * piece_elems;
  const int64_t src = i * piece_elems;
  if constexpr (VEC) {
    *(u32x4 *)(k_cache + dst) = *(const u32x4 *)(k_new + src);
    *(u32x4 *)(v_cache + dst) = *(const u32x4 *)(v_new + src);
  } else {
    k_cache[dst] = k_new[src];
    v_cache[dst] = v_new[src];
  }
}

}  // namespace

// Looks up the no-allocation scratch's address on `device` (made current
// here; the caller's current device is restored).  Called once per context
// at creation, so the entry's first call -- possibly inside a graph
// capture -- finds the address already known.
int noalloc_scratch_lookup(int device) {
  int prev = 0;
  WAFER_TRY(check_hip(hipGetDevice(&prev), "hipGetDevice"));
  WAFER_TRY(check_hip(hipSetDevice(device), "hipSetDevice"));
  ChunkState *unused = nullptr;
  const int st = scratch_for(device, &unused);
  WAFER_TRY(check_hip(hipSetDevice(prev), "hipSetDevice"));
  return st;
}

}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_attention_decode(wafer_hip_context *ctx, uint32_t format,
                                          const void *q, const void *k_cache,
                                          const void *v_cache, void *o, uint32_t batch,
                                          uint32_t q_heads, uint32_t kv_heads,
                                          uint32_t kv_len, uint32_t kv_capacity,
                                          uint32_t head_dim, float scale, uint32_t chunks) {
  return decode(ctx, format, q, k_cache, v_cache, o, batch, q_heads, kv_heads, kv_len, kv_capacity, head_dim, scale,
                chunks, false);
}

extern "C" int wafer_hip_attention_decode_noalloc(wafer_hip_context *ctx, uint32_t format,
                                                  const void *q, const void *k_cache,
                                                  const void *v_cache, void *o, uint32_t batch,
                                                  uint32_t q_heads, uint32_t kv_heads,
                                                  uint32_t kv_len, uint32_t kv_capacity,
                                                  uint32_t head_dim, float scale, uint32_t chunks) {
  return decode(ctx, format, q, k_cache, v_cache, o, batch, q_heads, kv_heads, kv_len, kv_capacity, head_dim, scale,
                chunks, true);
}

extern "C" int wafer_hip_attention_decode_append(wafer_hip_context *ctx, uint32_t format, const void *q,
                                                 const void *k_new, const void *v_new, void *k_cache,
                                                 void *v_cache, void *o, uint32_t batch, uint32_t q_heads,
                                                 uint32_t kv_heads, uint32_t tokens, uint32_t past_len,
                                                 uint32_t kv_capacity, uint32_t head_dim, float scale,
                                                 uint32_t chunks) {
  WAFER_CHECK_CTX(ctx);
  if (format != WAFER_FMT_BF16 && format != WAFER_FMT_F16)
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_decode_append: storage must be BF16 or F16");
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !o)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode_append: null tensor");
  if (batch == 0 || q_heads == 0 || kv_heads == 0 || tokens == 0 || head_dim == 0 || chunks == 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode_append: empty dimension");
  if (q_heads % kv_heads != 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode_append: q_heads % kv_heads != 0");
  if ((uint64_t)past_len + tokens > kv_capacity)
    return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode_append: past_len + tokens exceeds kv_capacity");
  if (head_dim > 128 || (head_dim > 64 && head_dim < 128))
    return fail(WAFER_HIP_E_UNSUPPORTED, "attention_decode_append: head_dim must be 1..64 or 128");
  if (!(scale > 0.0f)) return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode_append: scale must be positive");
  const bool fd = tokens == 1 && head_dim == D;
  if (fd) {
    const uint32_t G = q_heads / kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8)
      return fail(WAFER_HIP_E_UNSUPPORTED, "attention_decode_append: q_heads/kv_heads must be 1, 2, 4 or 8");
    if (chunks > 65535 || kv_heads > 65535 || batch > 65535)
      return fail(WAFER_HIP_E_INVALID_FIELD, "attention_decode_append: grid dimension above 65535");
  }
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  // the append: whole 16-byte pieces when every row is, else per element
  const bool vec = head_dim % 8 == 0 &&
                   (((uintptr_t)k_new | (uintptr_t)v_new | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15) == 0;
  const int piece_elems = vec ? 8 : 1;
  const int row_pieces = (int)head_dim / piece_elems;
  const int64_t pieces = (int64_t)batch * kv_heads * tokens * row_pieces;
  const dim3 grid((unsigned)((pieces + 255) / 256));
  if (vec)
    hipLaunchKernelGGL(kv_append_kernel<true>, grid, dim3(256), 0, ctx->stream, (const uint16_t *)k_new,
                       (const uint16_t *)v_new, (uint16_t *)k_cache, (uint16_t *)v_cache, pieces, piece_elems,
                       row_pieces, (int)tokens, (int)past_len, (int)kv_capacity);
  else
    hipLaunchKernelGGL(kv_append_kernel<false>, grid, dim3(256), 0, ctx->stream, (const uint16_t *)k_new,
                       (const uint16_t *)v_new, (uint16_t *)k_cache, (uint16_t *)v_cache, pieces, piece_elems,
                       row_pieces, (int)tokens, (int)past_len, (int)kv_capacity);
  WAFER_TRY(launch_status("kv_append_kernel"));
  // attention over the updated caches: query i sees keys j <= past_len + i
  // (lower-right causal), so one token sees the whole cache
  if (fd)
    return decode(ctx, format, q, k_cache, v_cache, o, batch, q_heads, kv_heads, past_len + 1, kv_capacity, head_dim,
                  scale, chunks, false);
  wafer_hip_attention_mask mask{};
  mask.flags = WAFER_HIP_ATT_CAUSAL;
  mask.kv_capacity = kv_capacity;
  mask.causal_diagonal = past_len;
  return attention_prefill_masked(ctx, format, q, k_cache, v_cache, o, batch, q_heads, kv_heads, tokens,
                                  past_len + tokens, head_dim, scale, &mask);
}
