// regions.hip -- fused TileRegions: RMSNorm, softmax, SwiGLU, GELU-tanh,
// RoPE and bias-add, each one coalesced single pass over HBM (two reads of
// the row for the row-reduction regions, the second from L2).
//
// Each region is the composition of managed elementwise / reduce commands
// the compiler emits for it, with the op mapping of getInstrElementwiseKindAttr
// (lib/Wafer/Conversion/TileToInstr/ComputeLowering.cpp:2555-2606): Exp ->
// ExpLp, Div -> Recip then Mul, no tile-level Sigmoid.  Intermediates stay
// F32 and are rounded per operation in the same order as the commands
// (built with -ffp-contract=off, so no multiply-add is fused), with one
// narrowing at the region output.  The row sums use a parallel tree, so they
// match the host's left-to-right sums within tolerance rather than bit for
// bit; every other step is the same IEEE operation sequence.
#include "common.h"

namespace wafer {
namespace {

constexpr int RT = 256;  // threads per row workgroup

__device__ inline float block_sum(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < RT / 64; ++i) s += red[i];
  __syncthreads();
  return s;
}
__device__ inline float block_max(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int i = 1; i < RT / 64; ++i) s = fmaxf(s, red[i]);
  __syncthreads();
  return s;
}


// y = x * Rsqrt(Sum(x*x) * (1/N) + eps) * w.  VEC: 8 columns per thread and
// access (cols % 8 == 0, tensors 16-byte aligned).
// ADD (VEC only): the row is the CT Add of x and r, narrowed to F and stored
// to `sum` in the first pass; the second pass reads the stored sum back.
template <uint32_t F, bool VEC, bool ADD = false>
__global__ __launch_bounds__(RT) void rmsnorm_kernel(const void *__restrict__ x,
                                                     const void *__restrict__ w,
                                                     void *__restrict__ y, int64_t cols,
                                                     float inv_n, float eps,
                                                     const void *__restrict__ r = nullptr,
                                                     void *__restrict__ sum = nullptr) {
  __shared__ float red[RT / 64];
  const int64_t base = (int64_t)blockIdx.x * cols;
  float s = 0.0f;
  if constexpr (VEC) {
    for (int64_t c = 8 * threadIdx.x; c < cols; c += 8 * RT) {
      float v[8];
      load8<F>(x, base + c, v);
      if constexpr (ADD) {
        float rv[8];
        load8<F>(r, base + c, rv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += rv[e];
        store8<F>(sum, base + c, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = round_to<F>(v[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[e] * v[e];
    }
  } else {
    for (int64_t c = threadIdx.x; c < cols; c += RT) {
      const float v = load_as_f32<F>(x, base + c);
      s += v * v;
    }
  }
  s = block_sum(s, red);
  const float rs = 1.0f / sqrtf(s * inv_n + eps);
  if constexpr (VEC) {
    for (int64_t c = 8 * threadIdx.x; c < cols; c += 8 * RT) {
      float v[8], wv[8], o[8];
      load8<F>(ADD ? (const void *)sum : x, base + c, v);  // this thread's own stores (same addresses)
      load8<F>(w, c, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[e] * rs * wv[e];
      store8<F>(y, base + c, o);
    }
  } else {
    for (int64_t c = threadIdx.x; c < cols; c += RT) {
      const float v = load_as_f32<F>(x, base + c);
      store_from_f32<F>(y, base + c, v * rs * load_as_f32<F>(w, c));
    }
  }
}

// The row workgroup kernel above with the row held in registers between the
// sum and the scaling (rows of at most 8 * RT * NCH columns, cols % 8 == 0,
// 16-byte aligned): x (for ADD, x and r) is read once and w is loaded before
// the reduction; the sums and products are the same, in the same order.
template <uint32_t F, int NCH, bool ADD>
__global__ __launch_bounds__(RT) void rmsnorm_row_kernel(const void *__restrict__ x, const void *__restrict__ r,
                                                         const void *__restrict__ w, void *__restrict__ sum,
                                                         void *__restrict__ y, int64_t cols, float inv_n,
                                                         float eps) {
  __shared__ float red[RT / 64];
  const int64_t base = (int64_t)blockIdx.x * cols;
  float v[NCH][8], wv[NCH][8];
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const int64_t c = 8 * ((int64_t)threadIdx.x + RT * q);
    if (c < cols) {
      load8<F>(x, base + c, v[q]);
      load8<F>(w, c, wv[q]);
    }
  }
  if constexpr (ADD) {
#pragma unroll
    for (int q = 0; q < NCH; ++q) {
      const int64_t c = 8 * ((int64_t)threadIdx.x + RT * q);
      if (c < cols) {
        float rv[8];
        load8<F>(r, base + c, rv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[q][e] += rv[e];
        store8<F>(sum, base + c, v[q]);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[q][e] = round_to<F>(v[q][e]);
      }
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int q = 0; q < NCH; ++q)
    if (8 * ((int64_t)threadIdx.x + RT * q) < cols) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[q][e] * v[q][e];
    }
  s = block_sum(s, red);
  const float rs = 1.0f / sqrtf(s * inv_n + eps);
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const int64_t c = 8 * ((int64_t)threadIdx.x + RT * q);
    if (c < cols) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[q][e] * rs * wv[q][e];
      store8<F>(y, base + c, o);
    }
  }
}

// Row counts from which the wave-per-row kernel below is used: it keeps one
// wave per row in flight (4 per CU at 1024 rows, where the workgroup kernel's
// 16 hide the latency chain better: 9.1 against 6.2 us at 1024 x 4096), and
// reads x once (72.5 against 68 % of HBM peak at 65536 x 4096).
constexpr uint64_t WAVE_ROWS = 4096;

// The same row region with one wave per row for rows of at most 512 * NCH
// columns (cols % 8 == 0, 16-byte aligned): the row stays in registers
// between the sum and the scaling (one read of x), the sum is a wave
// reduction (no LDS, no barrier), and a 256-thread workgroup serves 4 rows.
// ADD: the row is first the CT Add of x and r, narrowed to the storage format
// and stored to sum (bit for bit the Add command), and the norm reads the
// narrowed sum: Add followed by RMSNorm in one pass.
template <uint32_t F, int NCH, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_wave_kernel(const void *__restrict__ x, const void *__restrict__ r,
                                                           const void *__restrict__ w, void *__restrict__ sum,
                                                           void *__restrict__ y, int64_t rows, int64_t cols,
                                                           float inv_n, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves
  const int lane = threadIdx.x & 63;
  const int64_t base = row * cols;
  float v[NCH][8];
  float s = 0.0f;
  // every chunk load is issued before any is used: a chunk past the row
  // end loads the row's last chunk again and adds nothing
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const int64_t c = 8 * (lane + 64 * q);
    load8_nt<F>(x, base + (c < cols ? c : cols - 8), v[q]);
  }
  if constexpr (ADD) {
    float rv[NCH][8];
#pragma unroll
    for (int q = 0; q < NCH; ++q) {
      const int64_t c = 8 * (lane + 64 * q);
      load8_nt<F>(r, base + (c < cols ? c : cols - 8), rv[q]);
    }
#pragma unroll
    for (int q = 0; q < NCH; ++q) {
      const int64_t c = 8 * (lane + 64 * q);
      float t[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = v[q][e] + rv[q][e];
      if (c < cols) store8<F>(sum, base + c, t);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[q][e] = round_to<F>(t[e]);
    }
  }
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const bool in_row = 8 * (lane + 64 * q) < cols;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += in_row ? v[q][e] * v[q][e] : 0.0f;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  const float rs = 1.0f / sqrtf(s * inv_n + eps);
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const int64_t c = 8 * (lane + 64 * q);
    if (c < cols) {
      float wv[8], o[8];
      load8<F>(w, c, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[q][e] * rs * wv[e];
      store8<F>(y, base + c, o);
    }
  }
}

// e = ExpLp(x - rowmax); y = e * Recip(Sum(e)).  Rows of at most
// 8 * RT * NCH columns (cols % 8 == 0, 16-byte aligned): the row is read
// once into registers (NCH 16-byte chunks per thread) and each e is taken
// once; the scalar kernel below re-reads the row for each pass.  The grid
// has one workgroup per row.
template <uint32_t F, int NCH>
__device__ inline void softmax_vec_body(const void *__restrict__ x, void *__restrict__ y, int64_t cols, float *red) {
  const int64_t base = (int64_t)blockIdx.x * cols;
  float v[NCH][8];
  float m = -__builtin_inff();
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    const int64_t c = 8 * ((int64_t)threadIdx.x + ch * RT);
    if (c < cols) {
      load8_nt<F>(x, base + c, v[ch]);
#pragma unroll
      for (int e = 0; e < 8; ++e) m = fmaxf(m, v[ch][e]);
    }
  }
  m = block_max(m, red);
  float s = 0.0f;
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    if (8 * ((int64_t)threadIdx.x + ch * RT) < cols) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[ch][e] = explp_acc(v[ch][e] - m);
        s += v[ch][e];
      }
    }
  }
  s = block_sum(s, red);
  const float rc = 1.0f / s;
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    const int64_t c = 8 * ((int64_t)threadIdx.x + ch * RT);
    if (c < cols) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[ch][e] * rc;
      store8<F>(y, base + c, o);
    }
  }
}
// (single-parameter kernel names for DISPATCH_F)
template <uint32_t F>
__global__ __launch_bounds__(RT) void softmax_vec1(const void *__restrict__ x, void *__restrict__ y, int64_t cols) {
  __shared__ float red[RT / 64];
  softmax_vec_body<F, 1>(x, y, cols, red);
}
template <uint32_t F>
__global__ __launch_bounds__(RT) void softmax_vec2(const void *__restrict__ x, void *__restrict__ y, int64_t cols) {
  __shared__ float red[RT / 64];
  softmax_vec_body<F, 2>(x, y, cols, red);
}
template <uint32_t F>
__global__ __launch_bounds__(RT) void softmax_vec4(const void *__restrict__ x, void *__restrict__ y, int64_t cols) {
  __shared__ float red[RT / 64];
  softmax_vec_body<F, 4>(x, y, cols, red);
}

template <uint32_t F>
__global__ __launch_bounds__(RT) void softmax_kernel(const void *__restrict__ x,
                                                     void *__restrict__ y, int64_t cols) {
  __shared__ float red[RT / 64];
  const int64_t base = (int64_t)blockIdx.x * cols;
  float m = -__builtin_inff();
  for (int64_t c = threadIdx.x; c < cols; c += RT) m = fmaxf(m, load_as_f32<F>(x, base + c));
  m = block_max(m, red);
  float s = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += RT) s += explp_acc(load_as_f32<F>(x, base + c) - m);
  s = block_sum(s, red);
  const float rc = 1.0f / s;
  for (int64_t c = threadIdx.x; c < cols; c += RT)
    store_from_f32<F>(y, base + c, explp_acc(load_as_f32<F>(x, base + c) - m) * rc);
}

template <uint32_t F, bool VEC>
__global__ __launch_bounds__(256) void silu_mul_kernel(const void *__restrict__ gate,
                                                       const void *__restrict__ up,
                                                       void *__restrict__ y, uint64_t count) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t tail = 0;
  if constexpr (VEC) {
    for (uint64_t q = gid; q < count / 8; q += stride) {
      float g[8], u[8], r[8];
      load8_nt<F>(gate, (int64_t)(8 * q), g);
      load8_nt<F>(up, (int64_t)(8 * q), u);
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = silu_mul_1(g[e], u[e]);
      store8<F>(y, (int64_t)(8 * q), r);
    }
    tail = count / 8 * 8;
  }
  for (uint64_t i = tail + gid; i < count; i += stride)
    store_from_f32<F>(y, (int64_t)i, silu_mul_1(load_as_f32<F>(gate, (int64_t)i), load_as_f32<F>(up, (int64_t)i)));
}

template <uint32_t F, bool VEC>
__global__ __launch_bounds__(256) void gelu_tanh_kernel(const void *__restrict__ x,
                                                        void *__restrict__ y, uint64_t count) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t tail = 0;
  if constexpr (VEC) {
    for (uint64_t q = gid; q < count / 8; q += stride) {
      float v[8], r[8];
      load8_nt<F>(x, (int64_t)(8 * q), v);
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = gelu_tanh_1(v[e]);
      store8<F>(y, (int64_t)(8 * q), r);
    }
    tail = count / 8 * 8;
  }
  for (uint64_t i = tail + gid; i < count; i += stride)
    store_from_f32<F>(y, (int64_t)i, gelu_tanh_1(load_as_f32<F>(x, (int64_t)i)));
}

// Rotate-half RoPE: inv_freq[i] = 1/theta^(2i/D), angle = pos*inv_freq[d mod D/2],
// y = x*cos(angle) + rotate_half(x)*sin(angle), rotate_half(x) = [-x2, x1].
// One thread per rotation pair (d, d + head_dim/2) of a row (VEC: per 8
// consecutive pairs, head_dim % 16 == 0 and 16-byte aligned tensors): both
// outputs of a pair come from the same two inputs, so y may alias x.
// y[d] = x[d]*cos + rot[d]*sin with rot = (-x[d+half], x[d-half])
__device__ inline void rope_rot(float xl, float xh, float c, float s, float &yl, float &yh) {
  yl = xl * c + (-xh) * s;
  yh = xh * c + xl * s;
}
__device__ inline void rope_pair(float xl, float xh, float angle, float &yl, float &yh) {
  rope_rot(xl, xh, cosf(angle), sinf(angle), yl, yh);
}
__device__ inline float rope_inv_freq(float theta, int64_t i, int64_t head_dim) {
  return 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
}
template <uint32_t F, bool VEC>
__global__ __launch_bounds__(256) void rope_kernel(const void *x, void *y,
                                                   int64_t tokens, int64_t heads, int64_t head_dim,
                                                   const int32_t *__restrict__ positions,
                                                   float theta) {
  const int64_t half = head_dim / 2;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if constexpr (VEC) {
    // one thread per (token, 8 frequencies, head slice): the 8 angles'
    // cos / sin are taken once and applied to heads slice, slice + ns, ...
    // (the same values rope_pair computes per element); with ns slices of
    // per_tok groups filling a wave, one wave covers ns whole heads of one
    // token per step, contiguous in memory
    const int64_t per_tok = half / 8;
    const int64_t ns = (per_tok <= 64 && 64 % per_tok == 0) ? 64 / per_tok : 1;
    const int64_t groups = tokens * per_tok * ns;
    for (int64_t e = gid; e < groups; e += stride) {
      const int64_t t = e / (per_tok * ns);
      const int64_t r = e - t * (per_tok * ns);
      const int64_t hs = r / per_tok, i0 = (r - hs * per_tok) * 8;
      const float pos = (float)positions[t];
      float cs[8], sn[8];
      if (ns >= 8) {
        // the slices' lanes share the 8 angles of their group: lane slice k
        // (k < 8) takes angle k once, and every lane gathers all 8 (a wave
        // holds whole tokens: groups and the stride are multiples of 64)
        const int64_t g = r - hs * per_tok;
        const int kk = (int)(hs & 7);
        const float angle = pos * rope_inv_freq(theta, i0 + kk, head_dim);
        const float c1 = cosf(angle), s1 = sinf(angle);
        const int lane = (int)(threadIdx.x & 63);
        const int base_lane = lane - (int)r;  // lane of (slice 0, group 0) of this token
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int src = base_lane + k * (int)per_tok + (int)g;
          cs[k] = __shfl(c1, src);
          sn[k] = __shfl(s1, src);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float angle = pos * rope_inv_freq(theta, i0 + k, head_dim);
          cs[k] = cosf(angle);
          sn[k] = sinf(angle);
        }
      }
      if (hs >= heads) continue;
      auto one = [&](int64_t h) __attribute__((always_inline)) {
        const int64_t lo = (t * heads + h) * head_dim + i0, hi = lo + half;
        float xl[8], xh[8], yl[8], yh[8];
        load8_nt<F>(x, lo, xl);
        load8_nt<F>(x, hi, xh);
#pragma unroll
        for (int k = 0; k < 8; ++k) rope_rot(xl[k], xh[k], cs[k], sn[k], yl[k], yh[k]);
        store8<F>(y, lo, yl);
        store8<F>(y, hi, yh);
      };
      int64_t h = hs;
      for (; h + 3 * ns < heads; h += 4 * ns) {  // four heads' loads in flight
        one(h);
        one(h + ns);
        one(h + 2 * ns);
        one(h + 3 * ns);
      }
      for (; h < heads; h += ns) one(h);
    }
  } else {
    const int64_t pairs = tokens * heads * half;
    for (int64_t e = gid; e < pairs; e += stride) {
      const int64_t i = e % half;
      const int64_t rowi = e / half;  // (token, head)
      const int64_t t = rowi / heads;
      const int64_t lo = rowi * head_dim + i, hi = lo + half;
      float yl, yh;
      rope_pair(load_as_f32<F>(x, lo), load_as_f32<F>(x, hi), (float)positions[t] * rope_inv_freq(theta, i, head_dim),
                yl, yh);
      store_from_f32<F>(y, lo, yl);
      store_from_f32<F>(y, hi, yh);
    }
  }
}

// RoPE fused into the token-major -> head-major re-layout of a projection:
// y[h, t, :] = RoPE(x[t * ts + h * head_dim + :]) with the rope region's own
// expressions (rope_inv_freq, pos * inv_freq, cosf/sinf, rope_rot), so it
// equals head_permute followed by rope bit for bit.  One thread serves 8
// frequencies of one token for a group of HG heads and takes the 8 angles'
// cos/sin once for the group (the rope region recomputes them per head).
// head_dim % 16 == 0, ts % 8 == 0, 16-byte aligned tensors.
template <uint32_t F, int HG>
__global__ __launch_bounds__(256) void permute_rope_kernel(const void *x, void *y, int64_t tokens,
                                                           int64_t heads, int64_t head_dim, int64_t ts,
                                                           const int32_t *__restrict__ positions,
                                                           float theta) {
  const int64_t half = head_dim / 2, per_row = half / 8;
  const int64_t total = tokens * per_row * ((heads + HG - 1) / HG);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    // e = (group, token, chunk): consecutive lanes read consecutive chunks of
    // a token's heads and write consecutive chunks of head-major rows
    const int64_t c = e % per_row, tg = e / per_row;
    const int64_t t = tg % tokens, hg = tg / tokens;
    const int64_t i0 = c * 8;
    const float pos = (float)positions[t];
    float cs[8], sn[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float angle = pos * rope_inv_freq(theta, i0 + k, head_dim);
      cs[k] = cosf(angle);
      sn[k] = sinf(angle);
    }
#pragma unroll
    for (int hh = 0; hh < HG; ++hh) {
      const int64_t h = hg * HG + hh;
      if (h >= heads) break;
      const int64_t src = t * ts + h * head_dim + i0;
      const int64_t dst = (h * tokens + t) * head_dim + i0;
      float xl[8], xh[8], yl[8], yh[8];
      load8<F>(x, src, xl);
      load8<F>(x, src + half, xh);
#pragma unroll
      for (int k = 0; k < 8; ++k) rope_rot(xl[k], xh[k], cs[k], sn[k], yl[k], yh[k]);
      store8<F>(y, dst, yl);
      store8<F>(y, dst + half, yh);
    }
  }
}

// The same re-layout with one wave per (token, group of 64 / CPH heads),
// CPH = head_dim / 16 chunks of 8 frequencies per head: lane hh * CPH + c
// rotates chunk c of head hh of the group.  Every lane takes the cos / sin
// of one angle (frequency 8 c + hh % 8) and the 8 angles of its chunk come
// from the lanes of the same c through shuffles, so each angle is computed
// once per token and head group rather than per head and chunk.  A wave
// reads whole 64 / CPH-head spans of one token row and writes whole rows of
// each head.  head_dim 16 .. 128, a multiple of 16.
template <uint32_t F>
__global__ __launch_bounds__(256) void permute_rope_lanes_kernel(const void *x, void *y, int64_t tokens,
                                                                 int64_t heads, int64_t head_dim, int64_t ts,
                                                                 const int32_t *__restrict__ positions,
                                                                 float theta) {
  const int cph = (int)(head_dim / 16), hpw = 64 / cph;  // chunks per head, heads per wave
  const int64_t groups = (heads + hpw - 1) / hpw;
  const int64_t waves = tokens * groups;
  const int lane = threadIdx.x & 63;
  const int c = lane % cph, hh = lane / cph;
  const int64_t half = head_dim / 2, i0 = 8 * c;
  const int64_t wstride = (int64_t)gridDim.x * (blockDim.x / 64);
  for (int64_t w = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); w < waves; w += wstride) {
    const int64_t t = w / groups, h = (w % groups) * hpw + hh;
    const float pos = (float)positions[t];
    const float angle = pos * rope_inv_freq(theta, i0 + (hh & 7), head_dim);
    const float mc = cosf(angle), ms = sinf(angle);
    float cs[8], sn[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {  // every lane takes part, also past the last head
      cs[k] = __shfl(mc, k * cph + c);
      sn[k] = __shfl(ms, k * cph + c);
    }
    if (h < heads) {
      const int64_t src = t * ts + h * head_dim + i0;
      const int64_t dst = (h * tokens + t) * head_dim + i0;
      float xl[8], xh[8], yl[8], yh[8];
      load8<F>(x, src, xl);
      load8<F>(x, src + half, xh);
#pragma unroll
      for (int k = 0; k < 8; ++k) rope_rot(xl[k], xh[k], cs[k], sn[k], yl[k], yh[k]);
      store8<F>(y, dst, yl);
      store8<F>(y, dst + half, yh);
    }
  }
}

// VEC: 8 columns per thread (cols % 8 == 0, tensors 16-byte aligned)
template <uint32_t F, bool VEC>
__global__ __launch_bounds__(256) void bias_add_kernel(const void *__restrict__ x,
                                                       const float *__restrict__ bias,
                                                       void *__restrict__ y, int64_t rows,
                                                       int64_t cols) {
  const int64_t count = rows * cols;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if constexpr (VEC) {
    // the column of this thread's chunk advances by the stride's remainder
    // (one 64-bit division per thread, not one per chunk)
    const int64_t step = (8 * stride) % cols;
    int64_t c0 = (8 * gid) % cols;
    for (int64_t q = gid; q < count / 8; q += stride) {
      const int64_t e0 = 8 * q;
      float v[8], b[8], r[8];
      load8<F>(x, e0, v);  // (non-temporal loads measured slower here: 437 against 400 us at 256M f32)
      load8<WAFER_FMT_F32>(bias, c0, b);
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = v[e] + b[e];
      store8<F>(y, e0, r);
      c0 += step;
      if (c0 >= cols) c0 -= cols;
    }
  } else {
    for (int64_t e = gid; e < count; e += stride) store_from_f32<F>(y, e, load_as_f32<F>(x, e) + bias[e % cols]);
  }
}

unsigned grid_for(uint64_t count) {
  return (unsigned)std::min<uint64_t>((count + 255) / 256, 65536);
}

template <uint32_t F, bool ADD>
void launch_rmsnorm_wave(hipStream_t st, int nch, dim3 grid, const void *x, const void *r, const void *w, void *sum,
                         void *y, int64_t rows, int64_t cols, float inv_n, float eps) {
  if (nch == 1)
    hipLaunchKernelGGL((rmsnorm_wave_kernel<F, 1, ADD>), grid, dim3(256), 0, st, x, r, w, sum, y, rows, cols, inv_n,
                       eps);
  else if (nch == 2)
    hipLaunchKernelGGL((rmsnorm_wave_kernel<F, 2, ADD>), grid, dim3(256), 0, st, x, r, w, sum, y, rows, cols, inv_n,
                       eps);
  else if (nch == 4)
    hipLaunchKernelGGL((rmsnorm_wave_kernel<F, 4, ADD>), grid, dim3(256), 0, st, x, r, w, sum, y, rows, cols, inv_n,
                       eps);
  else
    hipLaunchKernelGGL((rmsnorm_wave_kernel<F, 8, ADD>), grid, dim3(256), 0, st, x, r, w, sum, y, rows, cols, inv_n,
                       eps);
}
template <bool ADD>
void launch_rmsnorm_wave_f(hipStream_t st, uint32_t format, int nch, dim3 grid, const void *x, const void *r,
                           const void *w, void *sum, void *y, int64_t rows, int64_t cols, float inv_n, float eps) {
  if (format == WAFER_FMT_F32)
    launch_rmsnorm_wave<WAFER_FMT_F32, ADD>(st, nch, grid, x, r, w, sum, y, rows, cols, inv_n, eps);
  else if (format == WAFER_FMT_BF16)
    launch_rmsnorm_wave<WAFER_FMT_BF16, ADD>(st, nch, grid, x, r, w, sum, y, rows, cols, inv_n, eps);
  else
    launch_rmsnorm_wave<WAFER_FMT_F16, ADD>(st, nch, grid, x, r, w, sum, y, rows, cols, inv_n, eps);
}

#define DISPATCH_F(format, KERNEL, GRID, BLOCK, ...)                                           \
  do {                                                                                         \
    if ((format) == WAFER_FMT_F32)                                                             \
      hipLaunchKernelGGL(KERNEL<WAFER_FMT_F32>, GRID, BLOCK, 0, ctx->stream, __VA_ARGS__);    \
    else if ((format) == WAFER_FMT_BF16)                                                       \
      hipLaunchKernelGGL(KERNEL<WAFER_FMT_BF16>, GRID, BLOCK, 0, ctx->stream, __VA_ARGS__);   \
    else                                                                                       \
      hipLaunchKernelGGL(KERNEL<WAFER_FMT_F16>, GRID, BLOCK, 0, ctx->stream, __VA_ARGS__);    \
  } while (0)

// format x {scalar, 8-wide} dispatch for the kernels with a VEC parameter
#define DISPATCH_FB(format, vec, KERNEL, GRID, BLOCK, ...)                                      \
  do {                                                                                         \
    if (vec) {                                                                                 \
      if ((format) == WAFER_FMT_F32)                                                           \
        hipLaunchKernelGGL((KERNEL<WAFER_FMT_F32, true>), GRID, BLOCK, 0, ctx->stream, __VA_ARGS__);  \
      else if ((format) == WAFER_FMT_BF16)                                                     \
        hipLaunchKernelGGL((KERNEL<WAFER_FMT_BF16, true>), GRID, BLOCK, 0, ctx->stream, __VA_ARGS__); \
      else                                                                                     \
        hipLaunchKernelGGL((KERNEL<WAFER_FMT_F16, true>), GRID, BLOCK, 0, ctx->stream, __VA_ARGS__);  \
    } else {                                                                                   \
      if ((format) == WAFER_FMT_F32)                                                           \
        hipLaunchKernelGGL((KERNEL<WAFER_FMT_F32, false>), GRID, BLOCK, 0, ctx->stream, __VA_ARGS__); \
      else if ((format) == WAFER_FMT_BF16)                                                     \
        hipLaunchKernelGGL((KERNEL<WAFER_FMT_BF16, false>), GRID, BLOCK, 0, ctx->stream, __VA_ARGS__);\
      else                                                                                     \
        hipLaunchKernelGGL((KERNEL<WAFER_FMT_F16, false>), GRID, BLOCK, 0, ctx->stream, __VA_ARGS__); \
    }                                                                                          \
  } while (0)

int prologue(wafer_hip_context *ctx, uint32_t format, const char *what) {
  WAFER_CHECK_CTX(ctx);
  if (!is_float_format(format))
    return fail(WAFER_HIP_E_UNSUPPORTED, std::string(what) + ": format must be F16, BF16 or F32");
  return check_hip(hipSetDevice(ctx->device), "hipSetDevice");
}

}  // namespace
}  // namespace wafer

namespace wafer {
namespace {
// the register-resident row kernel for rows of at most 8 * RT * 4 columns
template <bool ADD>
bool launch_rmsnorm_row(hipStream_t st, uint32_t format, uint64_t rows, uint64_t cols, const void *x, const void *r,
                        const void *w, void *sum, void *y, float inv_n, float eps) {
  if (cols > 8 * RT * 4) return false;
  const int nch = cols <= 8 * RT ? 1 : cols <= 16 * RT ? 2 : 4;
  const dim3 grid((unsigned)rows);
  const int64_t c = (int64_t)cols;
#define RMS_ROW(FMT, N) hipLaunchKernelGGL((rmsnorm_row_kernel<FMT, N, ADD>), grid, dim3(RT), 0, st, x, r, w, sum, y, c, inv_n, eps)
#define RMS_ROW_N(FMT)      \
  do {                       \
    if (nch == 1)            \
      RMS_ROW(FMT, 1);       \
    else if (nch == 2)       \
      RMS_ROW(FMT, 2);       \
    else                     \
      RMS_ROW(FMT, 4);       \
  } while (0)
  if (format == WAFER_FMT_F32) RMS_ROW_N(WAFER_FMT_F32);
  else if (format == WAFER_FMT_BF16) RMS_ROW_N(WAFER_FMT_BF16);
  else RMS_ROW_N(WAFER_FMT_F16);
#undef RMS_ROW_N
#undef RMS_ROW
  return true;
}
}  // namespace
}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_rmsnorm(wafer_hip_context *ctx, uint32_t format, const void *x,
                                 const void *w, void *y, uint64_t rows, uint64_t cols, float eps) {
  WAFER_TRY(prologue(ctx, format, "rmsnorm"));
  if (rows == 0 || cols == 0) return WAFER_HIP_OK;
  if (!x || !w || !y) return fail(WAFER_HIP_E_INVALID_FIELD, "rmsnorm: null tensor");
  if (rows > 0x7fffffffull) return fail(WAFER_HIP_E_INVALID_FIELD, "rmsnorm: too many rows");
  const float inv_n = 1.0f / (float)cols;
  const bool vec = cols % 8 == 0 && aligned16(x) && aligned16(w) && aligned16(y);
  if (vec && cols <= 4096 && rows >= WAVE_ROWS) {
    const dim3 grid((unsigned)((rows + 3) / 4));
    const int64_t r = (int64_t)rows, c = (int64_t)cols;
    const int nch = cols <= 512 ? 1 : cols <= 1024 ? 2 : cols <= 2048 ? 4 : 8;
    launch_rmsnorm_wave_f<false>(ctx->stream, format, nch, grid, x, nullptr, w, nullptr, y, r, c, inv_n, eps);
    return launch_status("rmsnorm_wave_kernel");
  }
  if (vec && launch_rmsnorm_row<false>(ctx->stream, format, rows, cols, x, nullptr, w, nullptr, y, inv_n, eps))
    return launch_status("rmsnorm_row_kernel");
  DISPATCH_FB(format, vec, rmsnorm_kernel, dim3((unsigned)rows), dim3(RT), x, w, y, (int64_t)cols, inv_n, eps);
  return launch_status("rmsnorm_kernel");
}

extern "C" int wafer_hip_add_rmsnorm(wafer_hip_context *ctx, uint32_t format, const void *x, const void *r,
                                     const void *w, void *sum, void *y, uint64_t rows, uint64_t cols, float eps) {
  WAFER_TRY(prologue(ctx, format, "add_rmsnorm"));
  if (rows == 0 || cols == 0) return WAFER_HIP_OK;
  if (!x || !r || !w || !sum || !y) return fail(WAFER_HIP_E_INVALID_FIELD, "add_rmsnorm: null tensor");
  if (rows > 0x7fffffffull) return fail(WAFER_HIP_E_INVALID_FIELD, "add_rmsnorm: too many rows");
  if (sum == y) return fail(WAFER_HIP_E_INVALID_FIELD, "add_rmsnorm: sum and y must be distinct");
  const bool vec = cols % 8 == 0 && aligned16(x) && aligned16(r) && aligned16(w) && aligned16(sum) && aligned16(y);
  if (!vec) {  // the Add command, then the region
    WAFER_TRY(wafer_hip_elementwise(ctx, 8u, format, x, r, sum, rows * cols));
    return wafer_hip_rmsnorm(ctx, format, sum, w, y, rows, cols, eps);
  }
  const float inv_n = 1.0f / (float)cols;
  if (cols <= 4096 && rows >= WAVE_ROWS) {
    const dim3 grid((unsigned)((rows + 3) / 4));
    const int nch = cols <= 512 ? 1 : cols <= 1024 ? 2 : cols <= 2048 ? 4 : 8;
    launch_rmsnorm_wave_f<true>(ctx->stream, format, nch, grid, x, r, w, sum, y, (int64_t)rows, (int64_t)cols,
                                inv_n, eps);
    return launch_status("rmsnorm_wave_kernel");
  }
  if (launch_rmsnorm_row<true>(ctx->stream, format, rows, cols, x, r, w, sum, y, inv_n, eps))
    return launch_status("rmsnorm_row_kernel");
  const dim3 grid((unsigned)rows);
  if (format == WAFER_FMT_F32)
    hipLaunchKernelGGL((rmsnorm_kernel<WAFER_FMT_F32, true, true>), grid, dim3(RT), 0, ctx->stream, x, w, y,
                       (int64_t)cols, inv_n, eps, r, sum);
  else if (format == WAFER_FMT_BF16)
    hipLaunchKernelGGL((rmsnorm_kernel<WAFER_FMT_BF16, true, true>), grid, dim3(RT), 0, ctx->stream, x, w, y,
                       (int64_t)cols, inv_n, eps, r, sum);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<WAFER_FMT_F16, true, true>), grid, dim3(RT), 0, ctx->stream, x, w, y,
                       (int64_t)cols, inv_n, eps, r, sum);
  return launch_status("rmsnorm_kernel");
}

extern "C" int wafer_hip_softmax(wafer_hip_context *ctx, uint32_t format, const void *x, void *y,
                                 uint64_t rows, uint64_t cols) {
  WAFER_TRY(prologue(ctx, format, "softmax"));
  if (rows == 0 || cols == 0) return WAFER_HIP_OK;
  if (!x || !y) return fail(WAFER_HIP_E_INVALID_FIELD, "softmax: null tensor");
  if (rows > 0x7fffffffull) return fail(WAFER_HIP_E_INVALID_FIELD, "softmax: too many rows");
  if (cols % 8 == 0 && cols <= 8 * RT * 4 && aligned16(x) && aligned16(y)) {
    const dim3 grid((unsigned)rows);
    if (cols <= 8 * RT) {
      DISPATCH_F(format, softmax_vec1, grid, dim3(RT), x, y, (int64_t)cols);
    } else if (cols <= 16 * RT) {
      DISPATCH_F(format, softmax_vec2, grid, dim3(RT), x, y, (int64_t)cols);
    } else {
      DISPATCH_F(format, softmax_vec4, grid, dim3(RT), x, y, (int64_t)cols);
    }
    return launch_status("softmax_vec");
  }
  DISPATCH_F(format, softmax_kernel, dim3((unsigned)rows), dim3(RT), x, y, (int64_t)cols);
  return launch_status("softmax_kernel");
}

extern "C" int wafer_hip_silu_mul(wafer_hip_context *ctx, uint32_t format, const void *gate,
                                  const void *up, void *y, uint64_t count) {
  WAFER_TRY(prologue(ctx, format, "silu_mul"));
  if (count == 0) return WAFER_HIP_OK;
  if (!gate || !up || !y) return fail(WAFER_HIP_E_INVALID_FIELD, "silu_mul: null tensor");
  const bool vec = aligned16(gate) && aligned16(up) && aligned16(y);
  DISPATCH_FB(format, vec, silu_mul_kernel, dim3(grid_for(vec ? (count + 7) / 8 : count)), dim3(256), gate, up,
              y, count);
  return launch_status("silu_mul_kernel");
}

extern "C" int wafer_hip_gelu_tanh(wafer_hip_context *ctx, uint32_t format, const void *x, void *y,
                                   uint64_t count) {
  WAFER_TRY(prologue(ctx, format, "gelu_tanh"));
  if (count == 0) return WAFER_HIP_OK;
  if (!x || !y) return fail(WAFER_HIP_E_INVALID_FIELD, "gelu_tanh: null tensor");
  const bool vec = aligned16(x) && aligned16(y);
  DISPATCH_FB(format, vec, gelu_tanh_kernel, dim3(grid_for(vec ? (count + 7) / 8 : count)), dim3(256), x, y,
              count);
  return launch_status("gelu_tanh_kernel");
}

extern "C" int wafer_hip_rope(wafer_hip_context *ctx, uint32_t format, const void *x, void *y,
                              uint64_t tokens, uint64_t heads, uint64_t head_dim,
                              const int32_t *positions, float theta) {
  WAFER_TRY(prologue(ctx, format, "rope"));
  if (head_dim % 2) return fail(WAFER_HIP_E_INVALID_FIELD, "rope: head_dim must be even");
  const uint64_t count = tokens * heads * head_dim;
  if (count == 0) return WAFER_HIP_OK;
  if (!x || !y || !positions) return fail(WAFER_HIP_E_INVALID_FIELD, "rope: null tensor");
  const bool vec = head_dim % 16 == 0 && aligned16(x) && aligned16(y);
  const uint64_t per_tok = vec ? head_dim / 16 : 1;  // (>= 1: vec needs head_dim % 16 == 0)
  const uint64_t ns = (per_tok <= 64 && 64 % per_tok == 0) ? 64 / per_tok : 1;
  DISPATCH_FB(format, vec, rope_kernel, dim3(grid_for(vec ? tokens * per_tok * ns : count / 2)), dim3(256), x, y,
              (int64_t)tokens, (int64_t)heads, (int64_t)head_dim, positions, theta);
  return launch_status("rope_kernel");
}

template <uint32_t F>
void launch_permute_rope(hipStream_t st, int hg, dim3 grid, const void *src, void *dst, int64_t tokens,
                         int64_t heads, int64_t head_dim, int64_t ts, const int32_t *positions, float theta) {
  if (hg == 8)
    hipLaunchKernelGGL((permute_rope_kernel<F, 8>), grid, dim3(256), 0, st, src, dst, tokens, heads, head_dim, ts,
                       positions, theta);
  else if (hg == 4)
    hipLaunchKernelGGL((permute_rope_kernel<F, 4>), grid, dim3(256), 0, st, src, dst, tokens, heads, head_dim, ts,
                       positions, theta);
  else if (hg == 2)
    hipLaunchKernelGGL((permute_rope_kernel<F, 2>), grid, dim3(256), 0, st, src, dst, tokens, heads, head_dim, ts,
                       positions, theta);
  else
    hipLaunchKernelGGL((permute_rope_kernel<F, 1>), grid, dim3(256), 0, st, src, dst, tokens, heads, head_dim, ts,
                       positions, theta);
}

extern "C" int wafer_hip_head_permute_rope(wafer_hip_context *ctx, uint32_t format, const void *src,
                                           void *dst, uint64_t tokens, uint64_t heads,
                                           uint64_t head_dim, uint64_t token_stride,
                                           const int32_t *positions, float theta) {
  WAFER_TRY(prologue(ctx, format, "head_permute_rope"));
  if (tokens == 0 || heads == 0 || head_dim == 0) return WAFER_HIP_OK;
  if (!src || !dst || !positions) return fail(WAFER_HIP_E_INVALID_FIELD, "head_permute_rope: null tensor");
  if (head_dim % 16 || token_stride % 8)
    return fail(WAFER_HIP_E_UNSUPPORTED, "head_permute_rope: head_dim must be a multiple of 16, token_stride of 8");
  if (token_stride < heads * head_dim)
    return fail(WAFER_HIP_E_INVALID_FIELD, "head_permute_rope: token_stride < heads * head_dim");
  if (!aligned16(src) || !aligned16(dst))
    return fail(WAFER_HIP_E_INVALID_FIELD, "head_permute_rope: tensors must be 16-byte aligned");
  if (head_dim <= 128) {  // one wave per (token, head group); the loop keeps the grid bounded
    const uint64_t waves = tokens * ((heads + 64 / (head_dim / 16) - 1) / (64 / (head_dim / 16)));
    const dim3 grid((unsigned)std::min<uint64_t>((waves + 3) / 4, 65536));
    const int64_t a0 = (int64_t)tokens, a1 = (int64_t)heads, a2 = (int64_t)head_dim, a3 = (int64_t)token_stride;
    if (format == WAFER_FMT_F32)
      hipLaunchKernelGGL(permute_rope_lanes_kernel<WAFER_FMT_F32>, grid, dim3(256), 0, ctx->stream, src, dst, a0, a1,
                         a2, a3, positions, theta);
    else if (format == WAFER_FMT_BF16)
      hipLaunchKernelGGL(permute_rope_lanes_kernel<WAFER_FMT_BF16>, grid, dim3(256), 0, ctx->stream, src, dst, a0,
                         a1, a2, a3, positions, theta);
    else
      hipLaunchKernelGGL(permute_rope_lanes_kernel<WAFER_FMT_F16>, grid, dim3(256), 0, ctx->stream, src, dst, a0, a1,
                         a2, a3, positions, theta);
    return launch_status("permute_rope_lanes_kernel");
  }
  // head_dim above 128: the largest head group (8, 4, 2, 1) that keeps the
  // grid at 32768 threads or more: the cos/sin work shrinks with the group,
  // the memory parallelism with the thread count
  const uint64_t rows = tokens * (head_dim / 16);
  int hg = 8;
  while (hg > 1 && rows * ((heads + hg - 1) / hg) < 32768) hg /= 2;
  const uint64_t total = rows * ((heads + hg - 1) / hg);
  const dim3 grid(grid_for(total));
  const int64_t a0 = (int64_t)tokens, a1 = (int64_t)heads, a2 = (int64_t)head_dim, a3 = (int64_t)token_stride;
  if (format == WAFER_FMT_F32)
    launch_permute_rope<WAFER_FMT_F32>(ctx->stream, hg, grid, src, dst, a0, a1, a2, a3, positions, theta);
  else if (format == WAFER_FMT_BF16)
    launch_permute_rope<WAFER_FMT_BF16>(ctx->stream, hg, grid, src, dst, a0, a1, a2, a3, positions, theta);
  else
    launch_permute_rope<WAFER_FMT_F16>(ctx->stream, hg, grid, src, dst, a0, a1, a2, a3, positions, theta);
  return launch_status("permute_rope_kernel");
}

extern "C" int wafer_hip_bias_add(wafer_hip_context *ctx, uint32_t format, const void *x,
                                  const float *bias, void *y, uint64_t rows, uint64_t cols) {
  WAFER_TRY(prologue(ctx, format, "bias_add"));
  if (rows * cols == 0) return WAFER_HIP_OK;
  if (!x || !bias || !y) return fail(WAFER_HIP_E_INVALID_FIELD, "bias_add: null tensor");
  const bool vec = cols % 8 == 0 && aligned16(x) && aligned16(bias) && aligned16(y);
  DISPATCH_FB(format, vec, bias_add_kernel, dim3(grid_for(vec ? rows * cols / 8 : rows * cols)), dim3(256), x,
              bias, y, (int64_t)rows, (int64_t)cols);
  return launch_status("bias_add_kernel");
}
