// comparator.hip -- the program-boundary output gate and error statistics
// on the GPU: compareProgramTensorExpectedOutput and
// computeProgramTensorComparisonStatistics
// (lib/Wafer/Simulator/Invocation/ProgramTensorComparison.cpp:267-497,
// include/Wafer/Simulator/Invocation/ProgramTensorComparison.h:35-71).
//
// Both tensors stay in HBM.  One pass accumulates, per element of an F16 /
// BF16 / F32 pair decoded exactly to double: the similarity sums (dot,
// |a|^2, |e|^2, |a-e|^2) and the absolute-error sum (plain double within
// groups of eight elements, compensated per thread, double-double across
// threads: an error bound of about ten units in the last place of a double,
// independent of the element count, where the reference's in-order long
// double sums carry n * 2^-64), exact and
// mismatch counts, the ULP-distance sum (exact, integer), maxima, the first
// element that ends the comparison (non-finite actual / expected, non-finite
// tolerance) and the mismatch samples the reference reports (first mismatch,
// largest absolute error, largest error/tolerance ratio; ties keep the first
// element).  Per-block partials are merged in a fixed order, so results are
// deterministic.
//
// Nearest-rank p99 / p999 of the absolute error and of the ULP distance are
// found by radix selection over the exact keys (the bits of the nonnegative
// double |a-e|, which order like the values, and the integer ULP distance):
// a pass histograms one 8-bit digit of every key that matches the prefix
// chosen so far, a one-block step kernel picks the digit that holds the
// wanted rank.  The digits start at the top set bit of the largest key, so a
// ULP distance of at most 255 needs one pass.  The selected value is the
// reference's sorted[rank - 1] exactly.
#include "common.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace wafer {
namespace {

constexpr uint64_t NONE = ~uint64_t(0);
constexpr int NT = 256;

// ---- double-double accumulation (Knuth's TwoSum) ----------------------------
struct DD {
  double hi, lo;
};
__device__ inline DD dd_add(DD a, double b) {
  const double s = a.hi + b;
  const double bb = s - a.hi;
  double e = (a.hi - (s - bb)) + (b - bb);
  e += a.lo;
  const double hi = s + e;
  return {hi, e - (hi - s)};
}
__device__ inline DD dd_add(DD a, DD b) { return dd_add(dd_add(a, b.hi), b.lo); }

// Per-thread running sums use Kahan's compensated summation (sum in hi, the
// running compensation in lo; error about 2u times the sum of magnitudes,
// independent of the count), converted to double-double for the merges.
__device__ inline void kahan_add(DD &k, double x) {
  const double y = x - k.lo;
  const double t = k.hi + y;
  k.lo = (t - k.hi) - y;
  k.hi = t;
}
__device__ inline DD kahan_to_dd(DD k) { return dd_add(DD{k.hi, 0.0}, -k.lo); }

struct Acc {
  DD dot, aa, bb, ee, abs;
  uint64_t exact, mism, ulp_sum, max_ulp;
  uint64_t bad;  // 4 * element + kind (1 actual, 2 expected non-finite, 3 tolerance)
  uint64_t first_mm, mm_abs_idx, mm_ratio_idx;
  double max_abs, mm_abs, mm_ratio;
};

__device__ inline void acc_init(Acc &a) {
  a.dot = a.aa = a.bb = a.ee = a.abs = DD{0.0, 0.0};
  a.exact = a.mism = a.ulp_sum = a.max_ulp = 0;
  a.bad = a.first_mm = a.mm_abs_idx = a.mm_ratio_idx = NONE;
  a.max_abs = 0.0;
  a.mm_abs = a.mm_ratio = -1.0;
}

// keep (value desc, element asc): the reference updates on a strictly
// larger value while scanning in element order
__device__ inline void take_max(double &v, uint64_t &i, double v2, uint64_t i2) {
  if (i2 == NONE) return;
  if (i == NONE || v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

__device__ inline void acc_merge(Acc &a, const Acc &b) {
  a.dot = dd_add(a.dot, b.dot);
  a.aa = dd_add(a.aa, b.aa);
  a.bb = dd_add(a.bb, b.bb);
  a.ee = dd_add(a.ee, b.ee);
  a.abs = dd_add(a.abs, b.abs);
  a.exact += b.exact;
  a.mism += b.mism;
  a.ulp_sum += b.ulp_sum;
  a.max_ulp = a.max_ulp > b.max_ulp ? a.max_ulp : b.max_ulp;
  a.max_abs = a.max_abs > b.max_abs ? a.max_abs : b.max_abs;
  a.bad = a.bad < b.bad ? a.bad : b.bad;
  a.first_mm = a.first_mm < b.first_mm ? a.first_mm : b.first_mm;
  take_max(a.mm_abs, a.mm_abs_idx, b.mm_abs, b.mm_abs_idx);
  take_max(a.mm_ratio, a.mm_ratio_idx, b.mm_ratio, b.mm_ratio_idx);
}

// ---- element decoding ----------------------------------------------------------
// decodeBinaryFloat (ProgramTensorComparison.cpp:87-112): exact in double;
// an all-ones exponent is non-finite.
template <uint32_t F> __device__ inline bool decode(uint32_t bits, double &v) {
  if constexpr (F == WAFER_FMT_F32) {
    v = (double)u2f(bits);
    return ((bits >> 23) & 0xffu) != 0xffu;
  } else if constexpr (F == WAFER_FMT_BF16) {
    v = (double)bf16_to_f32((uint16_t)bits);
    return ((bits >> 7) & 0xffu) != 0xffu;
  } else {
    // v_cvt_f32_f16 widens every finite f16 exactly (subnormals included)
    v = (double)(float)__builtin_bit_cast(_Float16, (uint16_t)bits);
    return ((bits >> 10) & 0x1fu) != 0x1fu;
  }
}

// getUlpOrderKey (ProgramTensorComparison.cpp:147-152): sign-aware monotonic
// key of the storage bits
template <uint32_t F> __device__ inline uint64_t order_key(uint32_t bits) {
  constexpr int W = F == WAFER_FMT_F32 ? 32 : 16;
  const uint64_t sign = uint64_t(1) << (W - 1);
  const uint64_t mag = (uint64_t)bits & (sign - 1);
  return ((uint64_t)bits & sign) ? sign - mag : sign + mag;
}

template <uint32_t F> __device__ inline uint64_t ulp_distance(uint32_t ab, uint32_t eb, double av, double ev) {
  if (av == ev) return 0;
  const uint64_t ka = order_key<F>(ab), ke = order_key<F>(eb);
  return ka >= ke ? ka - ke : ke - ka;
}

// What a pass accumulates: everything (the statistics entry), the
// elementwise gate (mismatch count and samples) or the similarity gate
// (similarity sums and the mismatch count).
enum Mode { FULL = 0, GATE_ELEMENTWISE = 1, GATE_SIMILARITY = 2 };

template <uint32_t F, int MODE>
__device__ inline void visit(Acc &a, uint64_t i, uint32_t ab, uint32_t eb, double atol, double rtol) {
  double av, ev;
  const bool fa = decode<F>(ab, av), fe = decode<F>(eb, ev);
  if (!fa || !fe) {
    const uint64_t code = 4 * i + (fa ? 2 : 1);
    a.bad = a.bad < code ? a.bad : code;
    return;
  }
  const double ad = fabs(av - ev);
  const double tol = atol + rtol * fabs(ev);
  if (!isfinite(tol)) {
    a.bad = a.bad < 4 * i + 3 ? a.bad : 4 * i + 3;
    return;
  }
  if constexpr (MODE != GATE_ELEMENTWISE) {
    kahan_add(a.dot, av * ev);
    kahan_add(a.aa, av * av);
    kahan_add(a.bb, ev * ev);
    const double d = av - ev;
    kahan_add(a.ee, d * d);
  }
  if constexpr (MODE == FULL) {
    kahan_add(a.abs, ad);
    a.exact += ad == 0.0;
    const uint64_t u = ulp_distance<F>(ab, eb, av, ev);
    a.ulp_sum += u;
    a.max_ulp = a.max_ulp > u ? a.max_ulp : u;
    a.max_abs = a.max_abs > ad ? a.max_abs : ad;
  }
  if (ad > tol) {
    ++a.mism;
    if constexpr (MODE != GATE_SIMILARITY) {
      if (a.first_mm == NONE) a.first_mm = i;
      take_max(a.mm_abs, a.mm_abs_idx, ad, i);
      take_max(a.mm_ratio, a.mm_ratio_idx, tol == 0.0 ? INFINITY : ad / tol, i);
    }
  }
}

// Eight consecutive elements i0..i0+7, as visit() does them one by one,
// except that the similarity sums (and the absolute-error sum) of the group
// are first formed in plain double -- each term added with one rounding
// (fma of the exact product, which is exact for F16 / BF16 / F32 operands)
// -- and only the group sums go into the compensated per-thread sums.  The
// error bound grows from Kahan's ~2u to ~10u of the sum of magnitudes, still
// a few units in the last place of a double, and the f64 work per element
// falls about threefold (the pass was bound by f64 issue, not HBM).
// Elements that end the comparison (non-finite input or tolerance)
// contribute no terms, as in visit().
template <uint32_t F, int MODE>
__device__ inline void visit8(Acc &a, uint64_t i0, const uint32_t (&ab)[8], const uint32_t (&eb)[8], double atol,
                              double rtol) {
  double pd = 0.0, pa = 0.0, pb = 0.0, pe = 0.0, pabs = 0.0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint64_t i = i0 + e;
    double av, ev;
    const bool fa = decode<F>(ab[e], av), fe = decode<F>(eb[e], ev);
    if (!fa || !fe) {
      const uint64_t code = 4 * i + (fa ? 2 : 1);
      a.bad = a.bad < code ? a.bad : code;
      continue;
    }
    const double ad = fabs(av - ev);
    const double tol = atol + rtol * fabs(ev);
    if (!isfinite(tol)) {
      a.bad = a.bad < 4 * i + 3 ? a.bad : 4 * i + 3;
      continue;
    }
    if constexpr (MODE != GATE_ELEMENTWISE) {
      pd = __builtin_fma(av, ev, pd);
      pa = __builtin_fma(av, av, pa);
      pb = __builtin_fma(ev, ev, pb);
      const double d = av - ev;
      pe = __builtin_fma(d, d, pe);
    }
    if constexpr (MODE == FULL) {
      pabs += ad;
      a.exact += ad == 0.0;
      const uint64_t u = ulp_distance<F>(ab[e], eb[e], av, ev);
      a.ulp_sum += u;
      a.max_ulp = a.max_ulp > u ? a.max_ulp : u;
      a.max_abs = a.max_abs > ad ? a.max_abs : ad;
    }
    if (ad > tol) {
      ++a.mism;
      if constexpr (MODE != GATE_SIMILARITY) {
        if (a.first_mm == NONE) a.first_mm = i;
        take_max(a.mm_abs, a.mm_abs_idx, ad, i);
        take_max(a.mm_ratio, a.mm_ratio_idx, tol == 0.0 ? INFINITY : ad / tol, i);
      }
    }
  }
  if constexpr (MODE != GATE_ELEMENTWISE) {
    kahan_add(a.dot, pd);
    kahan_add(a.aa, pa);
    kahan_add(a.bb, pb);
    kahan_add(a.ee, pe);
  }
  if constexpr (MODE == FULL) kahan_add(a.abs, pabs);
}

// Raw storage bits of element i.
template <uint32_t F> __device__ inline uint32_t bits_at(const void *p, uint64_t i) {
  if constexpr (F == WAFER_FMT_F32)
    return ((const uint32_t *)p)[i];
  else
    return ((const uint16_t *)p)[i];
}

// The raw 16-byte words holding eight consecutive elements (one for 16-bit
// formats, two for F32; bases 16-byte aligned, i a multiple of 8), and their
// split into per-element bits.
struct Raw8 {
  u32x4 lo, hi;
};
template <uint32_t F> __device__ inline Raw8 raw8(const void *p, uint64_t i) {
  Raw8 r;
  if constexpr (F == WAFER_FMT_F32) {
    r.lo = ((const u32x4 *)p)[i / 4];
    r.hi = ((const u32x4 *)p)[i / 4 + 1];
  } else {
    r.lo = ((const u32x4 *)p)[i / 8];
    r.hi = r.lo;
  }
  return r;
}
template <uint32_t F> __device__ inline void unpack8(const Raw8 &r, uint32_t (&b)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (F == WAFER_FMT_F32) {
      b[e] = r.lo[e];
      b[4 + e] = r.hi[e];
    } else {
      b[2 * e] = r.lo[e] & 0xffffu;
      b[2 * e + 1] = r.lo[e] >> 16;
    }
  }
}

// Eight consecutive elements' bits with 16-byte loads (bases 16-byte aligned,
// i a multiple of 8).
template <uint32_t F> __device__ inline void bits8(const void *p, uint64_t i, uint32_t (&b)[8]) {
  if constexpr (F == WAFER_FMT_F32) {
    const u32x4 lo = ((const u32x4 *)p)[i / 4], hi = ((const u32x4 *)p)[i / 4 + 1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      b[e] = lo[e];
      b[4 + e] = hi[e];
    }
  } else {
    const u32x4 w = ((const u32x4 *)p)[i / 8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      b[2 * e] = w[e] & 0xffffu;
      b[2 * e + 1] = w[e] >> 16;
    }
  }
}

// Visits every element in groups of eight: lane-contiguous groups, then a
// scalar tail.  fn(i, actual_bits, expected_bits).
template <uint32_t F, typename Fn>
__device__ inline void for_each_element(const void *act, const void *exp, uint64_t n, bool vec, Fn &&fn) {
  const uint64_t groups = vec ? n / 8 : 0;
  const uint64_t step = (uint64_t)gridDim.x * NT;
  for (uint64_t g = (uint64_t)blockIdx.x * NT + threadIdx.x; g < groups; g += step) {
    uint32_t ab[8], eb[8];
    bits8<F>(act, g * 8, ab);
    bits8<F>(exp, g * 8, eb);
#pragma unroll
    for (int e = 0; e < 8; ++e) fn(g * 8 + e, ab[e], eb[e]);
  }
  for (uint64_t i = groups * 8 + (uint64_t)blockIdx.x * NT + threadIdx.x; i < n; i += step)
    fn(i, bits_at<F>(act, i), bits_at<F>(exp, i));
}

__device__ inline DD shfl_xor(DD v, int m) { return {__shfl_xor(v.hi, m), __shfl_xor(v.lo, m)}; }
__device__ inline uint64_t shfl_xor(uint64_t v, int m) { return (uint64_t)__shfl_xor((unsigned long long)v, m); }
__device__ inline double shfl_xor(double v, int m) { return __shfl_xor(v, m); }

// Merges the accumulators of a block: butterfly within each wave (fixed
// pairing, so the result is deterministic), then the four wave results in
// wave order.  Thread 0 holds the block's total.
__device__ inline void block_reduce(Acc &a) {
  for (int m = 1; m < 64; m *= 2) {
    Acc o;
    o.dot = shfl_xor(a.dot, m);
    o.aa = shfl_xor(a.aa, m);
    o.bb = shfl_xor(a.bb, m);
    o.ee = shfl_xor(a.ee, m);
    o.abs = shfl_xor(a.abs, m);
    o.exact = shfl_xor(a.exact, m);
    o.mism = shfl_xor(a.mism, m);
    o.ulp_sum = shfl_xor(a.ulp_sum, m);
    o.max_ulp = shfl_xor(a.max_ulp, m);
    o.bad = shfl_xor(a.bad, m);
    o.first_mm = shfl_xor(a.first_mm, m);
    o.mm_abs_idx = shfl_xor(a.mm_abs_idx, m);
    o.mm_ratio_idx = shfl_xor(a.mm_ratio_idx, m);
    o.max_abs = shfl_xor(a.max_abs, m);
    o.mm_abs = shfl_xor(a.mm_abs, m);
    o.mm_ratio = shfl_xor(a.mm_ratio, m);
    // the lower lane of each pair keeps (lower, upper) order
    if (threadIdx.x & m) {
      Acc t = o;
      acc_merge(t, a);
      a = t;
    } else {
      acc_merge(a, o);
    }
  }
  __shared__ Acc waves[NT / 64];
  if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = a;
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < NT / 64; ++w) acc_merge(a, waves[w]);
}

template <uint32_t F, int MODE>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void stats_kernel(const void *__restrict__ act, const void *__restrict__ exp,
                                                   uint64_t n, bool vec, double atol, double rtol,
                                                   Acc *__restrict__ partials) {
  Acc a;
  acc_init(a);
  const uint64_t groups = vec ? n / 8 : 0;
  const uint64_t step = (uint64_t)gridDim.x * NT;
  // the next group's 16-byte loads are issued before the current group is
  // visited, so their latency hides behind that work
  uint64_t g = (uint64_t)blockIdx.x * NT + threadIdx.x;
  Raw8 na{}, ne{};
  if (g < groups) {
    na = raw8<F>(act, g * 8);
    ne = raw8<F>(exp, g * 8);
  }
  for (; g < groups; g += step) {
    const Raw8 ca = na, ce = ne;
    if (g + step < groups) {
      na = raw8<F>(act, (g + step) * 8);
      ne = raw8<F>(exp, (g + step) * 8);
    }
    uint32_t ab[8], eb[8];
    unpack8<F>(ca, ab);
    unpack8<F>(ce, eb);
    visit8<F, MODE>(a, g * 8, ab, eb, atol, rtol);
  }
  for (uint64_t i = groups * 8 + (uint64_t)blockIdx.x * NT + threadIdx.x; i < n; i += step)
    visit<F, MODE>(a, i, bits_at<F>(act, i), bits_at<F>(exp, i), atol, rtol);
  a.dot = kahan_to_dd(a.dot);
  a.aa = kahan_to_dd(a.aa);
  a.bb = kahan_to_dd(a.bb);
  a.ee = kahan_to_dd(a.ee);
  a.abs = kahan_to_dd(a.abs);
  block_reduce(a);
  if (threadIdx.x == 0) partials[blockIdx.x] = a;
}

// ---- radix selection ---------------------------------------------------------------
// Selection targets: 0 p99 |a-e|, 1 p999 |a-e|, 2 p99 ULP, 3 p999 ULP.
// Digits are DIG bits wide, taken from the top set bit of the largest key
// down; bits on which every remaining candidate agrees (the AND and OR of
// the candidate keys of the last pass) are fixed without a pass.  The
// per-target histograms are summed in HBM (64-bit atomics), and a target
// whose state equals the previous target's (same key, same prefix so far)
// shares that target's histogram.
constexpr int DIG = 11, BINS = 1 << DIG;

struct Select {
  uint64_t prefix, mask, k, result;
  int32_t shift, width, done, pad;
};

__device__ inline void select_init(Select &s, uint64_t maxkey, uint64_t k) {
  s.prefix = s.mask = 0;
  s.k = k;
  s.result = 0;
  s.pad = 0;
  if (maxkey == 0) {
    s.done = 1;
    s.shift = s.width = 0;
    return;
  }
  const int msb = 63 - __builtin_clzll(maxkey);
  s.shift = msb >= DIG - 1 ? msb - (DIG - 1) : 0;
  s.width = msb - s.shift + 1;
  s.done = 0;
}

__host__ __device__ inline int passes_for(uint64_t maxkey) {
  if (maxkey == 0) return 0;
  const int bits = 64 - __builtin_clzll(maxkey);
  return (bits + DIG - 1) / DIG;
}

__device__ inline bool same_state(const Select &a, const Select &b) {
  return !a.done && !b.done && a.prefix == b.prefix && a.mask == b.mask && a.shift == b.shift &&
         a.width == b.width;
}

// Merges the per-block partials in block order, seeds the selections and
// clears the histogram sums.
__global__ __launch_bounds__(NT) void finalize_kernel(const Acc *__restrict__ partials, int blocks,
                                                      Acc *__restrict__ out, Select *__restrict__ sel,
                                                      unsigned long long *__restrict__ ghist, uint64_t k99,
                                                      uint64_t k999) {
  for (int i = threadIdx.x; i < 4 * BINS; i += NT) ghist[i] = 0;
  if (threadIdx.x < 4) {
    ghist[4 * BINS + threadIdx.x] = ~0ull;  // AND of candidate keys
    ghist[4 * BINS + 4 + threadIdx.x] = 0;  // OR of candidate keys
  }
  Acc a;
  acc_init(a);
  for (int b = threadIdx.x; b < blocks; b += NT) acc_merge(a, partials[b]);
  block_reduce(a);
  if (threadIdx.x == 0) {
    *out = a;
    const uint64_t abs_max = (uint64_t)__double_as_longlong(a.max_abs);
    select_init(sel[0], abs_max, k99);
    select_init(sel[1], abs_max, k999);
    select_init(sel[2], a.max_ulp, k99);
    select_init(sel[3], a.max_ulp, k999);
  }
}

// Adds one to bin b of a block histogram; lanes of a wave that share a bin
// (common: most errors are zero or equal) add with one atomic per bin for
// the two most frequent leaders, the rest add individually.
__device__ inline void hist_add(uint32_t *h, bool on, uint32_t b) {
  bool pending = on;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const uint64_t pm = __ballot(pending);
    if (pm == 0) return;
    const int leader = __builtin_ctzll(pm);
    const uint32_t lb = __builtin_amdgcn_readlane(b, leader);
    const bool mine = pending && b == lb;
    const uint64_t m = __ballot(mine);
    if ((int)(threadIdx.x & 63) == leader) atomicAdd(&h[lb], (uint32_t)__popcll(m));
    pending = pending && !mine;
  }
  if (pending) atomicAdd(&h[b], 1u);
}

template <uint32_t F>
__global__ __launch_bounds__(NT) void select_hist_kernel(const void *__restrict__ act, const void *__restrict__ exp,
                                                         uint64_t n, bool vec, const Select *__restrict__ sel,
                                                         unsigned long long *__restrict__ ghist) {
  __shared__ uint32_t h[4][BINS];
  __shared__ Select s[4];
  __shared__ int live[4];
  if (threadIdx.x < 4) s[threadIdx.x] = sel[threadIdx.x];
  __syncthreads();
  if (threadIdx.x < 4) {
    const int t = threadIdx.x;
    live[t] = !s[t].done && !((t & 1) && same_state(s[t - 1], s[t]));
  }
  for (int i = threadIdx.x; i < 4 * BINS; i += NT) (&h[0][0])[i] = 0;
  __syncthreads();
  if (!live[0] && !live[1] && !live[2] && !live[3]) return;
  uint64_t kand[4] = {~0ull, ~0ull, ~0ull, ~0ull}, kor[4] = {0, 0, 0, 0};
  for_each_element<F>(act, exp, n, vec, [&](uint64_t, uint32_t ab, uint32_t eb) {
    double av, ev;
    decode<F>(ab, av);
    decode<F>(eb, ev);
    uint64_t key[4];
    key[0] = key[1] = (uint64_t)__double_as_longlong(fabs(av - ev));
    key[2] = key[3] = ulp_distance<F>(ab, eb, av, ev);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (!live[t]) continue;  // uniform
      const bool on = (key[t] & s[t].mask) == s[t].prefix;
      const uint32_t b = (uint32_t)((key[t] >> s[t].shift) & ((uint64_t(1) << s[t].width) - 1));
      if (on) {
        kand[t] &= key[t];
        kor[t] |= key[t];
      }
      hist_add(h[t], on, b);
    }
  });
  __syncthreads();
  for (int i = threadIdx.x; i < 4 * BINS; i += NT) {
    const uint32_t c = (&h[0][0])[i];
    if (c) atomicAdd(&ghist[i], (unsigned long long)c);
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (!live[t]) continue;
    for (int m = 1; m < 64; m *= 2) {
      kand[t] &= shfl_xor(kand[t], m);
      kor[t] |= shfl_xor(kor[t], m);
    }
    if ((threadIdx.x & 63) == 0) {
      atomicAnd(&ghist[4 * BINS + t], (unsigned long long)kand[t]);
      atomicOr(&ghist[4 * BINS + 4 + t], (unsigned long long)kor[t]);
    }
  }
}

// One block: for each target, find the digit that holds rank k in the
// summed histogram (its own, or the shared one), narrow the prefix; then
// clear the sums for the next pass.
__global__ __launch_bounds__(NT) void select_step_kernel(unsigned long long *__restrict__ ghist,
                                                         Select *__restrict__ sel) {
  constexpr int PER = BINS / NT;
  __shared__ Select s[4];
  __shared__ int src[4];
  __shared__ uint64_t scan[NT];
  __shared__ int found;
  __shared__ uint64_t found_below;
  if (threadIdx.x < 4) s[threadIdx.x] = sel[threadIdx.x];
  __syncthreads();
  if (threadIdx.x < 4) {
    const int t = threadIdx.x;
    src[t] = (t & 1) && same_state(s[t - 1], s[t]) ? t - 1 : t;
  }
  __syncthreads();
  for (int t = 0; t < 4; ++t) {
    if (s[t].done) continue;  // uniform
    const unsigned long long *hc = ghist + src[t] * BINS;
    uint64_t c[PER], sum = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      c[j] = hc[threadIdx.x * PER + j];
      sum += c[j];
    }
    scan[threadIdx.x] = sum;
    __syncthreads();
    // inclusive scan over the per-thread sums (Hillis-Steele)
    for (int d = 1; d < NT; d *= 2) {
      const uint64_t v = threadIdx.x >= d ? scan[threadIdx.x - d] : 0;
      __syncthreads();
      scan[threadIdx.x] += v;
      __syncthreads();
    }
    if (threadIdx.x == 0) found = -1;
    __syncthreads();
    const uint64_t before = scan[threadIdx.x] - sum, k = s[t].k;
    if (before < k && k <= scan[threadIdx.x]) {
      uint64_t below = before;
      int bin = threadIdx.x * PER + PER - 1;
      for (int j = 0; j < PER; ++j) {
        if (below + c[j] >= k) {
          bin = threadIdx.x * PER + j;
          break;
        }
        below += c[j];
      }
      found = bin;
      found_below = below;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      Select &x = s[t];
      // k never exceeds the count of keys under the prefix; the last bin is
      // a guard that keeps the state well-formed
      const int bin = found >= 0 ? found : (1 << x.width) - 1;
      x.k -= found >= 0 ? found_below : 0;
      x.prefix |= (uint64_t)bin << x.shift;
      x.mask |= ((uint64_t(1) << x.width) - 1) << x.shift;
      // bits below the digit on which every candidate of this pass agrees
      // hold the same value in the answer: fix them, then start the next
      // digit at the highest bit that still varies
      const uint64_t low = x.shift ? (uint64_t(1) << x.shift) - 1 : 0;
      const uint64_t kand = ghist[4 * BINS + src[t]], kor = ghist[4 * BINS + 4 + src[t]];
      const uint64_t fixed = ~(kand ^ kor) & low;
      x.prefix |= kand & fixed;
      x.mask |= fixed;
      const uint64_t varying = low & ~x.mask;
      if (varying == 0) {
        x.done = 1;
        x.result = x.prefix;
      } else {
        const int msb = 63 - __builtin_clzll(varying);
        x.shift = msb >= DIG - 1 ? msb - (DIG - 1) : 0;
        x.width = msb - x.shift + 1;
      }
    }
    __syncthreads();
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 4 * BINS; i += NT) ghist[i] = 0;
  if (threadIdx.x < 4) {
    ghist[4 * BINS + threadIdx.x] = ~0ull;
    ghist[4 * BINS + 4 + threadIdx.x] = 0;
    sel[threadIdx.x] = s[threadIdx.x];
  }
}

// Raw comparison: first differing byte.
__global__ __launch_bounds__(NT) void raw_diff_kernel(const uint8_t *__restrict__ a, const uint8_t *__restrict__ b,
                                                      uint64_t n, unsigned long long *__restrict__ first) {
  const uint64_t step = (uint64_t)gridDim.x * NT;
  for (uint64_t i = (uint64_t)blockIdx.x * NT + threadIdx.x; i < n; i += step)
    if (a[i] != b[i]) {
      atomicMin(first, (unsigned long long)i);
      return;
    }
}

// ---- host side ---------------------------------------------------------------------
// ProgramElementType (include/Wafer/Frontend/ProgramElementType.h:17-32)
const char *dtype_name(uint32_t d) {
  static const char *names[] = {"bool", "i8",  "u8",  "i16", "u16",  "i32",  "u32",
                                "i64",  "u64", "f16", "bf16", "f32", "tf32", "f64"};
  return d < 14 ? names[d] : "unknown";
}
int dtype_bytes(uint32_t d) {
  switch (d) {
  case WAFER_DT_BOOL: case WAFER_DT_I8: case WAFER_DT_U8: return 1;
  case WAFER_DT_I16: case WAFER_DT_U16: case WAFER_DT_F16: case WAFER_DT_BF16: return 2;
  case WAFER_DT_I32: case WAFER_DT_U32: case WAFER_DT_F32: case WAFER_DT_TF32: return 4;
  case WAFER_DT_I64: case WAFER_DT_U64: case WAFER_DT_F64: return 8;
  default: return 0;
  }
}
bool dtype_floating(uint32_t d) { return d >= WAFER_DT_F16 && d <= WAFER_DT_F64; }
bool dtype_tolerant(uint32_t d) { return d == WAFER_DT_F16 || d == WAFER_DT_BF16 || d == WAFER_DT_F32; }
uint32_t storage_format(uint32_t d) {
  return d == WAFER_DT_F16 ? WAFER_FMT_F16 : d == WAFER_DT_BF16 ? WAFER_FMT_BF16 : WAFER_FMT_F32;
}

std::string shape_string(const wafer_hip_program_tensor *t) {
  std::string s = "[";
  for (uint32_t i = 0; i < t->rank; ++i) {
    if (i) s += ',';
    s += std::to_string(t->shape[i]);
  }
  return s + "]";
}

// raw_ostream prints doubles as %e
std::string fmt_e(double v) {
  char b[64];
  snprintf(b, sizeof b, "%e", v);
  return b;
}

struct Verdict {
  uint32_t *code;
  char *detail;
  size_t detail_bytes;
  int set(uint32_t c, const std::string &d) {
    *code = c;
    if (detail && detail_bytes) {
      const size_t n = std::min(d.size(), detail_bytes - 1);
      memcpy(detail, d.data(), n);
      detail[n] = 0;
    }
    return WAFER_HIP_OK;
  }
};

int check_tensor(const wafer_hip_program_tensor *t, const char *role) {
  if (!t) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(role) + ": null tensor");
  const int eb = dtype_bytes(t->dtype);
  if (eb == 0) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(role) + ": unknown dtype");
  if (t->rank && !t->shape) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(role) + ": null shape");
  uint64_t bytes = (uint64_t)eb;
  for (uint32_t i = 0; i < t->rank; ++i) {
    if (t->shape[i] < 0) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(role) + ": negative extent");
    if (t->shape[i] && bytes > UINT64_MAX / (uint64_t)t->shape[i])
      return fail(WAFER_HIP_E_INVALID_FIELD, std::string(role) + ": byte count overflows");
    bytes *= (uint64_t)t->shape[i];
  }
  // ProgramTensor::create (ProgramInvocation.cpp:139-149)
  if (bytes != t->bytes)
    return fail(WAFER_HIP_E_INVALID_FIELD, std::string(role) + ": byte count disagrees with dtype and shape");
  if (bytes && !t->data) return fail(WAFER_HIP_E_INVALID_FIELD, std::string(role) + ": null data");
  return WAFER_HIP_OK;
}

// validateProgramTensorComparisonPolicy (ProgramTensorComparison.cpp:499-516)
bool policy_valid(const wafer_hip_comparison_policy &p) {
  if (!std::isfinite(p.atol) || !std::isfinite(p.rtol) || p.atol < 0.0 || p.rtol < 0.0) return false;
  if (p.has_similarity && (!std::isfinite(p.minimum_cosine) || p.minimum_cosine < 0.0 || p.minimum_cosine > 1.0 ||
                           !std::isfinite(p.maximum_relative_l2) || p.maximum_relative_l2 < 0.0))
    return false;
  return true;
}
const char *policy_message(const wafer_hip_comparison_policy &p) {
  if (!std::isfinite(p.atol) || !std::isfinite(p.rtol) || p.atol < 0.0 || p.rtol < 0.0)
    return "absolute and relative tolerances must be finite and nonnegative";
  return "similarity requires finite minimum cosine in [0,1] and nonnegative relative L2";
}

// Metadata checks shared by both entries, in the reference's order.  Returns
// true when a verdict was set.
bool metadata_verdict(const wafer_hip_program_tensor *a, const wafer_hip_program_tensor *e, Verdict &v) {
  if (a->dtype != e->dtype) {
    v.set(WAFER_CMP_DTYPE_MISMATCH, std::string("actual=") + dtype_name(a->dtype) + " expected=" + dtype_name(e->dtype));
    return true;
  }
  bool same = a->rank == e->rank;
  for (uint32_t i = 0; same && i < a->rank; ++i) same = a->shape[i] == e->shape[i];
  if (!same) {
    v.set(WAFER_CMP_SHAPE_MISMATCH, "actual=" + shape_string(a) + " expected=" + shape_string(e));
    return true;
  }
  if (a->bytes != e->bytes) {
    v.set(WAFER_CMP_BYTE_SIZE_MISMATCH, "actual=" + std::to_string(a->bytes) + " expected=" + std::to_string(e->bytes));
    return true;
  }
  return false;
}

// Host image of the merged accumulator: sums as long double (hi + lo).
struct Totals {
  long double dot, aa, bb, ee, abs;
  uint64_t exact, mism, ulp_sum, max_ulp, bad, first_mm, mm_abs_idx, mm_ratio_idx;
  double max_abs;
  uint64_t q_abs99, q_abs999, q_ulp99, q_ulp999;
};

long double ld(const DD &d) { return (long double)d.hi + (long double)d.lo; }

// TensorSimilarity::cosine / relativeL2 (ProgramTensorComparison.cpp:23-51)
double cosine_of(const Totals &t) {
  if (t.aa == 0.0L || t.bb == 0.0L) return t.aa == t.bb ? 1.0 : 0.0;
  long double c = t.dot / sqrtl(t.aa) / sqrtl(t.bb);
  c = c < -1.0L ? -1.0L : c > 1.0L ? 1.0L : c;
  return (double)c;
}
double rel_l2_of(const Totals &t) {
  if (t.bb == 0.0L) return t.ee == 0.0L ? 0.0 : INFINITY;
  return (double)sqrtl(t.ee / t.bb);
}

// Runs the statistics pass (and, when `quantiles`, the selections) over n
// finite-format elements; fills `t`.
int run_stats(wafer_hip_context *ctx, uint32_t fmt, const void *act, const void *exp, uint64_t n, double atol,
              double rtol, int mode, Totals &t) {
  const bool quantiles = mode == FULL;
  WAFER_TRY(refuse_capture(ctx, "compare"));  // the statistics are read back to the host
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  const uint64_t want = (n + (uint64_t)NT * 8 - 1) / ((uint64_t)NT * 8);
  // one full round of workgroups: as many per CU as the statistics kernel's
  // registers allow (a second, partial round of a grid-stride pass would
  // hold the whole pass for another block's share)
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)stats_kernel<WAFER_FMT_BF16, FULL>, NT, 0) !=
          hipSuccess ||
      per_cu < 1) {
    (void)hipGetLastError();  // the query's failure is not the launch's
    per_cu = 1;
  }
  const int blocks = (int)std::max<uint64_t>(1, std::min<uint64_t>(want, (uint64_t)cus * per_cu));
  const size_t acc_bytes = ((size_t)blocks + 1) * sizeof(Acc);
  const size_t sel_off = (acc_bytes + 255) & ~size_t(255);
  const size_t hist_off = sel_off + 256;
  const size_t need = hist_off + (size_t)(4 * BINS + 8) * sizeof(unsigned long long);
  WAFER_TRY(ensure_workspace(ctx, &ctx->workspace, &ctx->workspace_bytes, need));
  uint8_t *ws = (uint8_t *)ctx->workspace;
  Acc *partials = (Acc *)ws, *final_acc = partials + blocks;
  Select *sel = (Select *)(ws + sel_off);
  unsigned long long *ghist = (unsigned long long *)(ws + hist_off);
  const bool vec = aligned16(act) && aligned16(exp);
  // nearest rank, ProgramTensorComparison.cpp:164-171
  auto rank = [&](double q) {
    uint64_t r = (uint64_t)std::ceil(q * (double)n);
    return std::max<uint64_t>(1, std::min<uint64_t>(r, n));
  };
#define WAFER_STATS(F, M)                                                                                      \
  hipLaunchKernelGGL((stats_kernel<F, M>), dim3(blocks), dim3(NT), 0, ctx->stream, act, exp, n, vec, atol, rtol, \
                     partials)
#define WAFER_STATS_F(F)                                      \
  do {                                                        \
    if (mode == FULL) WAFER_STATS(F, FULL);                   \
    else if (mode == GATE_ELEMENTWISE) WAFER_STATS(F, GATE_ELEMENTWISE); \
    else WAFER_STATS(F, GATE_SIMILARITY);                     \
  } while (0)
  if (fmt == WAFER_FMT_F32) WAFER_STATS_F(WAFER_FMT_F32);
  else if (fmt == WAFER_FMT_BF16) WAFER_STATS_F(WAFER_FMT_BF16);
  else WAFER_STATS_F(WAFER_FMT_F16);
#undef WAFER_STATS_F
#undef WAFER_STATS
  WAFER_TRY(launch_status("stats_kernel"));
  hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(NT), 0, ctx->stream, partials, blocks, final_acc, sel, ghist,
                     rank(0.99), rank(0.999));
  WAFER_TRY(launch_status("finalize_kernel"));
  Acc h;
  WAFER_TRY(check_hip(hipMemcpyAsync(&h, final_acc, sizeof h, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync"));
  WAFER_TRY(check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize"));
  Select hs[4] = {};
  if (quantiles && h.bad == NONE) {
    // the digits each key needs, from the largest key (known on the host now)
    uint64_t abs_max_bits;
    memcpy(&abs_max_bits, &h.max_abs, 8);
    const int passes = std::max(passes_for(abs_max_bits), passes_for(h.max_ulp));
    for (int pass = 0; pass < passes; ++pass) {
#define WAFER_HIST(F)                                                                                      \
  hipLaunchKernelGGL(select_hist_kernel<F>, dim3(blocks), dim3(NT), 0, ctx->stream, act, exp, n, vec, sel, \
                     ghist)
      if (fmt == WAFER_FMT_F32) WAFER_HIST(WAFER_FMT_F32);
      else if (fmt == WAFER_FMT_BF16) WAFER_HIST(WAFER_FMT_BF16);
      else WAFER_HIST(WAFER_FMT_F16);
#undef WAFER_HIST
      WAFER_TRY(launch_status("select_hist_kernel"));
      hipLaunchKernelGGL(select_step_kernel, dim3(1), dim3(NT), 0, ctx->stream, ghist, sel);
      WAFER_TRY(launch_status("select_step_kernel"));
    }
    WAFER_TRY(check_hip(hipMemcpyAsync(hs, sel, sizeof hs, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync"));
    WAFER_TRY(check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize"));
    for (int i = 0; i < 4; ++i)
      if (!hs[i].done) return fail(WAFER_HIP_E_RUNTIME, "comparison quantile selection did not converge");
  }
  t.dot = ld(h.dot);
  t.aa = ld(h.aa);
  t.bb = ld(h.bb);
  t.ee = ld(h.ee);
  t.abs = ld(h.abs);
  t.exact = h.exact;
  t.mism = h.mism;
  t.ulp_sum = h.ulp_sum;
  t.max_ulp = h.max_ulp;
  t.bad = h.bad;
  t.first_mm = h.first_mm;
  t.mm_abs_idx = h.mm_abs_idx;
  t.mm_ratio_idx = h.mm_ratio_idx;
  t.max_abs = h.max_abs;
  t.q_abs99 = hs[0].result;
  t.q_abs999 = hs[1].result;
  t.q_ulp99 = hs[2].result;
  t.q_ulp999 = hs[3].result;
  return WAFER_HIP_OK;
}

// Element i of a device tensor, decoded on the host (diagnostics only).
int fetch_value(wafer_hip_context *ctx, uint32_t fmt, const void *p, uint64_t i, double &v) {
  uint32_t bits = 0;
  const int eb = fmt == WAFER_FMT_F32 ? 4 : 2;
  WAFER_TRY(check_hip(hipMemcpy(&bits, (const uint8_t *)p + i * eb, eb, hipMemcpyDeviceToHost), "hipMemcpy"));
  v = fmt == WAFER_FMT_F32 ? (double)u2f(bits)
      : fmt == WAFER_FMT_BF16 ? (double)bf16_to_f32((uint16_t)bits)
                              : (double)f16_to_f32((uint16_t)bits);
  return WAFER_HIP_OK;
}

// The verdict for a non-finite value or tolerance at t.bad.
int bad_verdict(const Totals &t, Verdict &v) {
  const uint64_t i = t.bad / 4, kind = t.bad % 4;
  if (kind == 1) return v.set(WAFER_CMP_ACTUAL_NONFINITE, "element=" + std::to_string(i));
  if (kind == 2) return v.set(WAFER_CMP_EXPECTED_NONFINITE, "element=" + std::to_string(i));
  return v.set(WAFER_CMP_INVALID_TOLERANCE, "computed tolerance is not finite at element=" + std::to_string(i));
}

int float_gate(wafer_hip_context *ctx, const wafer_hip_program_tensor *a, const wafer_hip_program_tensor *e,
               const wafer_hip_comparison_policy &p, Verdict &v) {
  const uint32_t fmt = storage_format(a->dtype);
  const uint64_t n = a->bytes / dtype_bytes(a->dtype);
  if (p.has_similarity && n == 0)
    return v.set(WAFER_CMP_UNSUPPORTED_STATISTICS_DTYPE, "similarity requires a non-empty tensor");
  if (n == 0) return v.set(WAFER_CMP_ACCEPTED, "");
  Totals t;
  WAFER_TRY(run_stats(ctx, fmt, a->data, e->data, n, p.atol, p.rtol,
                      p.has_similarity ? GATE_SIMILARITY : GATE_ELEMENTWISE, t));
  if (t.bad != NONE) return bad_verdict(t, v);
  if (p.has_similarity) {
    const double c = cosine_of(t), r = rel_l2_of(t);
    if (c >= p.minimum_cosine && r <= p.maximum_relative_l2) return v.set(WAFER_CMP_ACCEPTED, "");
    return v.set(WAFER_CMP_NUMERIC_MISMATCH, "cosine=" + fmt_e(c) + " minimum_cosine=" + fmt_e(p.minimum_cosine) +
                                                 " relative_l2=" + fmt_e(r) + " maximum_relative_l2=" +
                                                 fmt_e(p.maximum_relative_l2) + " elementwise_mismatches=" +
                                                 std::to_string(t.mism) + "/" + std::to_string(n));
  }
  if (t.mism == 0) return v.set(WAFER_CMP_ACCEPTED, "");
  // numericMismatchSummary (ProgramTensorComparison.cpp:196-220)
  auto sample = [&](uint64_t i, double &tol, double &ad) -> std::string {
    double av = 0, ev = 0;
    fetch_value(ctx, fmt, a->data, i, av);
    fetch_value(ctx, fmt, e->data, i, ev);
    ad = std::fabs(av - ev);
    tol = p.atol + p.rtol * std::fabs(ev);
    return "element=" + std::to_string(i) + " actual=" + fmt_e(av) + " expected=" + fmt_e(ev) +
           " abs_error=" + fmt_e(ad) + " tolerance=" + fmt_e(tol);
  };
  double tol, ad;
  const std::string first = sample(t.first_mm, tol, ad);
  const std::string mx = sample(t.mm_abs_idx, tol, ad);
  sample(t.mm_ratio_idx, tol, ad);
  const double ratio = tol == 0.0 ? INFINITY : ad / tol;
  return v.set(WAFER_CMP_NUMERIC_MISMATCH, "mismatches=" + std::to_string(t.mism) + "/" + std::to_string(n) +
                                               " first={" + first + "} max_abs={" + mx + "} max_tolerance_ratio=" +
                                               fmt_e(ratio) + " at_element=" + std::to_string(t.mm_ratio_idx));
}

int raw_gate(wafer_hip_context *ctx, const wafer_hip_program_tensor *a, const wafer_hip_program_tensor *e,
             Verdict &v) {
  if (a->bytes == 0) return v.set(WAFER_CMP_ACCEPTED, "");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  uint8_t *words = nullptr;
  WAFER_TRY(status_words(ctx, "compare (raw bytes)", &words));
  unsigned long long *first = (unsigned long long *)(words + 64);
  const unsigned long long none = ~0ull;
  WAFER_TRY(fill_words(ctx, first, 2, 0xffffffffu));
  const unsigned grid = (unsigned)std::min<uint64_t>((a->bytes + NT - 1) / NT, 8192);
  hipLaunchKernelGGL(raw_diff_kernel, dim3(grid), dim3(NT), 0, ctx->stream, (const uint8_t *)a->data,
                     (const uint8_t *)e->data, a->bytes, first);
  WAFER_TRY(launch_status("raw_diff_kernel"));
  unsigned long long idx = none;
  WAFER_TRY(check_hip(hipMemcpyAsync(&idx, first, sizeof idx, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync"));
  WAFER_TRY(check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize"));
  if (idx == none) return v.set(WAFER_CMP_ACCEPTED, "");
  uint8_t x = 0, y = 0;
  WAFER_TRY(check_hip(hipMemcpy(&x, (const uint8_t *)a->data + idx, 1, hipMemcpyDeviceToHost), "hipMemcpy"));
  WAFER_TRY(check_hip(hipMemcpy(&y, (const uint8_t *)e->data + idx, 1, hipMemcpyDeviceToHost), "hipMemcpy"));
  return v.set(WAFER_CMP_RAW_MISMATCH, "byte=" + std::to_string(idx) + " actual=" + std::to_string(x) +
                                           " expected=" + std::to_string(y));
}

}  // namespace
}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_compare_expected(wafer_hip_context *ctx, const wafer_hip_program_tensor *actual,
                                          const wafer_hip_program_tensor *expected,
                                          const wafer_hip_comparison_policy *policy, uint32_t *verdict,
                                          char *detail, size_t detail_bytes) {
  WAFER_CHECK_CTX(ctx);
  if (!policy || !verdict) return fail(WAFER_HIP_E_INVALID_FIELD, "compare: null policy or verdict");
  WAFER_TRY(check_tensor(actual, "actual"));
  WAFER_TRY(check_tensor(expected, "expected"));
  Verdict v{verdict, detail, detail_bytes};
  if (!policy_valid(*policy)) return v.set(WAFER_CMP_INVALID_TOLERANCE, policy_message(*policy));
  if (metadata_verdict(actual, expected, v)) return WAFER_HIP_OK;
  const uint32_t d = actual->dtype;
  if (dtype_floating(d) && !dtype_tolerant(d))
    return v.set(WAFER_CMP_UNSUPPORTED_FLOATING_DTYPE,
                 std::string("dtype=") + dtype_name(d) + " has no expected-output policy");
  if (!dtype_tolerant(d)) return raw_gate(ctx, actual, expected, v);
  return float_gate(ctx, actual, expected, *policy, v);
}

extern "C" int wafer_hip_compare_statistics(wafer_hip_context *ctx, const wafer_hip_program_tensor *actual,
                                            const wafer_hip_program_tensor *expected,
                                            const wafer_hip_comparison_policy *policy, uint32_t *verdict,
                                            wafer_hip_comparison_statistics *out, char *detail,
                                            size_t detail_bytes) {
  WAFER_CHECK_CTX(ctx);
  if (!verdict || !out) return fail(WAFER_HIP_E_INVALID_FIELD, "compare_statistics: null verdict or output");
  WAFER_TRY(check_tensor(actual, "actual"));
  WAFER_TRY(check_tensor(expected, "expected"));
  const wafer_hip_comparison_policy none{};
  const wafer_hip_comparison_policy &p = policy ? *policy : none;
  Verdict v{verdict, detail, detail_bytes};
  memset(out, 0, sizeof *out);
  if (!policy_valid(p)) return v.set(WAFER_CMP_INVALID_TOLERANCE, policy_message(p));
  if (metadata_verdict(actual, expected, v)) return WAFER_HIP_OK;
  const uint32_t d = actual->dtype;
  if (!dtype_tolerant(d))
    return v.set(WAFER_CMP_UNSUPPORTED_STATISTICS_DTYPE,
                 std::string("dtype=") + dtype_name(d) + " has no source/model numeric statistics policy");
  const uint64_t n = actual->bytes / dtype_bytes(d);
  if (n == 0) return v.set(WAFER_CMP_UNSUPPORTED_STATISTICS_DTYPE, "numeric statistics require a non-empty tensor");
  Totals t;
  WAFER_TRY(run_stats(ctx, storage_format(d), actual->data, expected->data, n, p.atol, p.rtol, FULL, t));
  if (t.bad != NONE) return bad_verdict(t, v);
  // ProgramTensorComparison.cpp:481-496
  out->element_count = n;
  out->exact_element_count = t.exact;
  out->exact_fraction = (double)t.exact / (double)n;
  out->mean_absolute_error = (double)(t.abs / (long double)n);
  double q;
  memcpy(&q, &t.q_abs99, 8);
  out->p99_absolute_error = q;
  memcpy(&q, &t.q_abs999, 8);
  out->p999_absolute_error = q;
  out->maximum_absolute_error = t.max_abs;
  out->elementwise_mismatch_count = t.mism;
  out->cosine_similarity = cosine_of(t);
  out->relative_l2_error = rel_l2_of(t);
  out->mean_ulp_distance = (double)((long double)t.ulp_sum / (long double)n);
  out->p99_ulp_distance = t.q_ulp99;
  out->p999_ulp_distance = t.q_ulp999;
  out->maximum_ulp_distance = t.max_ulp;
  return v.set(WAFER_CMP_ACCEPTED, "");
}
