// formal_ops.hip -- the target commands the reference executes only on its
// formal lane: elementwise commands with a broadcast right operand (scalar,
// repeating unit, grouped 64-element blocks), relations (numeric or Bool
// results) and logic operations, and plain pooling.
//
// Semantics (all bit-exact):
//  * elementwise: executeElementwise
//    (lib/Wafer/Simulator/Kernel/TargetModelTensorNumeric.cpp:288-380; rhs
//    expansion :350-369) evaluated by evaluateFormalElementwiseLLVM
//    (lib/Wafer/Simulator/Reference/Formal/FormalNumericElementwise.cpp:23-230):
//    logic ops on Bool (nonzero = true); relations compare exactly, any NaN
//    operand makes Ne true and the others false, a numeric result is 1.0 or
//    0.0 in the input format; Abs / Neg / Max / Min / Relu return the
//    canonical quiet NaN for any NaN operand and otherwise move bits exactly
//    (Max / Min of two zeros: -0 only when both (Max) / either (Min) are -0;
//    otherwise the right operand only when strictly greater (Max) / less
//    (Min); Relu turns a negative nonzero value into +0); Recip, Square, Add,
//    Sub, Mul round once to nearest even in the input format (evaluated in
//    f32, exact for F32 and correctly rounded for F16 / BF16: a single f32
//    operation on F16 / BF16 values then one rounding to the narrow format
//    cannot double-round, 24 >= 2 * 11 + 2), a NaN result is the canonical
//    quiet NaN.  Validation: TargetModelCommandValidation.cpp:160-205 and
//    FormalNumericValidation.cpp:10-69.
//  * pooling: executePool (TargetModelTensorNumeric.cpp:467-586): NHWC
//    windows combined in (kernel row, kernel column) order with the formal
//    Max / Min (the first window element starts the result) or F32 Add from
//    +0.
#include "common.h"

#include <string>

namespace wafer {
namespace {

enum : uint32_t {
  OP_ABS = 0, OP_RECIP = 1, OP_SQUARE = 2, OP_NEG = 5, OP_MAX = 6, OP_MIN = 7, OP_ADD = 8, OP_SUB = 9, OP_MUL = 10,
  OP_EQ = 12, OP_NE = 13, OP_GE = 14, OP_GT = 15, OP_LE = 16, OP_LT = 17,
  OP_NOT = 18, OP_AND = 19, OP_OR = 20, OP_XOR = 21, OP_RELU = 31,
};
__host__ __device__ inline bool is_relation(uint32_t op) { return op >= OP_EQ && op <= OP_LT; }
__host__ __device__ inline bool is_logic(uint32_t op) { return op >= OP_NOT && op <= OP_XOR; }
inline bool in_formal_subset(uint32_t op) {
  switch (op) {
  case OP_ABS: case OP_RECIP: case OP_SQUARE: case OP_NEG: case OP_MAX: case OP_MIN: case OP_ADD: case OP_SUB:
  case OP_MUL: case OP_RELU: return true;
  default: return is_relation(op) || is_logic(op);
  }
}
inline bool registered(uint32_t op) { return op <= 10 || (op >= 12 && op <= 34); }
__host__ __device__ inline bool binary(uint32_t op) {
  return op == OP_MAX || op == OP_MIN || op == OP_ADD || op == OP_SUB || op == OP_MUL || is_relation(op) ||
         op == OP_AND || op == OP_OR || op == OP_XOR;
}

template <uint32_t F> __device__ inline uint32_t load_bits(const void *p, uint64_t i) {
  if constexpr (F == WAFER_FMT_F32) return ((const uint32_t *)p)[i];
  else if constexpr (F == WAFER_FMT_BOOL) return ((const uint8_t *)p)[i];
  else return ((const uint16_t *)p)[i];
}
template <uint32_t F> __device__ inline float widen(uint32_t b) {
  if constexpr (F == WAFER_FMT_F32) return u2f(b);
  else if constexpr (F == WAFER_FMT_BF16) return bf16_to_f32((uint16_t)b);
  else return f16_to_f32((uint16_t)b);
}
template <uint32_t F> __device__ inline uint32_t narrow(float v) {
  if constexpr (F == WAFER_FMT_F32) return v != v ? 0x7fc00000u : f2u(v);
  else if constexpr (F == WAFER_FMT_BF16) return f32_to_bf16(v);  // NaN -> 0x7fc0
  else return f32_to_f16(v);                                       // NaN -> 0x7e00
}
template <uint32_t F> constexpr uint32_t sign_bit() { return F == WAFER_FMT_F32 ? 0x80000000u : 0x8000u; }
template <uint32_t F> constexpr uint32_t qnan() {
  return F == WAFER_FMT_F32 ? 0x7fc00000u : (F == WAFER_FMT_BF16 ? 0x7fc0u : 0x7e00u);
}
template <uint32_t F> constexpr uint32_t one_bits() {
  return F == WAFER_FMT_F32 ? 0x3f800000u : (F == WAFER_FMT_BF16 ? 0x3f80u : 0x3c00u);
}

// the formal Max / Min on raw bits (no NaN operand)
template <uint32_t F> __device__ inline uint32_t formal_maxmin(bool is_max, uint32_t ab, uint32_t bb) {
  const float a = widen<F>(ab), b = widen<F>(bb);
  if (a == 0.0f && b == 0.0f) {
    const bool na = ab & sign_bit<F>(), nb = bb & sign_bit<F>();
    const bool neg = is_max ? (na && nb) : (na || nb);
    return neg ? sign_bit<F>() : 0u;
  }
  const bool take_b = is_max ? a < b : a > b;
  return take_b ? bb : ab;
}

// one float-format element; returns the result bits in the result format
// (F, or Bool 0 / 1 for a relation with a Bool result)
template <uint32_t F> __device__ inline uint32_t formal_eval(uint32_t op, uint32_t ab, uint32_t bb, bool numeric) {
  const float a = widen<F>(ab), b = widen<F>(bb);
  const bool nan_a = a != a, nan_b = binary(op) && b != b;
  if (is_relation(op)) {
    bool r;
    if (nan_a || nan_b) {
      r = op == OP_NE;
    } else {
      switch (op) {
      case OP_EQ: r = a == b; break;
      case OP_NE: r = a != b; break;
      case OP_GE: r = a >= b; break;
      case OP_GT: r = a > b; break;
      case OP_LE: r = a <= b; break;
      default: r = a < b; break;
      }
    }
    return numeric ? (r ? one_bits<F>() : 0u) : (r ? 1u : 0u);
  }
  if ((op == OP_ABS || op == OP_NEG || op == OP_MAX || op == OP_MIN || op == OP_RELU) && (nan_a || nan_b))
    return qnan<F>();
  switch (op) {
  case OP_ABS: return ab & ~sign_bit<F>();
  case OP_NEG: return ab ^ sign_bit<F>();
  case OP_MAX: return formal_maxmin<F>(true, ab, bb);
  case OP_MIN: return formal_maxmin<F>(false, ab, bb);
  case OP_RELU: return ((ab & sign_bit<F>()) && a != 0.0f) ? 0u : ab;
  case OP_RECIP: return narrow<F>(1.0f / a);
  case OP_SQUARE: return narrow<F>(a * a);
  case OP_ADD: return narrow<F>(a + b);
  case OP_SUB: return narrow<F>(a - b);
  default: return narrow<F>(a * b);  // OP_MUL
  }
}

struct EwArgs {
  const void *lhs, *rhs;
  void *dst;
  uint64_t count;
  uint32_t op, mode, param, scalar;  // mode 0 full, 1 scalar, 2 unit (param), 3 group (param)
  bool numeric;                      // relation result in the input format
  int *status;                       // logic ops: set to 1 on a non-canonical Bool operand
};

template <uint32_t F>
__global__ __launch_bounds__(256) void formal_ew_kernel(const EwArgs a) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.count; i += stride) {
    const uint32_t lb = load_bits<F>(a.lhs, i);
    uint32_t rb = 0;
    if (binary(a.op)) {
      switch (a.mode) {
      case 1: rb = a.scalar; break;
      case 2: rb = load_bits<F>(a.rhs, i % a.param); break;
      case 3: rb = load_bits<F>(a.rhs, i / a.param * 64 + i % 64); break;
      default: rb = load_bits<F>(a.rhs, i); break;
      }
    }
    if constexpr (F == WAFER_FMT_BOOL) {
      if (lb > 1u || rb > 1u) *a.status = 1;  // (racing writes of the same value)
      const bool l = lb != 0, r = rb != 0;
      bool v;
      switch (a.op) {
      case OP_NOT: v = !l; break;
      case OP_AND: v = l && r; break;
      case OP_OR: v = l || r; break;
      default: v = l != r; break;
      }
      ((uint8_t *)a.dst)[i] = v ? 1 : 0;
    } else {
      const uint32_t r = formal_eval<F>(a.op, lb, rb, a.numeric);
      if (is_relation(a.op) && !a.numeric) ((uint8_t *)a.dst)[i] = (uint8_t)r;
      else if constexpr (F == WAFER_FMT_F32) ((uint32_t *)a.dst)[i] = r;
      else ((uint16_t *)a.dst)[i] = (uint16_t)r;
    }
  }
}

struct PoolArgs {
  const void *src;
  void *dst;
  uint32_t n, ih, iw, c, oh, ow, kw, kh, sw, sh;
  uint32_t op;  // 117 Maximum, 119 Minimum, 116 Sum (F32)
};

template <uint32_t F>
__global__ __launch_bounds__(256) void pool_kernel(const PoolArgs a) {
  const uint64_t count = (uint64_t)a.n * a.oh * a.ow * a.c;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < count; e += stride) {
    const uint64_t c = e % a.c, w = (e / a.c) % a.ow, h = (e / ((uint64_t)a.c * a.ow)) % a.oh,
                   n = e / ((uint64_t)a.c * a.ow * a.oh);
    uint32_t r = 0;  // Sum starts from +0
    bool nan = false;
    for (uint32_t ky = 0; ky < a.kh; ++ky)
      for (uint32_t kx = 0; kx < a.kw; ++kx) {
        const uint64_t sy = h * a.sh + ky, sx = w * a.sw + kx;
        const uint32_t v = load_bits<F>(a.src, ((n * a.ih + sy) * a.iw + sx) * a.c + c);
        if (a.op == 116) {
          if constexpr (F == WAFER_FMT_F32) r = narrow<F>(u2f(r) + u2f(v));
        } else if (ky == 0 && kx == 0) {
          r = v;
          nan = widen<F>(v) != widen<F>(v);
        } else {
          nan = nan || widen<F>(v) != widen<F>(v);
          if (!nan) r = formal_maxmin<F>(a.op == 117, r, v);
        }
      }
    if (a.op != 116 && nan && a.kh * a.kw > 1) r = qnan<F>();  // a lone element is copied as is
    if constexpr (F == WAFER_FMT_F32) ((uint32_t *)a.dst)[e] = r;
    else ((uint16_t *)a.dst)[e] = (uint16_t)r;
  }
}

// 1x1 Max / Min windows of an integer or Bool format: the element itself
template <typename T>
__global__ __launch_bounds__(256) void pool_pick(const PoolArgs a) {
  const uint64_t count = (uint64_t)a.n * a.oh * a.ow * a.c;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < count; e += stride) {
    const uint64_t c = e % a.c, w = (e / a.c) % a.ow, h = (e / ((uint64_t)a.c * a.ow)) % a.oh,
                   n = e / ((uint64_t)a.c * a.ow * a.oh);
    ((T *)a.dst)[e] = ((const T *)a.src)[((n * a.ih + h * a.sh) * a.iw + w * a.sw) * a.c + c];
  }
}

unsigned blocks_for(uint64_t n) { return (unsigned)std::min<uint64_t>((n + 255) / 256, 65536); }

}  // namespace
}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_elementwise_formal(wafer_hip_context *ctx, const wafer_hip_elementwise_command *cmd,
                                            const void *lhs, const void *rhs, void *dst) {
  WAFER_CHECK_CTX(ctx);
  if (!cmd) return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise: null command");
  const wafer_hip_elementwise_command &v = *cmd;
  if (v.element_count == 0) return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise element_count must be positive");
  if (!registered(v.operation)) return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise operation is not registered");
  const uint32_t f = v.format;
  if (f > WAFER_FMT_U64) return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise format is unsupported by its target engine");
  const bool bin = binary(v.operation), logic = is_logic(v.operation), rel = is_relation(v.operation);
  const bool floating = f == WAFER_FMT_F16 || f == WAFER_FMT_BF16 || f == WAFER_FMT_F32;
  // validateElementwise (TargetModelCommandValidation.cpp:153-199)
  if ((rhs != nullptr) + (v.has_rhs_scalar != 0) != (bin ? 1 : 0))
    return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise rhs presence differs from operation arity");
  if (v.relation_numeric > 1 || (v.relation_numeric && !rel))
    return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise relation output kind is invalid");
  if (v.has_rhs_scalar &&
      (logic || v.rhs_unit_elements || !floating || (f != WAFER_FMT_F32 && v.rhs_scalar > 0xffffu)))
    return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise VS requires matching floating scalar bits");
  if (v.rhs_unit_elements && (!bin || logic || v.rhs_unit_elements > 64 || !floating))
    return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise RHS unit requires 1..64 floating elements");
  if (v.rhs_group_elements && (rel || v.rhs_unit_elements != 64 || v.rhs_group_elements % 64 ||
                               v.element_count % v.rhs_group_elements))
    return fail(WAFER_HIP_E_INVALID_FIELD, "grouped RHS requires arithmetic, unit 64 and complete groups");
  if (logic != (f == WAFER_FMT_BOOL) || (rel && f == WAFER_FMT_BOOL))
    return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise format differs from logic/relation operation class");
  if (v.element_count > 0xffffffffull)
    return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise element_count must fit uint32_t");
  // validateFormalElementwiseOperation (FormalNumericValidation.cpp:45-68); its failures surface as
  // FormalNumericFailure (TargetModelTensorNumeric.cpp:376-380)
  if (!in_formal_subset(v.operation))
    return fail(WAFER_HIP_E_NUMERIC, "elementwise operation is outside the formal subset");
  if (!logic && !floating) return fail(WAFER_HIP_E_NUMERIC, "elementwise formats are outside the formal subset");
  if (!lhs || !dst) return fail(WAFER_HIP_E_INVALID_FIELD, "elementwise: null tensor");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  EwArgs a{};
  a.lhs = lhs;
  a.rhs = rhs;
  a.dst = dst;
  a.count = v.element_count;
  a.op = v.operation;
  a.mode = v.has_rhs_scalar ? 1u : (v.rhs_group_elements ? 3u : (v.rhs_unit_elements ? 2u : 0u));
  a.param = v.rhs_group_elements ? v.rhs_group_elements : v.rhs_unit_elements;
  a.scalar = v.rhs_scalar;
  a.numeric = v.relation_numeric != 0;
  const dim3 grid(blocks_for(v.element_count));
  if (logic) {  // Bool operands must be canonical 0 / 1 (validateOperand): a status word reports others
    uint8_t *words = nullptr;
    WAFER_TRY(status_words(ctx, "a logic elementwise command", &words));
    a.status = (int *)words;
    WAFER_TRY(fill_words(ctx, a.status, 1, 0));
    hipLaunchKernelGGL(formal_ew_kernel<WAFER_FMT_BOOL>, grid, dim3(256), 0, ctx->stream, a);
    WAFER_TRY(launch_status("formal_ew_kernel"));
    int host = 0;
    WAFER_TRY(check_hip(hipMemcpyAsync(&host, a.status, sizeof(int), hipMemcpyDeviceToHost, ctx->stream),
                        "hipMemcpyAsync"));
    WAFER_TRY(check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize"));
    if (host) return fail(WAFER_HIP_E_NUMERIC, "elementwise Bool operand is not a canonical 0 / 1 value");
    return WAFER_HIP_OK;
  }
  if (f == WAFER_FMT_F32)
    hipLaunchKernelGGL(formal_ew_kernel<WAFER_FMT_F32>, grid, dim3(256), 0, ctx->stream, a);
  else if (f == WAFER_FMT_BF16)
    hipLaunchKernelGGL(formal_ew_kernel<WAFER_FMT_BF16>, grid, dim3(256), 0, ctx->stream, a);
  else
    hipLaunchKernelGGL(formal_ew_kernel<WAFER_FMT_F16>, grid, dim3(256), 0, ctx->stream, a);
  return launch_status("formal_ew_kernel");
}

extern "C" int wafer_hip_pool(wafer_hip_context *ctx, const wafer_hip_pool_command *cmd, const void *src,
                              void *dst) {
  WAFER_CHECK_CTX(ctx);
  if (!cmd) return fail(WAFER_HIP_E_INVALID_FIELD, "pool: null command");
  const wafer_hip_pool_command &p = *cmd;
  // command validation (TargetModelCommandValidation.cpp:423-447, limits Tx81InstructionLimits.h:12-16)
  if (p.operation < 115 || p.operation > 120) return fail(WAFER_HIP_E_INVALID_FIELD, "pool operation is not registered");
  const bool indexed = p.operation == 118 || p.operation == 120;
  if ((p.has_index_destination != 0) != indexed)
    return fail(WAFER_HIP_E_INVALID_FIELD, "pool index destination presence differs from pool kind");
  for (int i = 0; i < 4; ++i) {
    const uint32_t limit = i == 3 ? 16384u : 4096u;
    if (p.source_shape[i] < 1 || p.source_shape[i] > limit || p.destination_shape[i] < 1 ||
        p.destination_shape[i] > limit)
      return fail(WAFER_HIP_E_INVALID_FIELD, "pool shape dimension is outside its instruction range");
    if (p.pads[i] > 1023) return fail(WAFER_HIP_E_INVALID_FIELD, "pool pads must be in [0, 1023]");
    if (p.kernel_strides[i] < 1 || p.kernel_strides[i] > (i < 2 ? 255u : 1023u))
      return fail(WAFER_HIP_E_INVALID_FIELD, "pool kernel_strides are outside their instruction range");
  }
  if (p.format > WAFER_FMT_U64) return fail(WAFER_HIP_E_INVALID_FIELD, "pool format is unsupported by its target engine");
  // executePool (TargetModelTensorNumeric.cpp:467-507)
  if (p.has_index_destination || p.pads[0] || p.pads[1] || p.pads[2] || p.pads[3])
    return fail(WAFER_HIP_E_UNSUPPORTED, "plain pooling requires explicit input padding and no index output");
  if (p.source_shape[0] != p.destination_shape[0] || p.source_shape[3] != p.destination_shape[3])
    return fail(WAFER_HIP_E_INVALID_FIELD, "pooling must preserve batch and channel extents");
  for (int axis = 0; axis < 2; ++axis) {
    const uint64_t source = p.source_shape[axis + 1], kernel = p.kernel_strides[1 - axis],
                   stride = p.kernel_strides[3 - axis];
    if (source < kernel || (source - kernel) / stride + 1 != p.destination_shape[axis + 1])
      return fail(WAFER_HIP_E_INVALID_FIELD, "pooling result disagrees with its window geometry");
  }
  if (p.operation == 116 && p.format != WAFER_FMT_F32)
    return fail(WAFER_HIP_E_UNSUPPORTED, "plain sum pooling currently qualifies F32 accumulation only");
  if (p.operation != 116 && p.operation != 117 && p.operation != 119)
    return fail(WAFER_HIP_E_UNSUPPORTED, "pooling kind has no qualified plain numeric implementation");
  const bool single = p.kernel_strides[0] == 1 && p.kernel_strides[1] == 1;
  const bool floating = p.format == WAFER_FMT_F16 || p.format == WAFER_FMT_BF16 || p.format == WAFER_FMT_F32;
  // a 1x1 Max / Min window copies its element without a formal combine; any combine of a
  // non-float format fails in the formal evaluator
  if (!floating && !single) return fail(WAFER_HIP_E_NUMERIC, "elementwise formats are outside the formal subset");
  if (!src || !dst) return fail(WAFER_HIP_E_INVALID_FIELD, "pool: null tensor");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  PoolArgs a{src, dst, p.source_shape[0], p.source_shape[1], p.source_shape[2], p.source_shape[3],
             p.destination_shape[1], p.destination_shape[2], p.kernel_strides[0], p.kernel_strides[1],
             p.kernel_strides[2], p.kernel_strides[3], p.operation};
  const uint64_t count = (uint64_t)a.n * a.oh * a.ow * a.c;
  const dim3 grid(blocks_for(count));
  if (!floating) {
    switch (format_bytes(p.format)) {
    case 1: hipLaunchKernelGGL(pool_pick<uint8_t>, grid, dim3(256), 0, ctx->stream, a); break;
    case 2: hipLaunchKernelGGL(pool_pick<uint16_t>, grid, dim3(256), 0, ctx->stream, a); break;
    case 4: hipLaunchKernelGGL(pool_pick<uint32_t>, grid, dim3(256), 0, ctx->stream, a); break;
    default: hipLaunchKernelGGL(pool_pick<uint64_t>, grid, dim3(256), 0, ctx->stream, a); break;
    }
    return launch_status("pool_pick");
  }
  if (p.format == WAFER_FMT_F32)
    hipLaunchKernelGGL(pool_kernel<WAFER_FMT_F32>, grid, dim3(256), 0, ctx->stream, a);
  else if (p.format == WAFER_FMT_BF16)
    hipLaunchKernelGGL(pool_kernel<WAFER_FMT_BF16>, grid, dim3(256), 0, ctx->stream, a);
  else
    hipLaunchKernelGGL(pool_kernel<WAFER_FMT_F16>, grid, dim3(256), 0, ctx->stream, a);
  return launch_status("pool_kernel");
}
