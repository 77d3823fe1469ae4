/*
 * wafer_hip.h -- C ABI of the MI355X (gfx950) numeric execution backend for
 * the kernels the Wafer compiler emits.
 *
 * The backend sits beside the reference's Reference (formal / managed) and
 * oneDNN CPU lanes.  Every entry point is `extern "C"`, takes plain device
 * pointers and sizes, and returns an int status (WAFER_HIP_OK == 0, negative
 * on failure; wafer_hip_last_error() then holds a message for the calling
 * thread).  No entry point falls back to a CPU path: a request the HIP
 * kernels cannot serve fails with WAFER_HIP_E_UNSUPPORTED.
 *
 * Memory: all tensor pointers are device pointers owned by the caller.  Work
 * is enqueued on the context's stream (wafer_hip_set_stream) and is
 * stream-ordered; wafer_hip_synchronize() waits for it.  Logical tensors are
 * dense row-major; raw 16-bit floats are passed as their storage bits.
 *
 * Format codes are the reference's Data_Format table
 * (lib/Wafer/Target/TargetFormat.cpp:62-63): I8=0 I16=1 F16=2 BF16=3 I32=4
 * F32=5 TF32=6 Bool=7 U8=8 U16=9 U32=10 I64=11 U64=12.
 */
#ifndef WAFER_HIP_H
#define WAFER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------
 * Negative images of TargetModelKernelErrorCode
 * (include/Wafer/Simulator/Kernel/TargetModelKernel.h:21-32) plus the HIP
 * runtime failure this backend adds. */
enum {
  WAFER_HIP_OK = 0,
  WAFER_HIP_E_INVALID_FIELD = -1,     /* InvalidCommandField */
  WAFER_HIP_E_BUDGET = -2,            /* WorkBudgetExceeded */
  WAFER_HIP_E_UNSUPPORTED = -3,       /* UnsupportedCommand */
  WAFER_HIP_E_MEMORY = -4,            /* MemoryReadFailure */
  WAFER_HIP_E_NUMERIC = -5,           /* FormalNumericFailure */
  WAFER_HIP_E_CODEC = -6,             /* PhysicalCodecFailure */
  WAFER_HIP_E_UNAVAILABLE = -7,       /* ...BackendUnavailable */
  WAFER_HIP_E_RUNTIME = -8            /* a HIP runtime call failed */
};

/* Format codes (TargetFormat.cpp:62-63). */
enum {
  WAFER_FMT_I8 = 0, WAFER_FMT_I16 = 1, WAFER_FMT_F16 = 2, WAFER_FMT_BF16 = 3,
  WAFER_FMT_I32 = 4, WAFER_FMT_F32 = 5, WAFER_FMT_TF32 = 6, WAFER_FMT_BOOL = 7,
  WAFER_FMT_U8 = 8, WAFER_FMT_U16 = 9, WAFER_FMT_U32 = 10, WAFER_FMT_I64 = 11,
  WAFER_FMT_U64 = 12
};

/* Physical layouts (PhysicalTensorDescriptor layout kinds,
 * lib/Wafer/Target/PhysicalTensor/PhysicalLayout.cpp:111-200). */
enum { WAFER_LAYOUT_TENSOR = 0, WAFER_LAYOUT_NTENSOR = 1, WAFER_LAYOUT_CX = 2,
       WAFER_LAYOUT_NCX = 3 };

/* TargetGemmOrientation (include/Wafer/Target/TargetFormat.h:92). */
enum { WAFER_GEMM_NORMAL = 0, WAFER_GEMM_TRANSPOSE = 1 };

/* kDisabledGemmPartialFormat (include/Wafer/Target/TargetCall.h:72). */
#define WAFER_GEMM_PSUM_DISABLED 13u

typedef struct wafer_hip_context wafer_hip_context;

/* ---- context ------------------------------------------------------------
 * Replaces the construction of a numeric backend object once per run
 * (tools/wafer-compile/wafer-compile.cpp:477-506).  A context binds one HIP
 * device and one stream (the null stream until set).  Calls on one context
 * are serialised by the caller, as SystemCTargetModel::issue serialises
 * backend calls (lib/Wafer/Simulator/SystemC/SystemCTargetModel.cpp:156-185).
 * Workspace: the context owns three device areas, each grown on first need
 * and never shrunk -- the split-K partial tiles of the MFMA GEMMs (up to
 * 4 * m * n * 4 bytes for the 16-bit GEMMs, 64 MiB at the decoder layer's
 * down projection), the re-laid-out [n,k] rhs of a Normal-orientation GEMM
 * (k * n * element bytes) and FD's chunk states for small batches.  Growing
 * is refused on a capturing stream, so a caller that captures runs each
 * shape once eagerly first.  A grown area's old buffer is kept until
 * wafer_hip_context_destroy, so graphs captured before a later, larger eager
 * call still replay on valid memory (the area at least doubles per growth,
 * bounding the retired buffers by its current size). */
int wafer_hip_context_create(int device, wafer_hip_context **out);
int wafer_hip_context_destroy(wafer_hip_context *ctx);
int wafer_hip_set_stream(wafer_hip_context *ctx, void *hip_stream);
int wafer_hip_synchronize(wafer_hip_context *ctx);
const char *wafer_hip_last_error(void);
/* Device buffers and synchronous copies for host-side callers that hold
 * tensors in host memory (the seam's TargetModelNumericTensor storage);
 * copies are ordered on the context's stream and complete on return. */
int wafer_hip_buffer_alloc(wafer_hip_context *ctx, uint64_t bytes, void **out);
int wafer_hip_buffer_free(wafer_hip_context *ctx, void *buffer);
int wafer_hip_copy_to_device(wafer_hip_context *ctx, void *dst, const void *src,
                             uint64_t bytes);
int wafer_hip_copy_to_host(wafer_hip_context *ctx, void *dst, const void *src,
                           uint64_t bytes);
/* Implementation string, the analogue of the evidence `implementation`
 * field (include/Wafer/Simulator/Kernel/TargetModelKernel.h:144-182). */
const char *wafer_hip_implementation(void);

/* The execution environment a qualification record binds: the analogue of
 * OneDNNExecutionEnvironment's identity fields
 * (include/Wafer/Simulator/OneDNN/OneDNNQualification.h:132-229 records its
 * digest).  Strings are NUL-terminated. */
typedef struct wafer_hip_environment_info {
  char gcn_arch_name[64];   /* e.g. "gfx950:sramecc+:xnack-" */
  char device_name[128];
  int32_t compute_units;
  int32_t hip_runtime_version;
  int32_t driver_version;
  int32_t warp_size;
  uint64_t global_memory_bytes;
  uint64_t lds_bytes_per_block;
} wafer_hip_environment_info;
int wafer_hip_environment(wafer_hip_context *ctx, wafer_hip_environment_info *out);

/* ---- per-command GEMM (formal semantics, bit-exact) ----------------------
 * Replaces wafer_tx81_gemm_oriented (runtime/crt/include/wafer_tx81_crt.h:44-49)
 * as executed by the formal lane, executeGemm
 * (lib/Wafer/Simulator/Reference/Numeric/FormalTensorNumeric.cpp:272-361):
 * for each output, acc = +0; for k in order acc = fma(widen(lhs), widen(rhs),
 * acc) with one RNE rounding; acc += psum (F32 add) when psum_format != 13;
 * dst = RNE(acc -> out_format).  lhs is [batch, m, k] (Transpose: [batch, k, m]),
 * rhs is [batch, k, n] (Transpose: [batch, n, k]), dst/psum [batch, m, n].
 * in_format/out_format in {F16, BF16, F32}; psum_format F32 or 13. */
int wafer_hip_gemm(wafer_hip_context *ctx, const void *lhs, const void *rhs,
                   void *dst, const void *psum, uint32_t m, uint32_t k,
                   uint32_t n, uint32_t batch, uint32_t in_format,
                   uint32_t out_format, uint32_t psum_format,
                   uint32_t lhs_orientation, uint32_t rhs_orientation);

/* ---- MFMA GEMM (bf16/f16 in, f32 accumulate; tolerance parity) ------------
 * The throughput path for large region-level GEMMs.  Same operand meaning as
 * wafer_hip_gemm with lhs Normal; the MFMA accumulation order differs from
 * the formal k-order, so results match the formal lane within tolerance.
 * out_format F32 or the input format.  Any m, n; k a multiple of 32 (64-byte
 * K stages); other k return WAFER_HIP_E_UNSUPPORTED.  Long-K shapes whose
 * 128x128 grid is at most one round of workgroups (k * 2 >= 16384 bytes, m
 * and n multiples of 256) split K over 4 workgroups with f32 partials in a
 * context-owned area (4 * m * n * 4 bytes, grown on first use; growing is
 * refused on a capturing stream, so a caller that captures runs the shape
 * once eagerly first).  Results repeat bit for bit for a given shape. */
int wafer_hip_gemm_mfma(wafer_hip_context *ctx, const void *lhs,
                        const void *rhs, void *dst, uint32_t m, uint32_t k,
                        uint32_t n, uint32_t in_format, uint32_t out_format,
                        uint32_t rhs_orientation);

/* MFMA GEMM with a residual add fused into the epilogue: dst = Add(narrow(lhs .
 * rhs), residual), the narrowed product of wafer_hip_gemm_mfma followed by the
 * CT Add command (ManagedReferenceTargetModel.cpp:230-299), same bits.
 * residual and dst [m, n] in the input format (BF16 or F16); dst may be the
 * residual buffer itself.  A decoder block's x + proj(a) after the down (or
 * O) projection. */
int wafer_hip_gemm_mfma_residual(wafer_hip_context *ctx, const void *lhs,
                                 const void *rhs, const void *residual,
                                 void *dst, uint32_t m, uint32_t k, uint32_t n,
                                 uint32_t in_format, uint32_t rhs_orientation);

/* MFMA GEMM with SwiGLU fused into the epilogue: rhs_gu is [2*features, k]
 * (Transposed orientation) with rows in 32-row groups, rows 32j + [0,16) the
 * gate rows 16j + [0,16) and rows 32j + 16 + [0,16) the up rows of the same
 * features; dst [m, features] = T(silu_mul(T(gate), T(up))), T = in_format
 * (BF16 or F16) -- the two narrowed products followed by the silu_mul region
 * (same bits); features a multiple of 16.  The region is the SwiGLU composition of
 * lib/Wafer/Conversion/TileToInstr/ComputeLowering.cpp:2555-2606 after two GEMMs. */
int wafer_hip_gemm_mfma_swiglu(wafer_hip_context *ctx, const void *lhs,
                               const void *rhs_gu, void *dst, uint32_t m,
                               uint32_t k, uint32_t features,
                               uint32_t in_format);

/* ---- f32 MFMA GEMM (tolerance parity) with a fused bias / GELU epilogue ----
 * Replaces the oneDNN lane's f32 matmul for F32 operands, executeOneDNN
 * (lib/Wafer/Simulator/OneDNN/OneDNNGemmAdapter.cpp:278-420: deterministic,
 * strict f32 math, an accumulation order of its own), with the bias_add and
 * gelu_tanh regions of an MLP block optionally fused after it.  dst [m,n] =
 * epilogue(lhs [m,k] . rhs), rhs [k,n] Normal or [n,k] Transpose, on
 * v_mfma_f32_32x32x2_f32 (f32 products, f32 accumulation in a fixed order:
 * results repeat bit for bit and match the formal lane within tolerance).
 * epilogue: NONE; BIAS (dst = acc + bias[n], the bias_add region's F32 add);
 * BIAS_GELU_TANH (gelu_tanh of that sum, the gelu_tanh region's formula).
 * Any m, n; k a multiple of 8; lhs, dst and a Transposed rhs 16-byte aligned.
 * Small grids split k over workgroups through a context-owned partial-tile
 * area (grown on first use; growing is refused on a capturing stream). */
enum {
  WAFER_HIP_EPILOGUE_NONE = 0,
  WAFER_HIP_EPILOGUE_BIAS = 1,
  WAFER_HIP_EPILOGUE_BIAS_GELU_TANH = 2
};
int wafer_hip_gemm_f32_mfma(wafer_hip_context *ctx, const float *lhs,
                            const float *rhs, const float *bias, float *dst,
                            uint32_t m, uint32_t k, uint32_t n,
                            uint32_t rhs_orientation, uint32_t epilogue);

/* ---- int8 GEMM -------------------------------------------------------------
 * No reference implementation exists (the formal and oneDNN lanes reject I8:
 * lib/Wafer/Simulator/Reference/Formal/FormalNumericValidation.cpp:78-83,
 * lib/Wafer/Simulator/OneDNN/OneDNNGemmAdapter.cpp:42-52); this follows the
 * closed form on the reference's routes: acc = sum_k int32(a)*int32(b) exactly,
 * y = bf16_RNE(f32_RNE(f32_RNE(acc) * scale[n])) (int32_fp32 route, CT Mul,
 * fp32_bf16 route; lib/Wafer/Target/TargetFormat.cpp:174,192).
 * a [m,k] i8, b [k,n] i8 (Transpose: [n,k]), scale [n] f32, y [m,n] bf16;
 * acc_out [m,n] i32 may be NULL.  Any m, n; k a multiple of 64 and at most
 * 131071 (|acc| <= k*128*128 < 2^31); other k are rejected.  A [k,n] b with
 * m and n multiples of 256, k of 128, at least 192 tiles of 256x256 and
 * k*n below 2^31 is read in place (no workspace, so such calls may be
 * captured); other [k,n] shapes are re-laid out to [n,k] in the context's
 * workspace first. */
int wafer_hip_gemm_i8(wafer_hip_context *ctx, const int8_t *a, const int8_t *b,
                      const float *scale, int32_t *acc_out, uint16_t *y,
                      uint32_t m, uint32_t k, uint32_t n,
                      uint32_t rhs_orientation);

/* ---- managed-reference elementwise / convert / reduce ---------------------
 * Replace TargetModelManagedReferenceBackend::execute
 * (include/Wafer/Simulator/Kernel/TargetModelKernel.h:187-200) on logical
 * (unpacked) tensors.  op is TargetElementwiseOperation
 * (include/Wafer/Target/TargetOperation.h:58-93); the float expressions follow
 * evaluateElementwise (lib/Wafer/Simulator/Reference/ManagedReferenceTargetModel.cpp:230-299).
 * in1 is ignored for unary ops. */
int wafer_hip_elementwise(wafer_hip_context *ctx, uint32_t op, uint32_t format,
                          const void *in0, const void *in1, void *dst,
                          uint64_t count);
/* opcode is a convert route of the Data_Format route table
 * (lib/Wafer/Target/TargetFormat.cpp:164-196), rounding TargetRoundingMode
 * (include/Wafer/Target/TargetOperation.h:175-181); NearestEven only. */
int wafer_hip_convert(wafer_hip_context *ctx, uint32_t opcode,
                      uint32_t rounding, const void *src, void *dst,
                      uint64_t count);
/* The (source, destination) formats of a served convert route, for callers
 * validating a FormalConvertOperation's descriptors (host only). */
int wafer_hip_convert_route(uint32_t opcode, uint32_t *source_format,
                            uint32_t *destination_format);
/* The managed lane works in the non-NaN domain: it refuses a NaN input
 * value and a NaN result (decodeNonNaN / encodeNonNaN,
 * lib/Wafer/Simulator/Reference/ManagedReferenceTargetModel.cpp:137-185).
 * wafer_hip_elementwise / _convert / _reduce compute IEEE results (a NaN
 * propagates); a caller that needs the managed lane's refusal checks the
 * logical inputs and the result with this entry, as the C++ seam does.
 * *first = the index of the first NaN among `count` F16/BF16/F32 values, or
 * `count` when there is none.  Synchronous (reads the index back); refused on
 * a capturing stream. */
int wafer_hip_first_nan(wafer_hip_context *ctx, uint32_t format,
                        const void *values, uint64_t count, uint64_t *first);
/* op TargetReduceOperation {Sum, Max, Min} and dim TargetReduceDimension
 * (TargetOperation.h:102-113); shape is the logical shape (rank <= 8) and dst
 * holds the shape with reduced dimensions set to 1. */
int wafer_hip_reduce(wafer_hip_context *ctx, uint32_t op, uint32_t dim,
                     uint32_t format, const int64_t *shape, uint32_t rank,
                     const void *src, void *dst);

/* ---- formal-lane commands (bit-exact) ---------------------------------------
 * Target commands that the reference executes on its formal lane only.
 * Tensors are logical: F16 / BF16 as 16-bit words, F32 as 32-bit words,
 * Bool as one byte per element holding 0 or 1 (the physical codec's bit
 * packing stays with the caller).
 *
 * An elementwise command (TargetElementwiseCommand,
 * include/Wafer/Target/TargetCommand.h) replaces executeElementwise
 * (lib/Wafer/Simulator/Kernel/TargetModelTensorNumeric.cpp:288-392), validated
 * as validateElementwise (TargetModelCommandValidation.cpp:153-199) and
 * evaluated as evaluateFormalElementwiseLLVM
 * (lib/Wafer/Simulator/Reference/Formal/FormalNumericElementwise.cpp:23-247):
 * operation is TargetElementwiseOperation (Abs, Recip, Square, Neg, Max, Min,
 * Add, Sub, Mul, the relations Eq..Lt, LogicNot..LogicXor, Relu; the other
 * registered operations fail with WAFER_HIP_E_NUMERIC, as the formal lane's
 * refusal surfaces there).  The right operand is a full tensor (rhs != NULL,
 * no unit / group), a scalar's bits (has_rhs_scalar, rhs NULL), a repeating
 * unit of rhs_unit_elements (1..64) values, or grouped 64-value blocks
 * (rhs_unit_elements 64, element i reads rhs[i / rhs_group_elements * 64 +
 * i % 64]).  relation_numeric 0 gives a Bool result, 1 the bits of 1.0 / +0
 * in the input format (TargetRelationOutput Numeric).  A logic command whose
 * Bool operand byte is neither 0 nor 1 fails with WAFER_HIP_E_NUMERIC after
 * the launch (it reads a status word back: synchronous, refused on a
 * capturing stream); the other commands are asynchronous. */
typedef struct wafer_hip_elementwise_command {
  uint32_t operation;          /* TargetElementwiseOperation */
  uint32_t format;             /* WAFER_FMT_F16 / BF16 / F32, or BOOL for logic */
  uint32_t relation_numeric;   /* 0 PackedBool, 1 Numeric (relations only) */
  uint32_t rhs_unit_elements;  /* 0 or 1..64 */
  uint32_t rhs_group_elements; /* 0 or a multiple of 64 dividing element_count */
  uint32_t has_rhs_scalar;
  uint32_t rhs_scalar;         /* raw bits in `format` */
  uint32_t reserved;
  uint64_t element_count;      /* 1 .. 2^32 - 1 */
} wafer_hip_elementwise_command;
int wafer_hip_elementwise_formal(wafer_hip_context *ctx,
                                 const wafer_hip_elementwise_command *cmd,
                                 const void *lhs, const void *rhs, void *dst);

/* Plain pooling (TargetPoolCommand) replacing executePool
 * (TargetModelTensorNumeric.cpp:467-586) after the command validation of
 * TargetModelCommandValidation.cpp:423-447.  NHWC logical tensors; operation
 * is TargetPoolingOperation (TargetOperation.h:149-156): Maximum / Minimum
 * combine each window in (kernel row, kernel column) order with the formal
 * Max / Min, Sum adds F32 values to +0 in the same order; Average, the
 * indexed kinds, nonzero pads and non-F32 Sum fail with
 * WAFER_HIP_E_UNSUPPORTED as in the reference.  kernel_strides =
 * {kernel W, kernel H, stride W, stride H}.  Asynchronous. */
typedef struct wafer_hip_pool_command {
  uint32_t operation;
  uint32_t format;
  uint32_t source_shape[4];      /* N, H, W, C */
  uint32_t destination_shape[4]; /* N, H, W, C */
  uint32_t pads[4];
  uint32_t kernel_strides[4];
  uint32_t has_index_destination;
} wafer_hip_pool_command;
int wafer_hip_pool(wafer_hip_context *ctx, const wafer_hip_pool_command *cmd,
                   const void *src, void *dst);

/* ---- physical codec (bit-exact) --------------------------------------------
 * Replace packPhysicalTensorLogicalValues / unpackPhysicalTensorLogicalValues
 * (lib/Wafer/Target/PhysicalTensor/PhysicalTensorCodec.cpp:156-226) with the
 * geometry of computePhysicalTensorGeometry (PhysicalLayout.cpp:111-200).
 * pack writes only the bytes logical elements own: the caller preloads
 * storage with the destination template. */
int wafer_hip_physical_bytes(uint32_t format, uint32_t layout,
                             const int64_t *shape, uint32_t rank,
                             int64_t *bytes);
int wafer_hip_pack(wafer_hip_context *ctx, uint32_t format, uint32_t layout,
                   const int64_t *shape, uint32_t rank, const void *logical,
                   void *storage, int64_t storage_bytes);
int wafer_hip_unpack(wafer_hip_context *ctx, uint32_t format, uint32_t layout,
                     const int64_t *shape, uint32_t rank, const void *storage,
                     int64_t storage_bytes, void *logical);

/* ---- region entries: online attention ---------------------------------------
 * FA prefill.  Semantics of the compiler's online-attention decomposition
 * (lib/Wafer/Transforms/Linalg/OnlineAttentionDecomposition.cpp:568-597,
 * finalize OnlineAttentionMaterialization.cpp:197-262): per KV block,
 * S = f32(q).f32(k) * scale (+ 0/-inf causal bias), m' = max(m, rowmax S),
 * alpha = ExpLp(m - m'), P = ExpLp(S - m'), l = l*alpha + rowsum(P),
 * acc = acc*alpha + bf16(P).V, out = narrow(acc * (1/l)).
 * q [batch, q_heads, q_len, head_dim], k/v [batch, kv_heads, kv_len, head_dim],
 * o like q; q_heads % kv_heads == 0 (GQA: q head h reads kv head
 * h / (q_heads/kv_heads)).  Causal: query i sees key j iff j <= i (and
 * j < kv_len).  format BF16 or F16 (the compiler's F16/BF16 attention
 * formation, include/Wafer/IR/LinalgExt/AttentionOps.td:42-46); head_dim 128
 * or 1..64; any q_len, kv_len >= 1 (kv_len up to 8388607).  head_dim 128
 * (BF16 or F16) runs the dedicated kernel, every other case the kernels of
 * wafer_hip_attention_prefill_masked with the causal flag alone. */
int wafer_hip_attention_prefill(wafer_hip_context *ctx, uint32_t format,
                                const void *q, const void *k, const void *v,
                                void *o, uint32_t batch, uint32_t q_heads,
                                uint32_t kv_heads, uint32_t q_len,
                                uint32_t kv_len, uint32_t head_dim,
                                float scale, uint32_t causal);
/* The same FA prefill on tensors addressed by element strides (batch, head,
 * row) for each of Q, K, V and O, so a caller can pass head slices of a
 * token-major projection ([T, heads * 128] rows) and receive a token-major
 * output without re-layout steps.  Same kernel walk, so the bits equal
 * wafer_hip_attention_prefill on the densely re-laid-out tensors.  BF16 or
 * F16, head_dim 128; strides non-negative multiples of 8, row strides >= 128,
 * 16-byte aligned tensors.  Additive (the reference's attention op has no
 * layout operands); a decoder block's V and O re-layouts are what it removes. */
typedef struct wafer_hip_attention_strides {
  int64_t q[3], k[3], v[3], o[3]; /* elements: batch, head, row */
} wafer_hip_attention_strides;
int wafer_hip_attention_prefill_strided(wafer_hip_context *ctx, uint32_t format,
                                        const void *q, const void *k,
                                        const void *v, void *o, uint32_t batch,
                                        uint32_t q_heads, uint32_t kv_heads,
                                        uint32_t q_len, uint32_t kv_len,
                                        uint32_t head_dim, float scale,
                                        uint32_t causal,
                                        const wafer_hip_attention_strides *strides);

/* FA prefill with the attention op's optional mask operand, its graph-defined
 * score region and its position bias (include/Wafer/IR/LinalgExt/AttentionOps.td:42-64;
 * applyScoreRegion lib/Wafer/Transforms/Linalg/OnlineAttentionDecomposition.cpp:279-426,
 * causal diagonal and valid-prefix ranges :185-210, zero_fully_masked
 * finalize lib/Wafer/Transforms/Linalg/OnlineAttentionMaterialization.cpp:229-242).
 * Per score: t = (q.k) * scale; ROUND_SCALED narrows t to the storage type;
 * with a bias, t = t + bias[b, h, i, j] and ROUND_BIASED narrows that sum;
 * t becomes -inf where key j is invisible to query i: j >= kv_len, CAUSAL
 * and j > i + causal_diagonal (0: top-left aligned as SDPA's is_causal;
 * kv_len - q_len: lower-right aligned), WINDOW and
 * j < i + causal_diagonal - window + 1, or a boolean mask that is zero.
 * A query row with no visible key yields exactly 0.
 * K/V heads are kv_capacity tokens apart (a cache of which the first kv_len
 * tokens are valid: the valid-KV-prefix case).  bias / keep element
 * (b, h, i, j) sits at [b*strides[0] + h*strides[1] + i*strides[2] + j]
 * (stride 0 broadcasts a dimension; j < kv_len is read).
 * format BF16 or F16; head_dim 64 or 128 (MFMA kernel) or 1..63 (one thread
 * per query row).  A NULL mask means no flags and no operands. */
#define WAFER_HIP_ATT_CAUSAL 1u
#define WAFER_HIP_ATT_WINDOW 2u
#define WAFER_HIP_ATT_ROUND_SCALED 4u
#define WAFER_HIP_ATT_ROUND_BIASED 8u
typedef struct wafer_hip_attention_mask {
  uint32_t flags;          /* WAFER_HIP_ATT_* */
  uint32_t kv_capacity;    /* K/V tokens per (batch, kv head); 0 = kv_len */
  int64_t causal_diagonal; /* CAUSAL / WINDOW anchor */
  int64_t window;          /* WINDOW: >= 1 keys ending at the diagonal */
  const float *bias;       /* additive F32 mask or NULL */
  int64_t bias_strides[3]; /* batch, head, query strides in elements */
  const uint8_t *keep;     /* boolean mask (nonzero = visible) or NULL */
  int64_t keep_strides[3];
} wafer_hip_attention_mask;
int wafer_hip_attention_prefill_masked(wafer_hip_context *ctx,
                                       uint32_t format, const void *q,
                                       const void *k, const void *v, void *o,
                                       uint32_t batch, uint32_t q_heads,
                                       uint32_t kv_heads, uint32_t q_len,
                                       uint32_t kv_len, uint32_t head_dim,
                                       float scale,
                                       const wafer_hip_attention_mask *mask);

/* FD decode: one query token per sequence.  Each of `chunks` KV chunks gets
 * its own online state, then the states are folded left to right
 * (lib/Wafer/Transforms/Linalg/SpatialRegionMaterialization.cpp:2391-2430,
 * merge OnlineAttentionMaterialization.cpp:264-373) and finalised as FA.
 * q [batch, q_heads, 1, head_dim]; k/v caches [batch, kv_heads, kv_capacity,
 * head_dim] of which the first kv_len tokens are valid; o like q.
 * format BF16 or F16; head_dim 128; q_heads/kv_heads in {1, 2, 4, 8}.
 * The context owns the partial-state workspace. */
int wafer_hip_attention_decode(wafer_hip_context *ctx, uint32_t format,
                               const void *q, const void *k_cache,
                               const void *v_cache, void *o, uint32_t batch,
                               uint32_t q_heads, uint32_t kv_heads,
                               uint32_t kv_len, uint32_t kv_capacity,
                               uint32_t head_dim, float scale,
                               uint32_t chunks);

/* FD decode without allocation: the same arguments, validation, kernels and
 * results as wafer_hip_attention_decode (bit for bit), for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  This entry has no counterpart in
 * the reference.  The chunk-grid path keeps its chunk states in the library's
 * static device scratch instead of the context workspace: at most 8192
 * states (batch * q_heads * chunks), 4.125 MiB held on each GPU the library
 * runs on until the process ends; a request beyond that fails with
 * WAFER_HIP_E_UNSUPPORTED before any launch.  It calls no hipMalloc / hipFree.
 * All calls on one GPU share that scratch (it keeps the last call's
 * contents; every state is written before it is read), so calls that overlap
 * on one GPU -- on different streams or from different threads -- race.
 * The scratch's device address is resolved by wafer_hip_context_create, so
 * even the first call on a context may run under a graph capture. */
int wafer_hip_attention_decode_noalloc(wafer_hip_context *ctx, uint32_t format,
                                       const void *q, const void *k_cache,
                                       const void *v_cache, void *o,
                                       uint32_t batch, uint32_t q_heads,
                                       uint32_t kv_heads, uint32_t kv_len,
                                       uint32_t kv_capacity, uint32_t head_dim,
                                       float scale, uint32_t chunks);

/* Decode step with the functional KV-cache append the compiler requires of a
 * flash-decoding function (classifyAlgorithm,
 * lib/Wafer/Transforms/Linalg/AttentionMatching.cpp:1385-1437: each of K and
 * V is returned as insert_slice(new, insert_slice(past, ...)) along the
 * sequence axis, as in the board cases attention-causal-decode-two-tokens and
 * attention-decode-kv-cache, test/Board/PyTorch/wafer_pytorch_board_cases.py:
 * 1098-1135, 1138-1360).  The caches are updated in place: rows
 * [past_len, past_len + tokens) of each (batch, kv head) of k_cache / v_cache
 * take k_new / v_new [batch, kv_heads, tokens, head_dim] byte for byte; the
 * first past_len rows are not written (the reference's validate demands the
 * prefix bit for bit).  Then attention of q [batch, q_heads, tokens,
 * head_dim] over the first past_len + tokens cache rows with query i seeing
 * keys j <= past_len + i (SDPA causal_lower_right; one token sees them all):
 * one token with head_dim 128 runs FD decode with `chunks` chunks
 * (wafer_hip_attention_decode), anything else the masked FA prefill
 * (wafer_hip_attention_prefill_masked, causal diagonal past_len, kv_capacity
 * the cache capacity).  o [batch, q_heads, tokens, head_dim].  format BF16 or
 * F16; head_dim 1..64 or 128; past_len + tokens <= kv_capacity. */
int wafer_hip_attention_decode_append(wafer_hip_context *ctx, uint32_t format,
                                      const void *q, const void *k_new,
                                      const void *v_new, void *k_cache,
                                      void *v_cache, void *o, uint32_t batch,
                                      uint32_t q_heads, uint32_t kv_heads,
                                      uint32_t tokens, uint32_t past_len,
                                      uint32_t kv_capacity, uint32_t head_dim,
                                      float scale, uint32_t chunks);

/* ---- region entries: fused TileRegions ----------------------------------------
 * Compositions of the managed elementwise / reduce commands with the op
 * mapping of getInstrElementwiseKindAttr
 * (lib/Wafer/Conversion/TileToInstr/ComputeLowering.cpp:2555-2606: Exp ->
 * ExpLp, Div -> Recip then Mul, no tile-level Sigmoid).  F32 intermediates,
 * one narrowing at the region output.  format F32, BF16 or F16. */
/* y = x * Rsqrt(Sum(x*x) * (1/cols) + eps) * w, per row. */
int wafer_hip_rmsnorm(wafer_hip_context *ctx, uint32_t format, const void *x,
                      const void *w, void *y, uint64_t rows, uint64_t cols,
                      float eps);
/* The residual Add command followed by the RMSNorm region, in one pass:
 * sum = x + r (CT Add, ManagedReferenceTargetModel.cpp:230-299, narrowed to
 * `format`) and y = rmsnorm(sum, w) as wafer_hip_rmsnorm computes it from the
 * stored sum; both outputs equal the two separate commands'.  No reference
 * counterpart as one command (the decoder block's x1 = x + attn; h2 =
 * RMSNorm(x1) pair).  sum and y must be distinct buffers. */
int wafer_hip_add_rmsnorm(wafer_hip_context *ctx, uint32_t format, const void *x,
                          const void *r, const void *w, void *sum, void *y,
                          uint64_t rows, uint64_t cols, float eps);
/* e = ExpLp(x - rowmax); y = e * Recip(Sum(e)). */
int wafer_hip_softmax(wafer_hip_context *ctx, uint32_t format, const void *x,
                      void *y, uint64_t rows, uint64_t cols);
/* y = g * Recip(1 + ExpLp(-g)) * u. */
int wafer_hip_silu_mul(wafer_hip_context *ctx, uint32_t format,
                       const void *gate, const void *up, void *y,
                       uint64_t count);
/* y = 0.5*x*(1 + Tanh(sqrt(2/pi)*(x + 0.044715*x^3))). */
int wafer_hip_gelu_tanh(wafer_hip_context *ctx, uint32_t format, const void *x,
                        void *y, uint64_t count);
/* Rotate-half RoPE over x [tokens, heads, head_dim] with positions [tokens]
 * (int32, device) and inv_freq[i] = 1/theta^(2i/head_dim).  y may alias x. */
int wafer_hip_rope(wafer_hip_context *ctx, uint32_t format, const void *x,
                   void *y, uint64_t tokens, uint64_t heads,
                   uint64_t head_dim, const int32_t *positions, float theta);
/* RoPE fused into the token-major -> head-major re-layout of a projection:
 * dst [heads, tokens, head_dim] = RoPE of src rows (token t, head h at
 * element t * token_stride + h * head_dim), positions [tokens].  Equal bit
 * for bit to wafer_hip_head_permute (direction 0) followed by wafer_hip_rope
 * on the head-major tensor with each row's token position.  The rope step is
 * the rotate-half form of the reference's RoPE region (ComputeLowering.cpp
 * element ops; test/Tools/Inputs/wafer_pytorch_xla_capture.py:1183-1260 for
 * the decoder block); the re-layout is the strided movement between the QKV
 * GEMM and the attention region.  head_dim a multiple of 16, token_stride
 * of 8, tensors 16-byte aligned; dst must not overlap src. */
int wafer_hip_head_permute_rope(wafer_hip_context *ctx, uint32_t format,
                                const void *src, void *dst, uint64_t tokens,
                                uint64_t heads, uint64_t head_dim,
                                uint64_t token_stride,
                                const int32_t *positions, float theta);
/* y = x + bias (bias F32 [cols], broadcast over rows). */
int wafer_hip_bias_add(wafer_hip_context *ctx, uint32_t format, const void *x,
                       const float *bias, void *y, uint64_t rows,
                       uint64_t cols);

/* ---- layout: token-major <-> head-major ---------------------------------------
 * The movement step a lowered decoder layer performs between its fused QKV
 * projection and the attention regions, and back before the output
 * projection (strided head slices, TargetModelStridedMemory.cpp:124-140 for
 * the reference's strided-movement addressing).  Bit-exact copy.
 * direction 0: src token-major, element (t, h, d) at src[t*token_stride +
 * h*head_dim + d] -> dst head-major [heads, tokens, head_dim];
 * direction 1: src head-major -> dst token-major with row stride token_stride.
 * head_dim and token_stride multiples of 16 bytes, tensors 16-byte aligned. */
int wafer_hip_head_permute(wafer_hip_context *ctx, uint32_t format,
                           const void *src, void *dst, uint64_t tokens,
                           uint64_t heads, uint64_t head_dim,
                           uint64_t token_stride, uint32_t direction);

/* ---- movement and fill commands (bit-exact) ------------------------------
 * Strided copy: the DMA read / DMA write / gather-scatter commands
 * (executeMovement, executeGatherScatter,
 * lib/Wafer/Simulator/Kernel/TargetModelMovement.cpp:53-146) over strided byte
 * layouts (forEachStridedSegment, lib/Wafer/Simulator/Memory/TargetModelStridedMemory.cpp:121-145):
 * a layout's segments run with iterations[0] innermost, start at
 * sum coord[d] * strides[d] and hold inner_bytes; the payload (byte_count =
 * segments * inner_bytes) is gathered through the source layout and written
 * through the destination layout.  A contiguous side has strides
 * {inner, inner*it0, inner*it0*it1}.  Field checks follow
 * validateDescriptor (lib/Wafer/Simulator/Kernel/TargetModelCommandValidation.cpp:83-111):
 * byte_count and inner_bytes positive, every iteration positive, byte_count =
 * inner_bytes * segments on both sides.  The source is read completely before
 * any byte is written, so src and dst may overlap.  Destination segments must
 * not overlap each other (WAFER_HIP_E_INVALID_FIELD, nothing written). */
int wafer_hip_strided_copy(wafer_hip_context *ctx, const void *src, void *dst,
                           uint64_t byte_count, uint32_t inner_bytes,
                           const uint32_t src_strides[3],
                           const uint32_t src_iterations[3],
                           const uint32_t dst_strides[3],
                           const uint32_t dst_iterations[3]);
/* Memset (executeMemset, lib/Wafer/Simulator/Kernel/TargetModelTensorNumeric.cpp:875-899):
 * element_count elements of `format` (linear, little-endian; Bool bit-packed
 * LSB first) set to `value`'s bits.  Rejected with WAFER_HIP_E_INVALID_FIELD
 * as TargetModelCommandValidation.cpp:312-325 and NumericCodec.cpp:44-67 do:
 * a zero count, a Bool count that is not a multiple of 8, value bits beyond
 * the storage width, nonzero TF32 padding bits [12:0]. */
int wafer_hip_memset(wafer_hip_context *ctx, void *dst, uint32_t format,
                     uint32_t value, uint64_t element_count);
/* Bit2FP (TargetModelTensorNumeric.cpp:198-233): Bool bits (LSB first) ->
 * 1.0 or +0 in F16/BF16/F32 (other formats: WAFER_HIP_E_UNSUPPORTED; a zero
 * count: WAFER_HIP_E_INVALID_FIELD). */
int wafer_hip_bit2fp(wafer_hip_context *ctx, const void *src_bits, void *dst,
                     uint32_t format, uint64_t element_count);
/* MaskMove (TargetModelTensorNumeric.cpp:235-282): dst[i] = src[i] where
 * mask[i] holds the bits of 1.0; any mask value other than +0 / 1.0 fails
 * with WAFER_HIP_E_UNSUPPORTED before dst is written.  F16/BF16/F32; a zero
 * count is WAFER_HIP_E_INVALID_FIELD. */
int wafer_hip_mask_move(wafer_hip_context *ctx, const void *src,
                        const void *mask, void *dst, uint32_t format,
                        uint64_t element_count);

/* ---- program-boundary comparison (output gate and error statistics) -------
 * compareProgramTensorExpectedOutput and computeProgramTensorComparisonStatistics
 * (lib/Wafer/Simulator/Invocation/ProgramTensorComparison.cpp:267-497;
 * include/Wafer/Simulator/Invocation/ProgramTensorComparison.h:20-71) over
 * device-resident compact row-major tensors.  The entries return WAFER_HIP_OK
 * once the comparison ran; *verdict then holds WAFER_CMP_ACCEPTED or the
 * reference's ProgramTensorComparisonErrorCode + 1, and `detail` (when given)
 * the reference's diagnostic text.  Negative statuses are reserved for misuse
 * of the ABI (null pointers, a byte count that disagrees with dtype and shape)
 * and HIP failures. */

/* ProgramElementType (include/Wafer/Frontend/ProgramElementType.h:17-32). */
enum {
  WAFER_DT_BOOL = 0, WAFER_DT_I8 = 1, WAFER_DT_U8 = 2, WAFER_DT_I16 = 3,
  WAFER_DT_U16 = 4, WAFER_DT_I32 = 5, WAFER_DT_U32 = 6, WAFER_DT_I64 = 7,
  WAFER_DT_U64 = 8, WAFER_DT_F16 = 9, WAFER_DT_BF16 = 10, WAFER_DT_F32 = 11,
  WAFER_DT_TF32 = 12, WAFER_DT_F64 = 13
};

/* ProgramTensorComparisonErrorCode + 1 (ProgramTensorComparison.h:21-32). */
enum {
  WAFER_CMP_ACCEPTED = 0,
  WAFER_CMP_INVALID_TOLERANCE = 1,
  WAFER_CMP_DTYPE_MISMATCH = 2,
  WAFER_CMP_SHAPE_MISMATCH = 3,
  WAFER_CMP_BYTE_SIZE_MISMATCH = 4,
  WAFER_CMP_UNSUPPORTED_FLOATING_DTYPE = 5,
  WAFER_CMP_UNSUPPORTED_STATISTICS_DTYPE = 6,
  WAFER_CMP_ACTUAL_NONFINITE = 7,
  WAFER_CMP_EXPECTED_NONFINITE = 8,
  WAFER_CMP_NUMERIC_MISMATCH = 9,
  WAFER_CMP_RAW_MISMATCH = 10
};

/* A ProgramTensor (dtype, shape, compact bytes) whose bytes are in device
 * memory; `bytes` must equal the element size times the shape product. */
typedef struct wafer_hip_program_tensor {
  uint32_t dtype;
  uint32_t rank;
  const int64_t *shape;
  const void *data;
  uint64_t bytes;
} wafer_hip_program_tensor;

/* ProgramTensorComparisonPolicy (ProgramTensorComparison.h:35-47). */
typedef struct wafer_hip_comparison_policy {
  double atol;
  double rtol;
  uint32_t has_similarity;
  double minimum_cosine;
  double maximum_relative_l2;
} wafer_hip_comparison_policy;

/* ProgramTensorComparisonStatistics (ProgramTensorComparison.h:55-71). */
typedef struct wafer_hip_comparison_statistics {
  uint64_t element_count;
  uint64_t exact_element_count;
  double exact_fraction;
  double mean_absolute_error;
  double p99_absolute_error;
  double p999_absolute_error;
  double maximum_absolute_error;
  uint64_t elementwise_mismatch_count;
  double cosine_similarity;
  double relative_l2_error;
  double mean_ulp_distance;
  uint64_t p99_ulp_distance;
  uint64_t p999_ulp_distance;
  uint64_t maximum_ulp_distance;
} wafer_hip_comparison_statistics;

/* The output gate: F16 / BF16 / F32 elementwise (|a - e| <= atol + rtol |e|)
 * or, with has_similarity, cosine >= minimum and relative L2 <= maximum over
 * the whole tensor; other floating dtypes fail closed; integer and Bool
 * storage compare byte for byte.  Replaces compareProgramTensorExpectedOutput
 * (ProgramTensorComparison.cpp:267-387). */
int wafer_hip_compare_expected(wafer_hip_context *ctx,
                               const wafer_hip_program_tensor *actual,
                               const wafer_hip_program_tensor *expected,
                               const wafer_hip_comparison_policy *policy,
                               uint32_t *verdict, char *detail,
                               size_t detail_bytes);
/* The error distribution of a finite F16 / BF16 / F32 pair: nearest-rank
 * quantiles over all elements, sign-aware ULP distances (equal signed zeros
 * at distance 0).  `policy` (may be NULL: atol = rtol = 0) sets only the
 * diagnostic mismatch count.  Replaces computeProgramTensorComparisonStatistics
 * (ProgramTensorComparison.cpp:389-497).  The ULP-distance sum is exact below
 * 2^64 (any F16/BF16 tensor; F32 tensors below 2^32 elements). */
int wafer_hip_compare_statistics(wafer_hip_context *ctx,
                                 const wafer_hip_program_tensor *actual,
                                 const wafer_hip_program_tensor *expected,
                                 const wafer_hip_comparison_policy *policy,
                                 uint32_t *verdict,
                                 wafer_hip_comparison_statistics *out,
                                 char *detail, size_t detail_bytes);

#ifdef __cplusplus
}
#endif

#endif /* WAFER_HIP_H */
