/*
 * wafer_oracle.h -- CPU restatement of the Wafer Reference backend semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * backend in vibe_compiler_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only to check or to time the
 * CPU lane.  The product path never links it and has no CPU fallback.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the PJLAB-CHIP/vibe_compiler tree).  Raw values are passed as their
 * storage bits: bf16/f16 as uint16_t, f32 as float, i8 as int8_t.
 *
 * Format codes follow the reference's Data_Format table
 * (lib/Wafer/Target/TargetFormat.cpp:62-63): I8=0 I16=1 F16=2 BF16=3 I32=4
 * F32=5 TF32=6 Bool=7 U8=8 U16=9 U32=10 I64=11 U64=12.
 */
#ifndef WAFER_ORACLE_H
#define WAFER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------- */
uint16_t oracle_f32_to_bf16(float value);   /* RNE, canonical qNaN 0x7fc0 */
float oracle_bf16_to_f32(uint16_t bits);
int oracle_f32_to_f16(float value, uint16_t *bits); /* 0 ok, -1 NaN */
float oracle_f16_to_f32(uint16_t bits);
float oracle_explp(float x);
float oracle_gemm_fma(float a, float b, float acc);

/* ---- physical layout codec (Tensor/NTensor/Cx/NCx) ----------------------- */
enum { ORACLE_LAYOUT_TENSOR = 0, ORACLE_LAYOUT_NTENSOR = 1,
       ORACLE_LAYOUT_CX = 2, ORACLE_LAYOUT_NCX = 3 };

typedef struct {
  int64_t physical_elements;
  int64_t physical_bytes;
  int64_t element_bits;
  int64_t c_block;
  int64_t cx_blocks;
  int64_t c0;
  int64_t aligned_c;
  int64_t outer_elements;
  int64_t block_outer_elements;
  int64_t outer_slice_stride;
  int64_t bank_align_elements;
} oracle_geometry;

int oracle_format_bits(int format);
int oracle_geometry_compute(int format, int layout, const int64_t *shape,
                            int rank, oracle_geometry *out);
int64_t oracle_bit_offset(int format, int layout, const int64_t *shape,
                          int rank, const int64_t *index);
int oracle_pack(int format, int layout, const int64_t *shape, int rank,
                const void *logical, uint8_t *storage, int64_t storage_bytes);
int oracle_unpack(int format, int layout, const int64_t *shape, int rank,
                  const uint8_t *storage, int64_t storage_bytes,
                  void *logical);

/* ---- formal GEMM -------------------------------------------------------- */
int oracle_gemm_formal(int in_format, int out_format, const void *lhs,
                       const void *rhs, const float *psum, void *dst,
                       int64_t m, int64_t k, int64_t n, int64_t batch,
                       int lhs_transpose, int rhs_transpose, int threads);

/* ---- int8 GEMM, exact int32 then dequant chain -------------------------- */
int oracle_gemm_i8(const int8_t *a, const int8_t *b, const float *scale,
                   int32_t *acc_out, uint16_t *y_bf16, int64_t m, int64_t k,
                   int64_t n, int rhs_transpose, int threads);

/* ---- managed-reference elementwise / convert / reduce ------------------- */
int oracle_elementwise(int op, int format, const void *in0, const void *in1,
                       void *dst, int64_t count);
int oracle_convert(int opcode, int rounding, const void *src, void *dst,
                   int64_t count);
int oracle_reduce(int op, int dim, int format, const int64_t *shape, int rank,
                  const void *src, void *dst);

/* ---- online attention (FA prefill, FD decode) --------------------------- */
int oracle_attention_prefill(int format, const uint16_t *q, const uint16_t *k,
                             const uint16_t *v, uint16_t *o, int batch,
                             int q_heads, int kv_heads, int q_len, int kv_len,
                             int head_dim, float scale, int causal,
                             int block_k, int threads);
/* flags: 1 causal (key j <= i + diagonal), 2 window (key j > i + diagonal -
 * window), 4 round the scaled score to the storage type, 8 round the score
 * plus additive mask to the storage type. */
int oracle_attention_prefill_ex(int format, const uint16_t *q,
                                const uint16_t *k, const uint16_t *v,
                                uint16_t *o, int batch, int q_heads,
                                int kv_heads, int q_len, int kv_len,
                                int kv_capacity, int head_dim, float scale,
                                uint32_t flags, int64_t diagonal,
                                int64_t window, const float *bias,
                                int64_t bias_sb, int64_t bias_sh,
                                int64_t bias_sq, const uint8_t *keep,
                                int64_t keep_sb, int64_t keep_sh,
                                int64_t keep_sq, int block_k, int threads);
float oracle_attention_score(int format, uint32_t flags, float raw,
                             float scale, const float *bias);
int oracle_attention_decode(int format, const uint16_t *q,
                            const uint16_t *k_cache, const uint16_t *v_cache,
                            uint16_t *o, int batch, int q_heads, int kv_heads,
                            int kv_len, int kv_capacity, int head_dim,
                            float scale, int chunks, int block_k,
                            int threads);

/* ---- fused regions ------------------------------------------------------ */
int oracle_rmsnorm(int format, const void *x, const void *w, void *y,
                   int64_t rows, int64_t cols, float eps);
int oracle_softmax(int format, const void *x, void *y, int64_t rows,
                   int64_t cols);
int oracle_silu_mul(int format, const void *gate, const void *up, void *y,
                    int64_t count);
int oracle_gelu_tanh(int format, const void *x, void *y, int64_t count);
int oracle_rope(int format, const void *x, void *y, int64_t tokens,
                int64_t heads, int64_t head_dim, const int32_t *positions,
                float theta);
int oracle_bias_add(int format, const void *x, const float *bias, void *y,
                    int64_t rows, int64_t cols);

/* ---- movement and fill commands ---------------------------------------- */
int oracle_strided_copy(const uint8_t *src, uint8_t *dst, uint32_t inner_bytes,
                        const uint32_t src_strides[3], const uint32_t src_iterations[3],
                        const uint32_t dst_strides[3], const uint32_t dst_iterations[3]);
int oracle_memset(uint8_t *dst, int format, uint32_t value, int64_t count);
int oracle_bit2fp(const uint8_t *bits, void *dst, int format, int64_t count);
int oracle_mask_move(const void *src, const void *mask, void *dst, int format, int64_t count);

/* ---- formal-lane elementwise and pooling --------------------------------- */
/* Logical tensors (F16 / BF16 as uint16 bits, F32 as uint32 bits, Bool as one
 * byte 0 / 1).  Returns 0, -1 for an operation outside the formal subset,
 * -3 for a Bool operand byte other than 0 / 1. */
int oracle_elementwise_formal(int op, int format, int relation_numeric, uint32_t unit, uint32_t group,
                              int has_scalar, uint32_t scalar, const void *lhs, const void *rhs, void *dst,
                              int64_t count);
/* op TargetPoolingOperation 116 Sum, 117 Maximum, 119 Minimum; NHWC shapes;
 * kernel_strides {kernel W, kernel H, stride W, stride H}. */
int oracle_pool(int op, int format, const uint32_t *src_shape, const uint32_t *dst_shape,
                const uint32_t *kernel_strides, const void *src, void *dst);

/* ---- program-boundary comparison ----------------------------------------- */
typedef struct oracle_cmp_stats {
  uint64_t element_count, exact_element_count;
  double exact_fraction, mean_absolute_error, p99_absolute_error, p999_absolute_error,
      maximum_absolute_error;
  uint64_t elementwise_mismatch_count;
  double cosine_similarity, relative_l2_error, mean_ulp_distance;
  uint64_t p99_ulp_distance, p999_ulp_distance, maximum_ulp_distance;
} oracle_cmp_stats;
/* dtype: 9 F16, 10 BF16, 11 F32 (ProgramElementType).  Returns the verdict
 * (0 accepted, ProgramTensorComparisonErrorCode + 1 otherwise); info[0..4] =
 * element that ended the scan, mismatch count, first mismatch, largest-error
 * mismatch, largest-ratio mismatch. */
int oracle_compare_floats(int dtype, const void *actual, const void *expected, int64_t n, double atol,
                          double rtol, int has_similarity, double minimum_cosine, double maximum_relative_l2,
                          double *cosine_out, double *relative_l2_out, int64_t *info);
int oracle_compare_statistics(int dtype, const void *actual, const void *expected, int64_t n, double atol,
                              double rtol, oracle_cmp_stats *out, int64_t *bad_element);

#ifdef __cplusplus
}
#endif

#endif
