// heads.hip -- token-major <-> head-major re-layout of attention operands.
//
// The projections of a decoder layer produce token-major rows
// [tokens, heads * head_dim] (Q, K and V side by side in one fused QKV
// output), while the attention regions read head-major tensors
// [heads, tokens, head_dim].  The reference compiler performs this step as
// a layout/movement command between the GEMM and the attention region
// (strided RDMA of the head slices); here it is one coalesced copy, bit
// for bit, 16 bytes per lane.
#include "common.h"

namespace wafer {
namespace {

// One lane moves one 16-byte piece.  dir 0: src token-major (row stride
// `ts` elements) -> dst head-major; dir 1: src head-major -> dst token-major
// (row stride `ts`).  `pieces` = head_dim * esize / 16.
__global__ __launch_bounds__(256) void head_permute_kernel(const uint8_t *__restrict__ src,
                                                           uint8_t *__restrict__ dst,
                                                           int64_t tokens, int64_t heads,
                                                           int64_t pieces, int64_t ts_bytes,
                                                           int dir) {
  const int64_t total = tokens * heads * pieces;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t row_bytes = pieces * 16;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    // e enumerates the head-major side: (h, t, piece), so the head-major
    // accesses are fully contiguous and the token-major ones are runs of
    // head_dim elements
    const int64_t p = e % pieces;
    const int64_t ht = e / pieces;
    const int64_t t = ht % tokens;
    const int64_t h = ht / tokens;
    const int64_t tok_off = t * ts_bytes + h * row_bytes + p * 16;
    const int64_t head_off = e * 16;
    if (dir == 0)
      *(u32x4 *)(dst + head_off) = *(const u32x4 *)(src + tok_off);
    else
      *(u32x4 *)(dst + tok_off) = *(const u32x4 *)(src + head_off);
  }
}

}  // namespace
}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_head_permute(wafer_hip_context *ctx, uint32_t format, const void *src,
                                      void *dst, uint64_t tokens, uint64_t heads,
                                      uint64_t head_dim, uint64_t token_stride,
                                      uint32_t direction) {
  WAFER_CHECK_CTX(ctx);
  if (!is_float_format(format))
    return fail(WAFER_HIP_E_UNSUPPORTED, "head_permute: format must be F16, BF16 or F32");
  if (direction > 1) return fail(WAFER_HIP_E_INVALID_FIELD, "head_permute: direction must be 0 or 1");
  const uint64_t esize = format == WAFER_FMT_F32 ? 4 : 2;
  if (tokens == 0 || heads == 0 || head_dim == 0) return WAFER_HIP_OK;
  if (!src || !dst) return fail(WAFER_HIP_E_INVALID_FIELD, "head_permute: null tensor");
  if ((head_dim * esize) % 16 != 0 || (token_stride * esize) % 16 != 0)
    return fail(WAFER_HIP_E_UNSUPPORTED, "head_permute: head_dim and token_stride must be multiples of 16 bytes");
  if (token_stride < heads * head_dim)
    return fail(WAFER_HIP_E_INVALID_FIELD, "head_permute: token_stride < heads * head_dim");
  if (((uintptr_t)src | (uintptr_t)dst) % 16 != 0)
    return fail(WAFER_HIP_E_INVALID_FIELD, "head_permute: tensors must be 16-byte aligned");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const uint64_t pieces = head_dim * esize / 16;
  const uint64_t total = tokens * heads * pieces;
  const unsigned grid = (unsigned)std::min<uint64_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(head_permute_kernel, dim3(grid), dim3(256), 0, ctx->stream,
                     (const uint8_t *)src, (uint8_t *)dst, (int64_t)tokens, (int64_t)heads,
                     (int64_t)pieces, (int64_t)(token_stride * esize), (int)direction);
  return launch_status("head_permute_kernel");
}
