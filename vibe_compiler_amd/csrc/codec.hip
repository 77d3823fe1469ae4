// codec.hip -- physical tensor codec on the GPU (bit-exact).
//
// Geometry of computePhysicalTensorGeometry
// (lib/Wafer/Target/PhysicalTensor/PhysicalLayout.cpp:111-200) and offsets of
// getBitOffset (:249-310):
//  * Tensor / NTensor: compact row-major span;
//  * Cx: the channel dimension C (last) splits into blocks of 64 channels
//    (128 for I8/U8); a remainder of at most 32 (64 for int8) is kept as a
//    tail aligned up to {4, 8, 16, 32, 64}, a larger one becomes a padded
//    full block (alignCxTail / computeCxC0, :51-85).  Storage is
//    [c_block][outer][64] followed by the tail [outer][c0]; the whole span is
//    aligned to a 256-byte bank line;
//  * NCx: the same per leading-N slice, each slice with its own bank-aligned
//    stride.
// pack writes only the bytes logical elements own, so padding keeps the
// destination template's bytes (PhysicalTensorCodec.cpp:189-226); the caller
// preloads storage with the template.  One thread per logical element.
#include "common.h"

namespace wafer {
namespace {

struct CodecGeom {
  int layout, rank, ebytes;
  int64_t shape[8];
  int64_t count;
  int64_t c_block, cx_blocks, c0, block_outer, slice_stride;
  int64_t physical_bytes;
};

int64_t align_up(int64_t v, int64_t a) { return v % a == 0 ? v : v + (a - v % a); }
int64_t align_tail(int64_t t) { return t <= 4 ? 4 : t <= 8 ? 8 : t <= 16 ? 16 : t <= 32 ? 32 : 64; }

int element_bits(uint32_t f) {
  static const int bits[] = {8, 16, 16, 16, 32, 32, 32, 1, 8, 16, 32, 64, 64};
  return f <= 12 ? bits[f] : -1;
}

int make_geom(uint32_t format, uint32_t layout, const int64_t *shape, uint32_t rank,
              CodecGeom *g) {
  const int bits = element_bits(format);
  if (bits < 0) return fail(WAFER_HIP_E_CODEC, "codec: unknown format");
  if (layout > 3) return fail(WAFER_HIP_E_CODEC, "codec: unknown layout");
  if (rank > 8 || (rank > 0 && !shape)) return fail(WAFER_HIP_E_CODEC, "codec: rank must be 0..8");
  *g = CodecGeom{};
  g->layout = (int)layout;
  g->rank = (int)rank;
  g->ebytes = bits / 8;
  g->count = 1;
  for (uint32_t i = 0; i < rank; ++i) {
    if (shape[i] < 0) return fail(WAFER_HIP_E_CODEC, "codec: negative dimension");
    g->shape[i] = shape[i];
    g->count *= shape[i];
  }
  if (layout == WAFER_LAYOUT_TENSOR || layout == WAFER_LAYOUT_NTENSOR) {
    g->physical_bytes = (g->count * bits + 7) / 8;
    return WAFER_HIP_OK;
  }
  if (rank == 0) return fail(WAFER_HIP_E_CODEC, "codec: Cx/NCx need rank >= 1");
  const bool i8block = format == WAFER_FMT_I8 || format == WAFER_FMT_U8;
  const int64_t block = i8block ? 128 : 64, retain = i8block ? 64 : 32;
  const int64_t c = shape[rank - 1], q = c / block, r = c % block;
  int64_t aligned_c;
  if (r == 0) { g->cx_blocks = q; g->c0 = 0; aligned_c = q * block; }
  else if (r <= retain) { g->cx_blocks = q; g->c0 = align_tail(r); aligned_c = q * block + g->c0; }
  else { g->cx_blocks = q + 1; g->c0 = 0; aligned_c = (q + 1) * block; }
  g->c_block = block;
  const int64_t bank = 2048 / bits;
  if (layout == WAFER_LAYOUT_NCX) {
    const int64_t slices = rank > 1 ? shape[0] : 1;
    int64_t bo = 1;
    for (uint32_t i = 1; i + 1 < rank; ++i) bo *= shape[i];
    g->block_outer = bo;
    g->slice_stride = align_up(bo * aligned_c, bank);
    g->physical_bytes = slices * g->slice_stride * bits / 8;
  } else {
    int64_t outer = 1;
    for (uint32_t i = 0; i + 1 < rank; ++i) outer *= shape[i];
    g->block_outer = outer;
    g->slice_stride = align_up(outer * aligned_c, bank);
    g->physical_bytes = g->slice_stride * bits / 8;
  }
  return WAFER_HIP_OK;
}

__device__ inline int64_t element_offset(const CodecGeom &g, int64_t linear) {
  if (g.layout == WAFER_LAYOUT_TENSOR || g.layout == WAFER_LAYOUT_NTENSOR) return linear;
  const int64_t cdim = g.shape[g.rank - 1];
  const int64_t c = linear % cdim;
  const int64_t rest = linear / cdim;  // row-major index over the leading dims
  int64_t phys = 0, outer = rest;
  if (g.layout == WAFER_LAYOUT_NCX && g.rank > 1) {
    const int64_t slice = rest / g.block_outer;
    outer = rest - slice * g.block_outer;
    phys = slice * g.slice_stride;
  }
  const int64_t full_c = g.cx_blocks * g.c_block;
  const int64_t block_stride = g.block_outer * g.c_block;
  if (c < full_c)
    phys += (c / g.c_block) * block_stride + outer * g.c_block + c % g.c_block;
  else
    phys += g.cx_blocks * block_stride + outer * g.c0 + (c - full_c);
  return phys;
}

template <int EB>
__global__ __launch_bounds__(256) void codec_kernel(CodecGeom g, const uint8_t *__restrict__ src,
                                                    uint8_t *__restrict__ dst, int pack) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < g.count; e += stride) {
    const int64_t p = element_offset(g, e);
    const uint8_t *s = pack ? src + e * EB : src + p * EB;
    uint8_t *d = pack ? dst + p * EB : dst + e * EB;
    if (EB == 1) *d = *s;
    else if (EB == 2) *(uint16_t *)d = *(const uint16_t *)s;
    else if (EB == 4) *(uint32_t *)d = *(const uint32_t *)s;
    else *(uint64_t *)d = *(const uint64_t *)s;
  }
}

int run_codec(wafer_hip_context *ctx, uint32_t format, uint32_t layout, const int64_t *shape,
              uint32_t rank, const void *src, void *dst, int64_t storage_bytes, int pack) {
  WAFER_CHECK_CTX(ctx);
  CodecGeom g;
  WAFER_TRY(make_geom(format, layout, shape, rank, &g));
  if (format == WAFER_FMT_BOOL)
    return fail(WAFER_HIP_E_UNSUPPORTED, "codec: bit-packed Bool tensors are not served on the GPU");
  if (storage_bytes != g.physical_bytes)
    return fail(WAFER_HIP_E_CODEC, "codec: storage size " + std::to_string(storage_bytes) +
                                       " != physical size " + std::to_string(g.physical_bytes));
  if (g.count == 0) return WAFER_HIP_OK;
  if (!src || !dst) return fail(WAFER_HIP_E_INVALID_FIELD, "codec: null tensor");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  const unsigned blocks = (unsigned)std::min<int64_t>((g.count + 255) / 256, 65536);
  switch (g.ebytes) {
  case 1: hipLaunchKernelGGL(codec_kernel<1>, dim3(blocks), dim3(256), 0, ctx->stream, g, (const uint8_t *)src, (uint8_t *)dst, pack); break;
  case 2: hipLaunchKernelGGL(codec_kernel<2>, dim3(blocks), dim3(256), 0, ctx->stream, g, (const uint8_t *)src, (uint8_t *)dst, pack); break;
  case 4: hipLaunchKernelGGL(codec_kernel<4>, dim3(blocks), dim3(256), 0, ctx->stream, g, (const uint8_t *)src, (uint8_t *)dst, pack); break;
  default: hipLaunchKernelGGL(codec_kernel<8>, dim3(blocks), dim3(256), 0, ctx->stream, g, (const uint8_t *)src, (uint8_t *)dst, pack); break;
  }
  return launch_status("codec_kernel");
}

}  // namespace
}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_physical_bytes(uint32_t format, uint32_t layout, const int64_t *shape,
                                        uint32_t rank, int64_t *bytes) {
  if (!bytes) return fail(WAFER_HIP_E_INVALID_FIELD, "physical_bytes: null output");
  CodecGeom g;
  WAFER_TRY(make_geom(format, layout, shape, rank, &g));
  *bytes = g.physical_bytes;
  return WAFER_HIP_OK;
}

extern "C" int wafer_hip_pack(wafer_hip_context *ctx, uint32_t format, uint32_t layout,
                              const int64_t *shape, uint32_t rank, const void *logical,
                              void *storage, int64_t storage_bytes) {
  return run_codec(ctx, format, layout, shape, rank, logical, storage, storage_bytes, 1);
}

extern "C" int wafer_hip_unpack(wafer_hip_context *ctx, uint32_t format, uint32_t layout,
                                const int64_t *shape, uint32_t rank, const void *storage,
                                int64_t storage_bytes, void *logical) {
  return run_codec(ctx, format, layout, shape, rank, storage, logical, storage_bytes, 0);
}
