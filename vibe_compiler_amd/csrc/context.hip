// context.hip -- context lifecycle, stream binding, error reporting and the
// workspace allocator shared by the entry points.
#include "common.h"

#include <cstdio>

namespace wafer {

static thread_local std::string g_last_error;

void set_error(const std::string &message) { g_last_error = message; }

int fail(int code, const std::string &message) {
  g_last_error = message;
  return code;
}

int check_hip(hipError_t err, const char *what) {
  if (err == hipSuccess) return WAFER_HIP_OK;
  char buf[256];
  std::snprintf(buf, sizeof(buf), "%s: %s", what, hipGetErrorString(err));
  return fail(WAFER_HIP_E_RUNTIME, buf);
}

int launch_status(const char *kernel) {
  return check_hip(hipGetLastError(), kernel);
}

int refuse_capture(wafer_hip_context *ctx, const char *what) {
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  WAFER_TRY(check_hip(hipStreamIsCapturing(ctx->stream, &capture), "hipStreamIsCapturing"));
  if (capture != hipStreamCaptureStatusNone)
    return fail(WAFER_HIP_E_UNSUPPORTED,
                std::string(what) + ": synchronises the stream or allocates, which a stream capture cannot record");
  return WAFER_HIP_OK;
}

namespace {
__global__ void fill_words_kernel(uint32_t *p, uint32_t n, uint32_t value) {
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) p[i] = value;
}
}  // namespace

int fill_words(wafer_hip_context *ctx, void *p, uint32_t n, uint32_t value) {
  hipLaunchKernelGGL(fill_words_kernel, dim3(1), dim3(64), 0, ctx->stream, (uint32_t *)p, n, value);
  return launch_status("fill_words_kernel");
}

int status_words(wafer_hip_context *ctx, const char *what, uint8_t **words) {
  WAFER_TRY(refuse_capture(ctx, what));
  if (!ctx->status) WAFER_TRY(check_hip(hipMalloc((void **)&ctx->status, 256), "hipMalloc(status)"));
  *words = (uint8_t *)ctx->status;
  return WAFER_HIP_OK;
}

// Grows *slot to at least `need` bytes (whole MiB, and at least twice the
// old size, so the buffers a slot retires sum to less than its current
// size).  The old buffer is not freed: it moves to ctx->retired and lives
// until the context is destroyed, so kernels still in flight on it and
// graphs captured while it was current keep valid memory.  The new buffer's
// contents are undefined.  Growing is refused on a capturing stream (the
// allocation cannot be recorded); a slot that is large enough is used as it
// is.
int ensure_workspace(wafer_hip_context *ctx, void **slot, size_t *slot_bytes,
                     size_t need) {
  if (*slot_bytes >= need) return WAFER_HIP_OK;
  WAFER_TRY(refuse_capture(ctx, "growing the context workspace"));
  size_t rounded = (need + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
  if (*slot && rounded < 2 * *slot_bytes) rounded = 2 * *slot_bytes;
  void *grown = nullptr;
  WAFER_TRY(check_hip(hipMalloc(&grown, rounded), "hipMalloc(workspace)"));
  if (*slot) ctx->retired.push_back(*slot);
  *slot = grown;
  *slot_bytes = rounded;
  return WAFER_HIP_OK;
}

}  // namespace wafer

using namespace wafer;

extern "C" int wafer_hip_context_create(int device, wafer_hip_context **out) {
  if (!out) return fail(WAFER_HIP_E_INVALID_FIELD, "null output pointer");
  *out = nullptr;
  int count = 0;
  WAFER_TRY(check_hip(hipGetDeviceCount(&count), "hipGetDeviceCount"));
  if (device < 0 || device >= count)
    return fail(WAFER_HIP_E_UNAVAILABLE, "no HIP device " + std::to_string(device));
  hipDeviceProp_t prop;
  WAFER_TRY(check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(WAFER_HIP_E_UNAVAILABLE,
                std::string("device is ") + prop.gcnArchName + ", kernels are built for gfx950");
  // the no-allocation decode entry's scratch address, resolved here (once
  // per device) rather than at that entry's first call, which may run
  // under a graph capture
  WAFER_TRY(noalloc_scratch_lookup(device));
  auto *ctx = new wafer_hip_context();
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount;
  *out = ctx;
  return WAFER_HIP_OK;
}

extern "C" int wafer_hip_context_destroy(wafer_hip_context *ctx) {
  if (!ctx) return WAFER_HIP_OK;
  int st = WAFER_HIP_OK;
  if (ctx->workspace || ctx->relayout || ctx->status || ctx->partials || !ctx->retired.empty()) {
    st = check_hip(hipSetDevice(ctx->device), "hipSetDevice");
    if (st == WAFER_HIP_OK) st = check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (ctx->workspace) st = check_hip(hipFree(ctx->workspace), "hipFree(workspace)");
    if (ctx->relayout) st = check_hip(hipFree(ctx->relayout), "hipFree(relayout)");
    if (ctx->status) st = check_hip(hipFree(ctx->status), "hipFree(status)");
    if (ctx->partials) st = check_hip(hipFree(ctx->partials), "hipFree(partials)");
    for (void *p : ctx->retired) st = check_hip(hipFree(p), "hipFree(retired workspace)");
  }
  delete ctx;
  return st;
}

extern "C" int wafer_hip_set_stream(wafer_hip_context *ctx, void *hip_stream) {
  WAFER_CHECK_CTX(ctx);
  ctx->stream = (hipStream_t)hip_stream;
  return WAFER_HIP_OK;
}

extern "C" int wafer_hip_synchronize(wafer_hip_context *ctx) {
  WAFER_CHECK_CTX(ctx);
  return check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

extern "C" const char *wafer_hip_last_error(void) { return g_last_error.c_str(); }

extern "C" const char *wafer_hip_implementation(void) {
  return "wafer-hip gfx950: formal-order FMA GEMM, bf16/f16/i8 MFMA GEMM, "
         "FA prefill (mfma_f32_32x32x16_bf16), FD decode (mfma_f32_16x16x32_bf16 + LSE fold), "
         "managed elementwise/convert/reduce, Cx/NCx codec, fused regions";
}

extern "C" int wafer_hip_environment(wafer_hip_context *ctx, wafer_hip_environment_info *out) {
  WAFER_CHECK_CTX(ctx);
  if (!out) return fail(WAFER_HIP_E_INVALID_FIELD, "environment: null output");
  memset(out, 0, sizeof *out);
  hipDeviceProp_t prop;
  WAFER_TRY(check_hip(hipGetDeviceProperties(&prop, ctx->device), "hipGetDeviceProperties"));
  strncpy(out->gcn_arch_name, prop.gcnArchName, sizeof out->gcn_arch_name - 1);
  strncpy(out->device_name, prop.name, sizeof out->device_name - 1);
  out->compute_units = prop.multiProcessorCount;
  out->warp_size = prop.warpSize;
  out->global_memory_bytes = prop.totalGlobalMem;
  out->lds_bytes_per_block = prop.sharedMemPerBlock;
  int v = 0;
  WAFER_TRY(check_hip(hipRuntimeGetVersion(&v), "hipRuntimeGetVersion"));
  out->hip_runtime_version = v;
  WAFER_TRY(check_hip(hipDriverGetVersion(&v), "hipDriverGetVersion"));
  out->driver_version = v;
  return WAFER_HIP_OK;
}

// ---- device buffers for host-side callers ---------------------------------
// The seam adapter moves TargetModelNumericTensor storage through these, so
// it needs nothing but this ABI.  Copies are ordered on the context's stream
// and complete before the call returns.
extern "C" int wafer_hip_buffer_alloc(wafer_hip_context *ctx, uint64_t bytes, void **out) {
  WAFER_CHECK_CTX(ctx);
  if (!out) return fail(WAFER_HIP_E_INVALID_FIELD, "buffer_alloc: null output pointer");
  *out = nullptr;
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  return check_hip(hipMalloc(out, bytes ? bytes : 1), "hipMalloc(buffer)");
}

extern "C" int wafer_hip_buffer_free(wafer_hip_context *ctx, void *buffer) {
  WAFER_CHECK_CTX(ctx);
  if (!buffer) return WAFER_HIP_OK;
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  WAFER_TRY(check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize"));
  return check_hip(hipFree(buffer), "hipFree(buffer)");
}

extern "C" int wafer_hip_copy_to_device(wafer_hip_context *ctx, void *dst, const void *src, uint64_t bytes) {
  WAFER_CHECK_CTX(ctx);
  if (bytes == 0) return WAFER_HIP_OK;
  if (!dst || !src) return fail(WAFER_HIP_E_INVALID_FIELD, "copy_to_device: null pointer");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  WAFER_TRY(check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync(H2D)"));
  return check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

extern "C" int wafer_hip_copy_to_host(wafer_hip_context *ctx, void *dst, const void *src, uint64_t bytes) {
  WAFER_CHECK_CTX(ctx);
  if (bytes == 0) return WAFER_HIP_OK;
  if (!dst || !src) return fail(WAFER_HIP_E_INVALID_FIELD, "copy_to_host: null pointer");
  WAFER_TRY(check_hip(hipSetDevice(ctx->device), "hipSetDevice"));
  WAFER_TRY(check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync(D2H)"));
  return check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}
