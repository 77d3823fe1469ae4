// npy_payload.h -- program-boundary I/O: the .npy payload codec of the
// reference's frontend (lib/Wafer/Frontend/NpyPayload.cpp), restated in
// plain C++17 so that a host program can load expected and input tensors,
// hand them to the device (wafer_hip_copy_to_device) and gate results with
// wafer_hip_compare_expected.
//
//   loadNpyTensorPayload   NpyPayload.cpp:368-413   (whole file -> dtype, shape, bytes)
//   parseNpyPayloadHeader  NpyPayload.cpp:415-430   (header only)
//   decodeProgramNpyDescr  NpyPayload.cpp:432-446   (descr -> ProgramElementType, bytes)
//
// Rules kept from the reference: magic "\x93NUMPY"; versions 1 (u16 header
// length at byte 8) and 2 (u32 at byte 8); headers above 1 MiB rejected; the
// 'descr', 'fortran_order' and 'shape' fields are required, Fortran order is
// rejected; descr '<f4' '<f8' '<f2' '|V2' (bf16) '|b1' '|i1' '<i2' '<i4'
// '<i8' (and '=' for '<' on a little-endian host); the payload must hold
// dtype size x shape product bytes (trailing bytes are ignored).
#pragma once

#include <cstdint>
#include <optional>
#include <string>
#include <utility>
#include <vector>

namespace wafer::model {

// ProgramElementType (include/Wafer/Frontend/ProgramElementType.h:17-32),
// the numbering of the C ABI's WAFER_DT_* codes.
enum class ProgramElementType : uint8_t { Bool, I8, U8, I16, U16, I32, U32, I64, U64, F16, BF16, F32, TF32, F64 };

struct NpyTensorPayload {
  ProgramElementType dtype;
  std::vector<int64_t> shape;
  std::vector<uint8_t> bytes;
};

struct NpyPayloadHeader {
  uint64_t fileSize = 0;
  uint64_t dataOffset = 0;
  std::string descr;
  bool fortranOrder = false;
  std::vector<int64_t> shape;
};

// A value or an error message (the reference returns llvm::Expected with an
// invalid_argument StringError).
template <typename T> struct NpyResult {
  std::optional<T> value;
  std::string error;
  explicit operator bool() const { return value.has_value(); }
};

NpyResult<NpyTensorPayload> loadNpyTensorPayload(const std::string &path);
NpyResult<NpyPayloadHeader> parseNpyPayloadHeader(const std::string &path);
std::optional<std::pair<ProgramElementType, uint64_t>> decodeProgramNpyDescr(const std::string &descr);

}  // namespace wafer::model

// C entry points for callers without C++ (a ctypes binding, a C driver).
// wafer_npy_load returns 0 and fills *dtype (WAFER_DT_*), shape[0..*rank)
// (at most max_rank entries), *data (malloc'ed, released with wafer_npy_free)
// and *bytes; on failure it returns -1 and writes the message into `error`.
extern "C" int wafer_npy_load(const char *path, uint32_t *dtype, int64_t *shape, uint32_t max_rank,
                              uint32_t *rank, uint8_t **data, uint64_t *bytes, char *error, size_t error_bytes);
extern "C" void wafer_npy_free(uint8_t *data);
