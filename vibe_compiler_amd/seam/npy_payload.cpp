// npy_payload.cpp -- the .npy payload codec (see npy_payload.h for the
// reference functions it restates).
#include "npy_payload.h"

#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <limits>

namespace wafer::model {
namespace {

// Upper bound for a parsed header (NpyPayload.cpp:29-32).
constexpr uint64_t kMaximumNpyHeaderBytes = 1 << 20;

bool little_endian_host() {
  const uint16_t probe = 1;
  uint8_t first;
  std::memcpy(&first, &probe, 1);
  return first == 1;
}

std::string trim_left(const std::string &s, size_t from) {
  while (from < s.size() && (s[from] == ' ' || s[from] == '\t' || s[from] == '\n' || s[from] == '\r')) ++from;
  return s.substr(from);
}

// The text after "'field':" (or "\"field\":"), left-trimmed
// (findNpyFieldValue, NpyPayload.cpp:40-54).
std::optional<std::string> field_value(const std::string &header, const std::string &field) {
  size_t key = header.find("'" + field + "'");
  if (key == std::string::npos) key = header.find("\"" + field + "\"");
  if (key == std::string::npos) return std::nullopt;
  const size_t colon = header.find(':', key);
  if (colon == std::string::npos) return std::nullopt;
  return trim_left(header, colon + 1);
}

std::optional<std::string> string_field(const std::string &header, const std::string &field) {
  const auto v = field_value(header, field);
  if (!v || v->empty()) return std::nullopt;
  const char quote = (*v)[0];
  if (quote != '\'' && quote != '"') return std::nullopt;
  const size_t end = v->find(quote, 1);
  if (end == std::string::npos) return std::nullopt;
  return v->substr(1, end - 1);
}

std::optional<bool> bool_field(const std::string &header, const std::string &field) {
  const auto v = field_value(header, field);
  if (!v) return std::nullopt;
  if (v->rfind("False", 0) == 0 || v->rfind("false", 0) == 0) return false;
  if (v->rfind("True", 0) == 0 || v->rfind("true", 0) == 0) return true;
  return std::nullopt;
}

std::string trim(const std::string &s) {
  size_t a = 0, b = s.size();
  while (a < b && std::isspace((unsigned char)s[a])) ++a;
  while (b > a && std::isspace((unsigned char)s[b - 1])) --b;
  return s.substr(a, b - a);
}

// A non-negative base-10 integer, the whole token (StringRef::getAsInteger).
std::optional<int64_t> parse_dim(const std::string &token) {
  if (token.empty()) return std::nullopt;
  size_t i = 0;
  bool neg = false;
  if (token[0] == '+' || token[0] == '-') {
    neg = token[0] == '-';
    i = 1;
  }
  if (i == token.size()) return std::nullopt;
  uint64_t v = 0;
  for (; i < token.size(); ++i) {
    if (token[i] < '0' || token[i] > '9') return std::nullopt;
    const uint64_t d = (uint64_t)(token[i] - '0');
    if (v > ((uint64_t)std::numeric_limits<int64_t>::max() - d) / 10) return std::nullopt;
    v = v * 10 + d;
  }
  if (neg && v != 0) return std::nullopt;  // dim < 0 is rejected
  return (int64_t)v;
}

// parseNpyShapeField (NpyPayload.cpp:86-112): the tuple between the first
// '(' and the first ')' after the key, comma separated, empty tokens skipped.
std::optional<std::vector<int64_t>> shape_field(const std::string &header) {
  const auto v = field_value(header, "shape");
  if (!v) return std::nullopt;
  const size_t open = v->find('('), close = v->find(')');
  if (open == std::string::npos || close == std::string::npos || close < open) return std::nullopt;
  std::string body = v->substr(open + 1, close - open - 1);
  std::vector<int64_t> shape;
  while (!body.empty()) {
    const size_t comma = body.find(',');
    const std::string token = trim(comma == std::string::npos ? body : body.substr(0, comma));
    body = comma == std::string::npos ? std::string() : body.substr(comma + 1);
    if (token.empty()) continue;
    const auto dim = parse_dim(token);
    if (!dim) return std::nullopt;
    shape.push_back(*dim);
  }
  return shape;
}

bool read_file(const std::string &path, std::vector<uint8_t> &bytes) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  f.seekg(0, std::ios::end);
  const std::streamoff size = f.tellg();
  if (size < 0) return false;
  f.seekg(0, std::ios::beg);
  bytes.resize((size_t)size);
  if (size > 0 && !f.read(reinterpret_cast<char *>(bytes.data()), size)) return false;
  return true;
}

// readNpyPayloadMetadata (NpyPayload.cpp:114-175) over the file's bytes;
// `bounded` adds the 1 MiB header limit of readNpyPayloadMetadataFromSource
// (:262-270), which the header-only parse uses.
NpyResult<NpyPayloadHeader> parse_header(const std::vector<uint8_t> &bytes, const std::string &name, bool bounded) {
  NpyResult<NpyPayloadHeader> r;
  if (bytes.size() < 10 || std::memcmp(bytes.data(), "\x93NUMPY", 6) != 0) {
    r.error = "npy payload is missing magic: " + name;
    return r;
  }
  const uint64_t major = bytes[6];
  uint64_t header_len = 0, header_offset = 0;
  if (major == 1) {
    header_offset = 10;
    header_len = (uint64_t)bytes[8] | ((uint64_t)bytes[9] << 8);
  } else if (major == 2) {
    if (bytes.size() < 12) {
      r.error = "truncated npy v2 header: " + name;
      return r;
    }
    header_offset = 12;
    header_len = (uint64_t)bytes[8] | ((uint64_t)bytes[9] << 8) | ((uint64_t)bytes[10] << 16) |
                 ((uint64_t)bytes[11] << 24);
  } else {
    r.error = "unsupported npy payload version: " + name;
    return r;
  }
  if (bounded && (header_len > kMaximumNpyHeaderBytes || header_offset + header_len > bytes.size())) {
    r.error = "npy payload header is truncated or unreasonably large: " + name;
    return r;
  }
  if (header_offset + header_len > bytes.size()) {
    r.error = "truncated npy payload header: " + name;
    return r;
  }
  const std::string header(reinterpret_cast<const char *>(bytes.data()) + header_offset, (size_t)header_len);
  const auto descr = string_field(header, "descr");
  const auto fortran = bool_field(header, "fortran_order");
  const auto shape = shape_field(header);
  if (!descr || !fortran || !shape) {
    r.error = "invalid npy payload header: " + name;
    return r;
  }
  NpyPayloadHeader h;
  h.fileSize = bytes.size();
  h.dataOffset = header_offset + header_len;
  h.descr = *descr;
  h.fortranOrder = *fortran;
  h.shape = *shape;
  r.value = std::move(h);
  return r;
}

}  // namespace

// decodeNpyDescr (NpyPayload.cpp:177-206)
std::optional<std::pair<ProgramElementType, uint64_t>> decodeProgramNpyDescr(const std::string &descr) {
  const bool le = little_endian_host();
  auto is = [&](const char *code) { return descr == std::string("<") + code || (le && descr == std::string("=") + code); };
  using T = ProgramElementType;
  if (is("f4")) return std::make_pair(T::F32, (uint64_t)4);
  if (is("f8")) return std::make_pair(T::F64, (uint64_t)8);
  if (is("f2")) return std::make_pair(T::F16, (uint64_t)2);
  if (descr == "|V2") return std::make_pair(T::BF16, (uint64_t)2);
  if (descr == "|b1") return std::make_pair(T::Bool, (uint64_t)1);
  if (descr == "|i1") return std::make_pair(T::I8, (uint64_t)1);
  if (is("i2")) return std::make_pair(T::I16, (uint64_t)2);
  if (is("i4")) return std::make_pair(T::I32, (uint64_t)4);
  if (is("i8")) return std::make_pair(T::I64, (uint64_t)8);
  return std::nullopt;
}

NpyResult<NpyPayloadHeader> parseNpyPayloadHeader(const std::string &path) {
  std::vector<uint8_t> bytes;
  if (!read_file(path, bytes)) {
    NpyResult<NpyPayloadHeader> r;
    r.error = "failed to read npy payload file: " + path;
    return r;
  }
  return parse_header(bytes, path, true);
}

NpyResult<NpyTensorPayload> loadNpyTensorPayload(const std::string &path) {
  NpyResult<NpyTensorPayload> r;
  std::vector<uint8_t> bytes;
  if (!read_file(path, bytes)) {
    r.error = "failed to read npy payload file: " + path;
    return r;
  }
  auto h = parse_header(bytes, path, false);
  if (!h) {
    r.error = h.error;
    return r;
  }
  if (h.value->fortranOrder) {
    r.error = "npy payload must be row-major: " + path;
    return r;
  }
  const auto decoded = decodeProgramNpyDescr(h.value->descr);
  if (!decoded) {
    r.error = "npy payload has unsupported dtype: " + path;
    return r;
  }
  uint64_t raw = decoded->second;
  for (int64_t dim : h.value->shape) {
    if (dim < 0 || (dim != 0 && raw > std::numeric_limits<uint64_t>::max() / (uint64_t)dim)) {
      r.error = "npy payload byte count is not representable: " + path;
      return r;
    }
    raw *= (uint64_t)dim;
  }
  if (h.value->dataOffset > bytes.size() || raw > bytes.size() - h.value->dataOffset) {
    r.error = "npy tensor payload is truncated: " + path;
    return r;
  }
  NpyTensorPayload p;
  p.dtype = decoded->first;
  p.shape = h.value->shape;
  p.bytes.assign(bytes.begin() + (std::ptrdiff_t)h.value->dataOffset,
                 bytes.begin() + (std::ptrdiff_t)(h.value->dataOffset + raw));
  r.value = std::move(p);
  return r;
}

}  // namespace wafer::model

extern "C" int wafer_npy_load(const char *path, uint32_t *dtype, int64_t *shape, uint32_t max_rank, uint32_t *rank,
                              uint8_t **data, uint64_t *bytes, char *error, size_t error_bytes) {
  auto fail = [&](const std::string &m) {
    if (error && error_bytes) {
      const size_t n = m.size() < error_bytes - 1 ? m.size() : error_bytes - 1;
      std::memcpy(error, m.data(), n);
      error[n] = 0;
    }
    return -1;
  };
  if (!path || !dtype || !rank || !data || !bytes || (max_rank && !shape)) return fail("wafer_npy_load: null argument");
  auto r = wafer::model::loadNpyTensorPayload(path);
  if (!r) return fail(r.error);
  if (r.value->shape.size() > max_rank) return fail("wafer_npy_load: rank exceeds max_rank");
  uint8_t *buf = (uint8_t *)std::malloc(r.value->bytes.empty() ? 1 : r.value->bytes.size());
  if (!buf) return fail("wafer_npy_load: out of memory");
  if (!r.value->bytes.empty()) std::memcpy(buf, r.value->bytes.data(), r.value->bytes.size());
  *dtype = (uint32_t)r.value->dtype;
  *rank = (uint32_t)r.value->shape.size();
  for (size_t i = 0; i < r.value->shape.size(); ++i) shape[i] = r.value->shape[i];
  *data = buf;
  *bytes = r.value->bytes.size();
  return 0;
}

extern "C" void wafer_npy_free(uint8_t *data) { std::free(data); }
