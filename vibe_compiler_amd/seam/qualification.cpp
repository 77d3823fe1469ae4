// qualification.cpp -- evidence records (see qualification.h).
#include "qualification.h"

#include "wafer_hip.h"

#include <dlfcn.h>

#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <sys/stat.h>
#include <unistd.h>

namespace wafer::model {
namespace {

TargetModelKernelError invalid(const std::string &detail) {
  return TargetModelKernelError{TargetModelKernelErrorCode::InvalidCommandField, detail};
}
TargetModelKernelError failure(const std::string &detail) {
  return TargetModelKernelError{TargetModelKernelErrorCode::OneDNNBackendFailure, detail};
}

// ---- SHA-256, FIPS 180-4 section 6.2 -----------------------------------------
constexpr uint32_t K256[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void sha256_block(uint32_t h[8], const uint8_t *p) {
  uint32_t w[64];
  for (int t = 0; t < 16; ++t)
    w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 | p[4 * t + 3];
  for (int t = 16; t < 64; ++t) {
    const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
    const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
    w[t] = w[t - 16] + s0 + w[t - 7] + s1;
  }
  uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
  for (int t = 0; t < 64; ++t) {
    const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K256[t] + w[t];
    const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
    hh = g;
    g = f;
    f = e;
    e = d + t1;
    d = c;
    c = b;
    b = a;
    a = t1 + t2;
  }
  h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}

std::string sha256_hex(const uint8_t *data, size_t n) {
  uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
  size_t i = 0;
  for (; i + 64 <= n; i += 64) sha256_block(h, data + i);
  uint8_t tail[128] = {};
  const size_t rem = n - i;
  std::memcpy(tail, data + i, rem);
  tail[rem] = 0x80;
  const size_t blocks = rem + 9 <= 64 ? 1 : 2;
  const uint64_t bits = (uint64_t)n * 8;
  for (int b = 0; b < 8; ++b) tail[blocks * 64 - 1 - b] = (uint8_t)(bits >> (8 * b));
  for (size_t b = 0; b < blocks; ++b) sha256_block(h, tail + 64 * b);
  static const char *hex = "0123456789abcdef";
  std::string out;
  out.reserve(64);
  for (int w = 0; w < 8; ++w)
    for (int s = 28; s >= 0; s -= 4) out.push_back(hex[(h[w] >> s) & 15]);
  return out;
}

bool is_digest(const std::string &v) {
  if (v.size() != 71 || v.compare(0, 7, "sha256:") != 0) return false;
  for (size_t i = 7; i < v.size(); ++i)
    if (!((v[i] >= '0' && v[i] <= '9') || (v[i] >= 'a' && v[i] <= 'f'))) return false;
  return true;
}

// ---- JSON text -------------------------------------------------------------------
void print_string(std::string &out, const std::string &s) {
  out.push_back('"');
  for (unsigned char c : s) {
    if (c == '"' || c == '\\') {
      out.push_back('\\');
      out.push_back((char)c);
    } else if (c < 0x20) {
      const char *shortEsc = c == '\b' ? "\\b" : c == '\f' ? "\\f" : c == '\n' ? "\\n" : c == '\r' ? "\\r" : c == '\t' ? "\\t" : nullptr;
      if (shortEsc) {
        out += shortEsc;
      } else {
        char buf[8];
        std::snprintf(buf, sizeof buf, "\\u%04x", c);
        out += buf;
      }
    } else {
      out.push_back((char)c);
    }
  }
  out.push_back('"');
}

void print_value(std::string &out, const Json &v) {
  switch (v.kind()) {
  case Json::Kind::Null: out += "null"; break;
  case Json::Kind::Bool: out += v.asBool() ? "true" : "false"; break;
  case Json::Kind::Int: out += std::to_string(v.asInt()); break;
  case Json::Kind::String: print_string(out, v.asString()); break;
  case Json::Kind::Array: {
    out.push_back('[');
    bool first = true;
    for (const Json &x : v.items()) {
      if (!first) out.push_back(',');
      first = false;
      print_value(out, x);
    }
    out.push_back(']');
    break;
  }
  case Json::Kind::Object: {
    out.push_back('{');
    bool first = true;
    for (const auto &kv : v.fields()) {  // std::map: keys in byte order
      if (!first) out.push_back(',');
      first = false;
      print_string(out, kv.first);
      out.push_back(':');
      print_value(out, kv.second);
    }
    out.push_back('}');
    break;
  }
  }
}

struct Parser {
  const std::string &t;
  size_t p = 0;
  std::string error;
  void ws() {
    while (p < t.size() && (t[p] == ' ' || t[p] == '\t' || t[p] == '\n' || t[p] == '\r')) ++p;
  }
  bool fail(const std::string &m) {
    if (error.empty()) error = m + " at offset " + std::to_string(p);
    return false;
  }
  bool lit(const char *w) {
    const size_t n = std::strlen(w);
    if (t.compare(p, n, w) != 0) return false;
    p += n;
    return true;
  }
  bool str(std::string &out) {
    if (p >= t.size() || t[p] != '"') return fail("expected a string");
    ++p;
    while (p < t.size() && t[p] != '"') {
      char c = t[p++];
      if ((unsigned char)c < 0x20) return fail("control character in a string");
      if (c == '\\') {
        if (p >= t.size()) return fail("truncated escape");
        const char e = t[p++];
        if (e == '"' || e == '\\' || e == '/') out.push_back(e);
        else if (e == 'n') out.push_back('\n');
        else if (e == 't') out.push_back('\t');
        else if (e == 'r') out.push_back('\r');
        else if (e == 'b') out.push_back('\b');
        else if (e == 'f') out.push_back('\f');
        else if (e == 'u') {
          if (p + 4 > t.size()) return fail("truncated escape");
          unsigned v = 0;
          for (int i = 0; i < 4; ++i) {
            const char h = t[p++];
            v <<= 4;
            if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
            else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
            else return fail("bad escape");
          }
          if (v >= 0x80) return fail("non-ASCII escape");
          out.push_back((char)v);
        } else {
          return fail("bad escape");
        }
      } else {
        out.push_back(c);
      }
    }
    if (p >= t.size()) return fail("unterminated string");
    ++p;
    return true;
  }
  bool value(Json &out, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= t.size()) return fail("unexpected end");
    const char c = t[p];
    if (c == '{') {
      ++p;
      std::map<std::string, Json> fields;
      ws();
      if (p < t.size() && t[p] == '}') {
        ++p;
        out = Json::object(std::move(fields));
        return true;
      }
      while (true) {
        ws();
        std::string key;
        if (!str(key)) return false;
        if (fields.count(key)) return fail("duplicate key " + key);
        ws();
        if (p >= t.size() || t[p] != ':') return fail("expected ':'");
        ++p;
        Json v;
        if (!value(v, depth + 1)) return false;
        fields.emplace(std::move(key), std::move(v));
        ws();
        if (p < t.size() && t[p] == ',') { ++p; continue; }
        if (p < t.size() && t[p] == '}') { ++p; break; }
        return fail("expected ',' or '}'");
      }
      out = Json::object(std::move(fields));
      return true;
    }
    if (c == '[') {
      ++p;
      std::vector<Json> items;
      ws();
      if (p < t.size() && t[p] == ']') {
        ++p;
        out = Json::array(std::move(items));
        return true;
      }
      while (true) {
        Json v;
        if (!value(v, depth + 1)) return false;
        items.push_back(std::move(v));
        ws();
        if (p < t.size() && t[p] == ',') { ++p; continue; }
        if (p < t.size() && t[p] == ']') { ++p; break; }
        return fail("expected ',' or ']'");
      }
      out = Json::array(std::move(items));
      return true;
    }
    if (c == '"') {
      std::string s;
      if (!str(s)) return false;
      out = Json::string(std::move(s));
      return true;
    }
    if (lit("true")) { out = Json::boolean(true); return true; }
    if (lit("false")) { out = Json::boolean(false); return true; }
    if (lit("null")) { out = Json(); return true; }
    if (c == '-' || (c >= '0' && c <= '9')) {
      const size_t start = p;
      if (t[p] == '-') ++p;
      while (p < t.size() && t[p] >= '0' && t[p] <= '9') ++p;
      if (p < t.size() && (t[p] == '.' || t[p] == 'e' || t[p] == 'E')) return fail("only integers are accepted");
      errno = 0;
      char *end = nullptr;
      const std::string digits = t.substr(start, p - start);
      const long long v = std::strtoll(digits.c_str(), &end, 10);
      if (errno || !end || *end) return fail("integer out of range");
      out = Json::integer(v);
      return true;
    }
    return fail("unexpected character");
  }
};

// ---- records -----------------------------------------------------------------------
const char *kRecordSchema = "wafer-hip-qualification-record";
const char *kEnvironmentSchema = "wafer-hip-execution-environment";
const char *kSpecSchema = "wafer-hip-qualification-spec";

const char *format_name(LogicalFormat f) {
  switch (f) {
  case LogicalFormat::F16: return "f16";
  case LogicalFormat::BF16: return "bf16";
  case LogicalFormat::F32: return "f32";
  default: return "unsupported";
  }
}
std::optional<LogicalFormat> format_from(const std::string &s) {
  if (s == "f16") return LogicalFormat::F16;
  if (s == "bf16") return LogicalFormat::BF16;
  if (s == "f32") return LogicalFormat::F32;
  return std::nullopt;
}

Json descriptor_json(const PhysicalTensorDescriptor &d) {
  std::vector<Json> shape;
  for (uint64_t x : d.getShape()) shape.push_back(Json::integer((int64_t)x));
  return Json::object({{"format", Json::integer((int64_t)d.getFormat())},
                       {"layout", Json::integer((int64_t)d.getLayout())},
                       {"shape", Json::array(std::move(shape))}});
}

// the library file behind the C ABI, for the environment's library digest
std::string library_digest() {
  Dl_info info;
  if (!dladdr((const void *)&wafer_hip_implementation, &info) || !info.dli_fname) return "unknown";
  std::ifstream f(info.dli_fname, std::ios::binary);
  if (!f) return "unknown";
  std::ostringstream ss;
  ss << f.rdbuf();
  return sha256Digest(ss.str());
}

// splitmix64 (Steele, Lea and Flood, "Fast splittable pseudorandom number
// generators", OOPSLA 2014): the case's value stream
uint64_t splitmix64(uint64_t &state) {
  uint64_t z = (state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// v in {-8..8}/8 as storage bits of `f` (exact in F16, BF16 and F32)
uint32_t dyadic_bits(LogicalFormat f, int v) {
  const float x = (float)v / 8.0f;
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if (f == LogicalFormat::F32) return u;
  if (f == LogicalFormat::BF16) return u >> 16;  // exact: at most 4 significant bits
  // F16 of a value with at most 4 significant bits and exponent in [-3, 0]
  if (v == 0) return (uint32_t)(u >> 16) & 0x8000u;
  const uint32_t sign = (u >> 16) & 0x8000u;
  const int e = (int)((u >> 23) & 0xff) - 127;
  const uint32_t frac = (u >> 13) & 0x3ffu;
  return sign | (uint32_t)(e + 15) << 10 | frac;
}

int storage_bytes_of(LogicalFormat f) { return f == LogicalFormat::F32 ? 4 : 2; }

// logical row-major values -> physical image over a template, on the GPU codec
Expected<std::vector<uint8_t>> pack_physical(wafer_hip_context *ctx, const PhysicalTensorDescriptor &d,
                                             const std::vector<uint8_t> &logical, uint8_t fill) {
  Expected<uint64_t> bytes = d.getStorageBytes();
  if (!bytes) return bytes.error();
  std::vector<uint8_t> out(*bytes, fill);
  void *dl = nullptr, *dp = nullptr;
  auto release = [&] {
    if (dl) wafer_hip_buffer_free(ctx, dl);
    if (dp) wafer_hip_buffer_free(ctx, dp);
  };
  std::vector<int64_t> shape(d.getShape().begin(), d.getShape().end());
  int st = wafer_hip_buffer_alloc(ctx, logical.size(), &dl);
  if (!st) st = wafer_hip_buffer_alloc(ctx, out.size(), &dp);
  if (!st) st = wafer_hip_copy_to_device(ctx, dl, logical.data(), logical.size());
  if (!st) st = wafer_hip_copy_to_device(ctx, dp, out.data(), out.size());
  if (!st)
    st = wafer_hip_pack(ctx, (uint32_t)d.getFormat(), (uint32_t)d.getLayout(), shape.data(), (uint32_t)shape.size(),
                        dl, dp, (int64_t)out.size());
  if (!st) st = wafer_hip_copy_to_host(ctx, out.data(), dp, out.size());
  release();
  if (st) return failure(std::string("qualification case packing: ") + wafer_hip_last_error());
  return out;
}

std::string payload_digest(const std::vector<TargetModelNumericTensor> &inputs) {
  std::string all;
  for (const auto &t : inputs) {
    const uint64_t n = t.storage.size();
    for (int b = 0; b < 8; ++b) all.push_back((char)(n >> (8 * b)));  // length-prefixed
    all.append(reinterpret_cast<const char *>(t.storage.data()), t.storage.size());
  }
  return sha256Digest(all);
}

Json operation_json(const FormalGemmOperation &op) {
  return Json::object({{"lhs", descriptor_json(op.lhs)},
                       {"rhs", descriptor_json(op.rhs)},
                       {"destination", descriptor_json(op.destination)},
                       {"m", Json::integer(op.m)},
                       {"k", Json::integer(op.k)},
                       {"n", Json::integer(op.n)},
                       {"batch_count", Json::integer(op.batchCount)},
                       {"lhs_orientation", Json::integer((int64_t)op.lhsOrientation)},
                       {"rhs_orientation", Json::integer((int64_t)op.rhsOrientation)},
                       {"psum", op.psum ? descriptor_json(*op.psum) : Json()}});
}

Expected<std::string> require_string(const Json &o, const std::string &key) {
  const Json *v = o.find(key);
  if (!v || v->kind() != Json::Kind::String) return invalid("qualification record field " + key + " is not a string");
  return v->asString();
}
Expected<std::string> require_digest(const Json &o, const std::string &key) {
  Expected<std::string> s = require_string(o, key);
  if (!s) return s;
  if (!is_digest(*s)) return invalid("qualification record field " + key + " is not lowercase SHA-256");
  return s;
}
Expected<int64_t> require_int(const Json &o, const std::string &key) {
  const Json *v = o.find(key);
  if (!v || v->kind() != Json::Kind::Int) return invalid("qualification field " + key + " is not an integer");
  return v->asInt();
}
bool exact_fields(const Json &o, std::initializer_list<const char *> keys) {
  if (o.kind() != Json::Kind::Object || o.fields().size() != keys.size()) return false;
  for (const char *k : keys)
    if (!o.find(k)) return false;
  return true;
}

}  // namespace

// ---- public -------------------------------------------------------------------------
std::string sha256Digest(const void *data, size_t bytes) {
  return "sha256:" + sha256_hex(static_cast<const uint8_t *>(data), bytes);
}
std::string sha256Digest(const std::string &text) { return sha256Digest(text.data(), text.size()); }

Json Json::boolean(bool v) { Json j; j.k = Kind::Bool; j.b = v; return j; }
Json Json::integer(int64_t v) { Json j; j.k = Kind::Int; j.i = v; return j; }
Json Json::string(std::string v) { Json j; j.k = Kind::String; j.s = std::move(v); return j; }
Json Json::array(std::vector<Json> v) { Json j; j.k = Kind::Array; j.a = std::move(v); return j; }
Json Json::object(std::map<std::string, Json> v) { Json j; j.k = Kind::Object; j.o = std::move(v); return j; }
const Json *Json::find(const std::string &key) const {
  auto it = o.find(key);
  return it == o.end() ? nullptr : &it->second;
}

std::string canonicalJson(const Json &value) {
  std::string out;
  print_value(out, value);
  out.push_back('\n');
  return out;
}

Expected<Json> parseJson(const std::string &text) {
  Parser ps{text, 0, {}};
  Json v;
  if (!ps.value(v, 0)) return invalid("invalid JSON: " + ps.error);
  ps.ws();
  if (ps.p != text.size()) return invalid("invalid JSON: trailing characters");
  return v;
}

Expected<HipExecutionEnvironment> captureHipExecutionEnvironment(const HipTargetModelBackend &backend) {
  wafer_hip_environment_info info;
  if (wafer_hip_environment(backend.context(), &info))
    return failure(std::string("environment: ") + wafer_hip_last_error());
  HipExecutionEnvironment env;
  env.record = Json::object({{"schema", Json::string(kEnvironmentSchema)},
                             {"backend_name", Json::string("wafer-hip")},
                             {"implementation", Json::string(wafer_hip_implementation())},
                             {"gcn_arch_name", Json::string(info.gcn_arch_name)},
                             {"device_name", Json::string(info.device_name)},
                             {"compute_units", Json::integer(info.compute_units)},
                             {"warp_size", Json::integer(info.warp_size)},
                             {"hip_runtime_version", Json::integer(info.hip_runtime_version)},
                             {"driver_version", Json::integer(info.driver_version)},
                             {"global_memory_bytes", Json::integer((int64_t)info.global_memory_bytes)},
                             {"lds_bytes_per_block", Json::integer((int64_t)info.lds_bytes_per_block)},
                             {"library_digest", Json::string(library_digest())}});
  env.digest = sha256Digest(canonicalJson(env.record));
  return env;
}

Expected<HipQualificationSpec> HipQualificationSpec::create(LogicalFormat input, LogicalFormat output, uint16_t m,
                                                            uint16_t k, uint16_t n, uint16_t batch,
                                                            TargetGemmOrientation rhsOrientation, uint64_t seed) {
  if (!format_from(format_name(input)))
    return invalid("qualification spec input format must be f16, bf16 or f32");
  if (!(output == input || ((input == LogicalFormat::F16 || input == LogicalFormat::BF16) && output == LogicalFormat::F32)))
    return invalid("qualification spec has an unsupported input/output format pair");
  if (!m || !k || !n || !batch) return invalid("qualification spec extents must be positive");
  if (seed > (uint64_t)INT64_MAX) return invalid("qualification spec seed must fit in int64");
  HipQualificationSpec s;
  s.input = input;
  s.output = output;
  s.m = m;
  s.k = k;
  s.n = n;
  s.batch = batch;
  s.rhsOrientation = rhsOrientation;
  s.seed = seed;
  return s;
}

Json HipQualificationSpec::toJson() const {
  return Json::object({{"schema", Json::string(kSpecSchema)},
                       {"input_format", Json::string(format_name(input))},
                       {"output_format", Json::string(format_name(output))},
                       {"m", Json::integer(m)},
                       {"k", Json::integer(k)},
                       {"n", Json::integer(n)},
                       {"batch_count", Json::integer(batch)},
                       {"rhs_orientation", Json::integer((int64_t)rhsOrientation)},
                       {"seed", Json::integer((int64_t)seed)}});
}

Expected<HipQualificationSpec> HipQualificationSpec::fromJson(const Json &j) {
  if (!exact_fields(j, {"schema", "input_format", "output_format", "m", "k", "n", "batch_count", "rhs_orientation",
                        "seed"}))
    return invalid("qualification spec has missing or unknown fields");
  auto schema = require_string(j, "schema");
  if (!schema) return schema.error();
  if (*schema != kSpecSchema) return invalid("qualification spec schema mismatch");
  auto fi = require_string(j, "input_format"), fo = require_string(j, "output_format");
  if (!fi) return fi.error();
  if (!fo) return fo.error();
  auto in = format_from(*fi), out = format_from(*fo);
  if (!in || !out) return invalid("qualification spec format is unknown");
  int64_t v[6];
  const char *keys[6] = {"m", "k", "n", "batch_count", "rhs_orientation", "seed"};
  for (int i = 0; i < 6; ++i) {
    auto x = require_int(j, keys[i]);
    if (!x) return x.error();
    v[i] = *x;
  }
  for (int i = 0; i < 4; ++i)
    if (v[i] < 1 || v[i] > 65535) return invalid("qualification spec extent out of range");
  if (v[4] != 0 && v[4] != 1) return invalid("qualification spec orientation is not a closed enum value");
  if (v[5] < 0) return invalid("qualification spec seed is negative");
  return create(*in, *out, (uint16_t)v[0], (uint16_t)v[1], (uint16_t)v[2], (uint16_t)v[3],
                (TargetGemmOrientation)v[4], (uint64_t)v[5]);
}

Expected<TargetModelGemmRequest> materializeHipQualificationCase(const HipTargetModelBackend &backend,
                                                                 const HipQualificationSpec &spec) {
  const bool batched = spec.batch > 1;
  const PhysicalTensorLayout L = batched ? PhysicalTensorLayout::NCx : PhysicalTensorLayout::Cx;
  auto shp = [&](uint64_t a, uint64_t b) {
    return batched ? std::vector<uint64_t>{spec.batch, a, b} : std::vector<uint64_t>{a, b};
  };
  const bool rt = spec.rhsOrientation == TargetGemmOrientation::Transpose;
  auto lhs = PhysicalTensorDescriptor::create(spec.input, L, shp(spec.m, spec.k));
  auto rhs = PhysicalTensorDescriptor::create(spec.input, L, rt ? shp(spec.n, spec.k) : shp(spec.k, spec.n));
  auto dst = PhysicalTensorDescriptor::create(spec.output, L, shp(spec.m, spec.n));
  if (!lhs) return lhs.error();
  if (!rhs) return rhs.error();
  if (!dst) return dst.error();
  uint64_t state = spec.seed;
  auto values = [&](const PhysicalTensorDescriptor &d) {
    const int eb = storage_bytes_of(d.getFormat());
    std::vector<uint8_t> out(d.getElementCount() * eb);
    for (uint64_t i = 0; i < d.getElementCount(); ++i) {
      const int v = (int)(splitmix64(state) % 17) - 8;
      const uint32_t bits = dyadic_bits(d.getFormat(), v);
      std::memcpy(&out[i * eb], &bits, eb);
    }
    return out;
  };
  auto a = pack_physical(backend.context(), *lhs, values(*lhs), 0);
  if (!a) return a.error();
  auto b = pack_physical(backend.context(), *rhs, values(*rhs), 0);
  if (!b) return b.error();
  auto bytes = dst->getStorageBytes();
  if (!bytes) return bytes.error();
  auto axes = getCanonicalFormalGemmGeometry(lhs->getShape().size());
  if (!axes) return axes.error();
  return TargetModelGemmRequest{
      FormalGemmOperation{*lhs, *rhs, *dst, spec.m, spec.k, spec.n, spec.batch, *axes, TargetGemmOrientation::Normal,
                          spec.rhsOrientation, std::nullopt},
      TargetModelNumericOperands{{{*lhs, std::move(*a)}, {*rhs, std::move(*b)}},
                                 {*dst, std::vector<uint8_t>(*bytes, 0xA5)}}};
}

std::string hipProblemDigest(const TargetModelGemmRequest &request) {
  Json j = Json::object({{"operation", operation_json(request.operation)},
                         {"input_payload_digest", Json::string(payload_digest(request.tensors.inputs))},
                         {"destination_template_digest",
                          Json::string(sha256Digest(request.tensors.destinationTemplate.storage.data(),
                                                    request.tensors.destinationTemplate.storage.size()))}});
  return sha256Digest(canonicalJson(j));
}

Expected<std::string> validateHipBackend(const HipTargetModelBackend &backend, const HipQualificationSpec &spec,
                                         const std::vector<uint8_t> &formalDestination, const std::string &outputPath) {
  struct stat sb;
  if (::stat(outputPath.c_str(), &sb) == 0) return invalid("qualification output exists and is never replaced: " + outputPath);
  auto env = captureHipExecutionEnvironment(backend);
  if (!env) return env.error();
  auto request = materializeHipQualificationCase(backend, spec);
  if (!request) return request.error();
  auto result = backend.tryExecute(*request);
  if (!result) return result.error();
  if (!result->has_value()) return failure("qualification case was not handled by the backend");
  const std::vector<uint8_t> &got = (*result)->destination.storage;
  if (got != formalDestination) {
    size_t first = 0;
    while (first < got.size() && first < formalDestination.size() && got[first] == formalDestination[first]) ++first;
    return failure("backend output differs from the formal lane at byte " + std::to_string(first));
  }
  const Json specJson = spec.toJson();
  Json record = Json::object(
      {{"schema", Json::string(kRecordSchema)},
       {"qualification_kind", Json::string("bit-exact")},
       {"comparator", Json::string("byte-exact physical destination against the formal lane")},
       {"spec", specJson},
       {"spec_digest", Json::string(sha256Digest(canonicalJson(specJson)))},
       {"environment", env->record},
       {"environment_digest", Json::string(env->digest)},
       {"problem_digest", Json::string(hipProblemDigest(*request))},
       {"input_payload_digest", Json::string(payload_digest(request->tensors.inputs))},
       {"destination_template_digest",
        Json::string(sha256Digest(request->tensors.destinationTemplate.storage.data(),
                                  request->tensors.destinationTemplate.storage.size()))},
       {"expected_backend_output_digest", Json::string(sha256Digest(got.data(), got.size()))},
       {"implementation", Json::string((*result)->evidence.implementation)}});
  const std::string text = canonicalJson(record);
  // create atomically: write a sibling, then link it into place (fails if the
  // target appeared meanwhile)
  const std::string tmp = outputPath + ".partial";
  {
    std::ofstream f(tmp, std::ios::binary | std::ios::trunc);
    if (!f || !f.write(text.data(), (std::streamsize)text.size())) return failure("cannot write " + tmp);
  }
  if (::link(tmp.c_str(), outputPath.c_str()) != 0) {
    std::remove(tmp.c_str());
    return failure("cannot create " + outputPath);
  }
  std::remove(tmp.c_str());
  return sha256Digest(text);
}

Expected<VerifiedHipQualificationRecord> loadVerifiedHipQualificationRecord(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return invalid("cannot read qualification record " + path);
  std::ostringstream ss;
  ss << f.rdbuf();
  const std::string text = ss.str();
  auto parsed = parseJson(text);
  if (!parsed) return parsed.error();
  if (canonicalJson(*parsed) != text) return invalid("qualification record is not in canonical form: " + path);
  const Json &r = *parsed;
  if (!exact_fields(r, {"schema", "qualification_kind", "comparator", "spec", "spec_digest", "environment",
                        "environment_digest", "problem_digest", "input_payload_digest",
                        "destination_template_digest", "expected_backend_output_digest", "implementation"}))
    return invalid("qualification record has missing or unknown fields");
  auto schema = require_string(r, "schema");
  if (!schema) return schema.error();
  if (*schema != kRecordSchema) return invalid("qualification record schema mismatch");
  auto kind = require_string(r, "qualification_kind");
  if (!kind) return kind.error();
  if (*kind != "bit-exact") return invalid("unknown qualification kind " + *kind);
  auto spec = HipQualificationSpec::fromJson(*r.find("spec"));
  if (!spec) return spec.error();
  VerifiedHipQualificationRecord v;
  const char *digests[] = {"spec_digest", "environment_digest", "problem_digest", "input_payload_digest",
                           "destination_template_digest", "expected_backend_output_digest"};
  std::string got[6];
  for (int i = 0; i < 6; ++i) {
    auto d = require_digest(r, digests[i]);
    if (!d) return d.error();
    got[i] = *d;
  }
  if (got[0] != spec->digest()) return invalid("qualification record spec digest does not match its spec");
  const Json *env = r.find("environment");
  if (env->kind() != Json::Kind::Object) return invalid("qualification record environment is not an object");
  auto env_schema = require_string(*env, "schema");
  if (!env_schema || *env_schema != kEnvironmentSchema) return invalid("qualification record environment schema mismatch");
  if (got[1] != sha256Digest(canonicalJson(*env)))
    return invalid("qualification record environment digest does not match its environment");
  auto impl = require_string(r, "implementation");
  if (!impl) return impl.error();
  v.recordDigest = sha256Digest(text);
  v.specDigest = got[0];
  v.environmentDigest = got[1];
  v.problemDigest = got[2];
  v.expectedOutputDigest = got[5];
  v.implementation = *impl;
  return v;
}

Expected<QualifiedHipExecution> VerifiedHipQualificationRecord::qualifyExecution(
    const HipExecutionEnvironment &environment, const TargetModelGemmRequest &request) const {
  if (environment.digest != environmentDigest)
    return invalid("qualification record environment does not match the execution environment");
  if (hipProblemDigest(request) != problemDigest)
    return invalid("qualification record problem does not match the requested operation and payload");
  return QualifiedHipExecution{recordDigest, expectedOutputDigest, implementation};
}

Expected<TargetModelOneDNNResult> executeQualifiedHip(const HipTargetModelBackend &backend,
                                                      const QualifiedHipExecution &qualified,
                                                      const TargetModelGemmRequest &request) {
  auto result = backend.tryExecute(request);
  if (!result) return result.error();
  if (!result->has_value()) return failure("qualified execution was not handled by the backend");
  TargetModelOneDNNResult out = std::move(**result);
  if (sha256Digest(out.destination.storage.data(), out.destination.storage.size()) != qualified.expectedOutputDigest)
    return failure("qualified execution output does not match the recorded output digest");
  out.evidence.evidenceKind = TargetModelOneDNNEvidenceKind::ExactQualificationRecord;
  out.evidence.evidenceDigest = qualified.recordDigest;
  return out;
}

}  // namespace wafer::model

extern "C" void wafer_sha256_digest(const void *data, size_t bytes, char out[72]) {
  const std::string d = wafer::model::sha256Digest(data, bytes);
  std::memcpy(out, d.c_str(), 72);
}

extern "C" int wafer_canonical_json(const char *text, char *out, size_t out_bytes) {
  auto parsed = wafer::model::parseJson(text ? text : "");
  const std::string result = parsed ? wafer::model::canonicalJson(*parsed) : parsed.error().detail;
  if (out && out_bytes) {
    const size_t n = result.size() < out_bytes - 1 ? result.size() : out_bytes - 1;
    std::memcpy(out, result.data(), n);
    out[n] = 0;
  }
  return parsed ? 0 : -1;
}
