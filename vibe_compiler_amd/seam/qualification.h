// qualification.h -- qualified-execution evidence records for the gfx950
// backend: the analogue of the reference's oneDNN qualification
// (include/Wafer/Simulator/OneDNN/OneDNNQualification.h:19-229,
// lib/Wafer/Simulator/OneDNN/OneDNNQualification*.cpp).
//
// A record binds one deterministic GEMM case (the spec), the execution
// environment it was validated on (device, runtime, driver, the digest of
// the backend library), the exact problem (operation, input payloads,
// destination template) and the destination bytes the formal lane produces
// for it.  It is written once by the validation stage, after the backend's
// output has been compared byte for byte with the formal lane's, as
// canonical JSON (keys sorted, compact, one trailing newline) whose SHA-256
// is the record digest.  At run time a verified record qualifies an
// execution only for the same environment digest and problem digest, and
// the executed output must hash to the recorded digest; the evidence then
// names the record (TargetModelOneDNNEvidenceKind::ExactQualificationRecord).
//
// Differences from the oneDNN flow, on purpose: the gfx950 GEMM is the
// formal order itself (bit-exact by construction and by test), so there is
// no calibration / frozen tolerance policy, only the "bit-exact" kind; and
// the formal lane's output is supplied by the caller of the validation stage
// (this library has no CPU lane).
#pragma once

#include "target_model_hip_backend.h"

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace wafer::model {

// SHA-256 (FIPS 180-4) as "sha256:" + 64 lowercase hex digits, the digest
// spelling of the reference's records.
std::string sha256Digest(const void *data, size_t bytes);
std::string sha256Digest(const std::string &text);

// A JSON value restricted to what the records hold: null, bool, int64,
// string, array, object.
class Json {
public:
  enum class Kind : uint8_t { Null, Bool, Int, String, Array, Object };
  Json() = default;
  static Json boolean(bool v);
  static Json integer(int64_t v);
  static Json string(std::string v);
  static Json array(std::vector<Json> v = {});
  static Json object(std::map<std::string, Json> v = {});
  Kind kind() const { return k; }
  bool asBool() const { return b; }
  int64_t asInt() const { return i; }
  const std::string &asString() const { return s; }
  const std::vector<Json> &items() const { return a; }
  const std::map<std::string, Json> &fields() const { return o; }
  Json &operator[](const std::string &key) { return o[key]; }
  const Json *find(const std::string &key) const;

private:
  Kind k = Kind::Null;
  bool b = false;
  int64_t i = 0;
  std::string s;
  std::vector<Json> a;
  std::map<std::string, Json> o;
};

// Keys sorted, no whitespace, one trailing newline (printCanonicalJSON,
// OneDNNQualification.cpp:51-80).
std::string canonicalJson(const Json &value);
Expected<Json> parseJson(const std::string &text);

struct HipExecutionEnvironment {
  Json record;          // the environment fields
  std::string digest;   // sha256 of canonicalJson(record)
};
Expected<HipExecutionEnvironment> captureHipExecutionEnvironment(const HipTargetModelBackend &backend);

// The deterministic case: operand formats, GEMM extents, rhs orientation,
// seed.  Operands are Cx (NCx when batched), values small dyadic rationals
// drawn from the seed, exactly representable in every float format.
class HipQualificationSpec {
public:
  static Expected<HipQualificationSpec> create(LogicalFormat input, LogicalFormat output, uint16_t m, uint16_t k,
                                               uint16_t n, uint16_t batch, TargetGemmOrientation rhsOrientation,
                                               uint64_t seed);
  static Expected<HipQualificationSpec> fromJson(const Json &json);
  Json toJson() const;
  std::string digest() const { return sha256Digest(canonicalJson(toJson())); }
  LogicalFormat input, output;
  uint16_t m, k, n, batch;
  TargetGemmOrientation rhsOrientation;
  uint64_t seed;

private:
  HipQualificationSpec() = default;
};

// The operation and physical payloads of a spec (lhs, rhs, destination
// template filled with 0xA5).
Expected<TargetModelGemmRequest> materializeHipQualificationCase(const HipTargetModelBackend &backend,
                                                                 const HipQualificationSpec &spec);

// sha256 over the canonical JSON of the operation and the digests of the
// input payloads and the destination template.
std::string hipProblemDigest(const TargetModelGemmRequest &request);

// The validation stage: run the spec's case on the backend, require its
// destination bytes to equal `formalDestination` (the formal lane's packed
// output for the same case) and write the record to `outputPath` (a new
// file; an existing one is never replaced).  Returns the record digest.
Expected<std::string> validateHipBackend(const HipTargetModelBackend &backend, const HipQualificationSpec &spec,
                                         const std::vector<uint8_t> &formalDestination, const std::string &outputPath);

struct QualifiedHipExecution {
  std::string recordDigest;
  std::string expectedOutputDigest;
  std::string implementation;
};

class VerifiedHipQualificationRecord {
public:
  const std::string &getRecordDigest() const { return recordDigest; }
  const std::string &getSpecDigest() const { return specDigest; }
  const std::string &getEnvironmentDigest() const { return environmentDigest; }
  const std::string &getProblemDigest() const { return problemDigest; }
  const std::string &getImplementation() const { return implementation; }
  // Qualifies an execution of exactly the recorded problem on exactly the
  // recorded environment.
  Expected<QualifiedHipExecution> qualifyExecution(const HipExecutionEnvironment &environment,
                                                   const TargetModelGemmRequest &request) const;

private:
  friend Expected<VerifiedHipQualificationRecord> loadVerifiedHipQualificationRecord(const std::string &path);
  VerifiedHipQualificationRecord() = default;
  std::string recordDigest, specDigest, environmentDigest, problemDigest, expectedOutputDigest, implementation;
};

// Reads a record: canonical form, exactly the known fields, well-formed
// digests, spec and environment digests that match their embedded objects.
Expected<VerifiedHipQualificationRecord> loadVerifiedHipQualificationRecord(const std::string &path);

// Runs a qualified execution; its output must hash to the recorded digest.
// Evidence: ExactQualificationRecord with the record digest.
Expected<TargetModelOneDNNResult> executeQualifiedHip(const HipTargetModelBackend &backend,
                                                      const QualifiedHipExecution &qualified,
                                                      const TargetModelGemmRequest &request);

}  // namespace wafer::model

// C export for non-C++ callers and tests: the SHA-256 digest text of a byte
// range (72 bytes with the terminator).
extern "C" void wafer_sha256_digest(const void *data, size_t bytes, char out[72]);
// The canonical form of a JSON text (0), or the parse error (-1), in `out`.
extern "C" int wafer_canonical_json(const char *text, char *out, size_t out_bytes);
