// qualify_check.cpp -- the qualification-record flow end to end on the GPU:
// for each spec, materialise the case, compute the formal lane's packed
// output with the CPU oracle (test infrastructure), run the validation stage
// (which writes the record), load and verify the record, qualify and run
// the same problem (evidence names the record), and check that every
// tampering is refused: a non-canonical or edited record, another payload,
// another environment, an output path that already exists.
//
// Usage: qualify_check <empty directory>.  Exit 0 when every check passes.
#include "qualification.h"

extern "C" {
#include "wafer_oracle.h"
}

#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>

using namespace wafer::model;

namespace {

int failures = 0;
void check(bool ok, const std::string &what) {
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
  std::fflush(stdout);
  if (!ok) ++failures;
}

size_t eb(LogicalFormat f) { return f == LogicalFormat::F32 ? 4 : 2; }

std::vector<int64_t> s64(const PhysicalTensorDescriptor &d) {
  return std::vector<int64_t>(d.getShape().begin(), d.getShape().end());
}

std::vector<uint8_t> unpack(const TargetModelNumericTensor &t) {
  std::vector<uint8_t> logical(t.key.getElementCount() * eb(t.key.getFormat()));
  const auto s = s64(t.key);
  oracle_unpack((int)t.key.getFormat(), (int)t.key.getLayout(), s.data(), (int)s.size(), t.storage.data(),
                (int64_t)t.storage.size(), logical.data());
  return logical;
}

// the formal lane's packed destination for a materialised case
std::vector<uint8_t> formal_destination(const TargetModelGemmRequest &r) {
  const FormalGemmOperation &op = r.operation;
  const auto a = unpack(r.tensors.inputs[0]), b = unpack(r.tensors.inputs[1]);
  std::vector<uint8_t> y(op.destination.getElementCount() * eb(op.destination.getFormat()));
  oracle_gemm_formal((int)op.lhs.getFormat(), (int)op.destination.getFormat(), a.data(), b.data(), nullptr, y.data(),
                     op.m, op.k, op.n, op.batchCount, 0, op.rhsOrientation == TargetGemmOrientation::Transpose, 4);
  std::vector<uint8_t> out = r.tensors.destinationTemplate.storage;
  const auto s = s64(op.destination);
  oracle_pack((int)op.destination.getFormat(), (int)op.destination.getLayout(), s.data(), (int)s.size(), y.data(),
              out.data(), (int64_t)out.size());
  return out;
}

std::string slurp(const std::string &p) {
  std::ifstream f(p, std::ios::binary);
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}
void spit(const std::string &p, const std::string &text) {
  std::ofstream f(p, std::ios::binary | std::ios::trunc);
  f << text;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc != 2) {
    std::printf("usage: qualify_check <empty directory>\n");
    return 2;
  }
  const std::string dir = argv[1];
  auto made = HipTargetModelBackend::create(0);
  if (!made) {
    std::printf("FAIL create: %s\n", made.error().detail.c_str());
    return 2;
  }
  const HipTargetModelBackend &be = **made;
  auto env = captureHipExecutionEnvironment(be);
  check((bool)env, "environment captured");
  if (!env) return 1;
  check(env->digest.size() == 71 && env->digest.rfind("sha256:", 0) == 0, "environment digest " + env->digest);

  struct Case { LogicalFormat in, out; uint16_t m, k, n, b; TargetGemmOrientation rt; uint64_t seed; const char *name; };
  const Case cases[] = {
      {LogicalFormat::F32, LogicalFormat::F32, 48, 70, 96, 1, TargetGemmOrientation::Normal, 20260803, "f32-cx"},
      {LogicalFormat::BF16, LogicalFormat::F32, 33, 129, 65, 3, TargetGemmOrientation::Transpose, 7, "bf16-f32-ncx-rt"},
      {LogicalFormat::F16, LogicalFormat::F16, 64, 256, 128, 1, TargetGemmOrientation::Normal, 11, "f16-cx"},
  };
  for (const Case &c : cases) {
    auto spec = HipQualificationSpec::create(c.in, c.out, c.m, c.k, c.n, c.b, c.rt, c.seed);
    check((bool)spec, std::string(c.name) + ": spec");
    if (!spec) continue;
    auto req = materializeHipQualificationCase(be, *spec);
    check((bool)req, std::string(c.name) + ": case materialised");
    if (!req) continue;
    auto again = materializeHipQualificationCase(be, *spec);
    check(again && hipProblemDigest(*again) == hipProblemDigest(*req), std::string(c.name) + ": case is deterministic");
    const std::vector<uint8_t> formal = formal_destination(*req);
    const std::string path = dir + "/" + c.name + ".json";
    auto digest = validateHipBackend(be, *spec, formal, path);
    check((bool)digest, std::string(c.name) + ": validation stage wrote the record");
    if (!digest) {
      std::printf("     %s\n", digest.error().detail.c_str());
      continue;
    }
    check(!validateHipBackend(be, *spec, formal, path), std::string(c.name) + ": an existing record is never replaced");
    std::vector<uint8_t> wrong = formal;
    wrong[wrong.size() / 2] ^= 1;
    check(!validateHipBackend(be, *spec, wrong, path + ".wrong"), std::string(c.name) + ": a wrong formal output is refused");
    auto rec = loadVerifiedHipQualificationRecord(path);
    check(rec && rec->getRecordDigest() == *digest && rec->getSpecDigest() == spec->digest(),
          std::string(c.name) + ": record loads and verifies");
    if (!rec) {
      std::printf("     %s\n", rec.error().detail.c_str());
      continue;
    }
    auto q = rec->qualifyExecution(*env, *req);
    check((bool)q, std::string(c.name) + ": execution qualified");
    if (q) {
      auto run = executeQualifiedHip(be, *q, *req);
      check(run && run->evidence.evidenceKind == TargetModelOneDNNEvidenceKind::ExactQualificationRecord &&
                run->evidence.evidenceDigest == *digest && run->destination.storage == formal,
            std::string(c.name) + ": qualified execution, evidence names the record");
    }
    // another payload: the problem digest differs
    TargetModelGemmRequest other = *req;
    other.tensors.inputs[0].storage[0] ^= 0x10;
    check(!rec->qualifyExecution(*env, other), std::string(c.name) + ": another payload is not qualified");
    // another environment
    HipExecutionEnvironment fake = *env;
    fake.record["driver_version"] = Json::integer(-1);
    fake.digest = sha256Digest(canonicalJson(fake.record));
    check(!rec->qualifyExecution(fake, *req), std::string(c.name) + ": another environment is not qualified");
    // tampered records
    const std::string text = slurp(path);
    spit(path + ".pretty", text.substr(0, text.size() - 1) + " \n");
    check(!loadVerifiedHipQualificationRecord(path + ".pretty"), std::string(c.name) + ": non-canonical record refused");
    std::string edited = text;
    const size_t at = edited.find("\"m\":");
    edited.replace(at, 4, "\"m\":1");
    spit(path + ".edited", edited);
    check(!loadVerifiedHipQualificationRecord(path + ".edited"),
          std::string(c.name) + ": edited spec refused (spec digest)");
    std::string extra = text;
    extra.insert(1, "\"aaa\":1,");
    spit(path + ".extra", extra);
    check(!loadVerifiedHipQualificationRecord(path + ".extra"), std::string(c.name) + ": unknown field refused");
  }
  std::printf("%s\n", failures ? "FAILED" : "ALL OK");
  return failures ? 1 : 0;
}
