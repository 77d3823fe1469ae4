// seam_check.cpp -- drives HipTargetModelBackend through the reference's two
// seams the way the simulator's command executor does
// (lib/Wafer/Simulator/Kernel/TargetModelTensorNumeric.cpp:160-183 and
// :750-826), and checks every result byte for byte against the CPU oracle
// (oracle/wafer_oracle.h, test infrastructure): unpack the physical inputs,
// run the command, pack into a copy of the destination template.
//
// Also checks the contract around the numbers: evidence fields the caller
// validates, untouched template bytes, and that bad requests fail with the
// right error code before any output exists.
//
// Exit status 0 when every check passes; one line per check on stdout.
#include "target_model_hip_backend.h"

extern "C" {
#include "wafer_oracle.h"
}

#include <cstdio>
#include <cstring>
#include <random>

using namespace wafer::model;

namespace {

int failures = 0;
void check(bool ok, const char *what) {
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
  std::fflush(stdout);
  if (!ok) ++failures;
}

PhysicalTensorDescriptor desc(LogicalFormat f, PhysicalTensorLayout l, std::vector<uint64_t> s) {
  Expected<PhysicalTensorDescriptor> d = PhysicalTensorDescriptor::create(f, l, std::move(s));
  if (!d) {
    std::printf("FAIL descriptor: %s\n", d.error().detail.c_str());
    std::exit(2);
  }
  return *d;
}

size_t elem_bytes(LogicalFormat f) { return f == LogicalFormat::F32 || f == LogicalFormat::I32 ? 4 : f == LogicalFormat::I8 ? 1 : 2; }

// logical values (raw storage bits) for a descriptor
std::vector<uint8_t> random_logical(const PhysicalTensorDescriptor &d, std::mt19937 &rng, float scale = 1.0f) {
  std::normal_distribution<float> nd(0.0f, scale);
  const uint64_t n = d.getElementCount();
  std::vector<uint8_t> out(n * elem_bytes(d.getFormat()));
  for (uint64_t i = 0; i < n; ++i) {
    const float v = nd(rng);
    if (d.getFormat() == LogicalFormat::F32) {
      std::memcpy(&out[4 * i], &v, 4);
    } else if (d.getFormat() == LogicalFormat::BF16) {
      uint32_t u;
      std::memcpy(&u, &v, 4);
      const uint16_t b = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
      std::memcpy(&out[2 * i], &b, 2);
    } else {
      uint16_t h = 0;
      oracle_f32_to_f16(v, &h);
      std::memcpy(&out[2 * i], &h, 2);
    }
  }
  return out;
}

std::vector<int64_t> s64(const PhysicalTensorDescriptor &d) {
  return std::vector<int64_t>(d.getShape().begin(), d.getShape().end());
}

// physical image of logical values over a template
std::vector<uint8_t> to_physical(const PhysicalTensorDescriptor &d, const std::vector<uint8_t> &logical, uint8_t fill) {
  std::vector<uint8_t> st(*d.getStorageBytes(), fill);
  const auto s = s64(d);
  oracle_pack((int)d.getFormat(), (int)d.getLayout(), s.data(), (int)s.size(), logical.data(), st.data(), (int64_t)st.size());
  return st;
}

void gemm_case(HipTargetModelBackend &be, std::mt19937 &rng, LogicalFormat fin, LogicalFormat fout, uint16_t B,
               uint16_t M, uint16_t K, uint16_t N, bool psum, bool rt, const char *name) {
  const bool batched = B > 1;
  const PhysicalTensorLayout L = batched ? PhysicalTensorLayout::NCx : PhysicalTensorLayout::Cx;
  auto shp = [&](uint64_t a, uint64_t b) {
    return batched ? std::vector<uint64_t>{B, a, b} : std::vector<uint64_t>{a, b};
  };
  PhysicalTensorDescriptor lhs = desc(fin, L, shp(M, K));
  PhysicalTensorDescriptor rhs = desc(fin, L, rt ? shp(N, K) : shp(K, N));
  PhysicalTensorDescriptor dst = desc(fout, L, shp(M, N));
  std::optional<PhysicalTensorDescriptor> ps;
  if (psum) ps = desc(LogicalFormat::F32, L, shp(M, N));
  auto a = random_logical(lhs, rng), b = random_logical(rhs, rng);
  std::vector<uint8_t> p = psum ? random_logical(*ps, rng) : std::vector<uint8_t>{};
  TargetModelGemmRequest req{FormalGemmOperation{lhs, rhs, dst, M, K, N, B, TargetGemmOrientation::Normal,
                                                 rt ? TargetGemmOrientation::Transpose : TargetGemmOrientation::Normal, ps},
                             TargetModelNumericOperands{{{lhs, to_physical(lhs, a, 0)}, {rhs, to_physical(rhs, b, 0)}},
                                                        {dst, std::vector<uint8_t>(*dst.getStorageBytes(), 0xA5)}}};
  if (psum) req.tensors.inputs.push_back({*ps, to_physical(*ps, p, 0)});
  // oracle: formal GEMM on the logical tensors, packed into the same template
  std::vector<uint8_t> want_logical(dst.getElementCount() * elem_bytes(fout));
  oracle_gemm_formal((int)fin, (int)fout, a.data(), b.data(), psum ? (const float *)p.data() : nullptr,
                     want_logical.data(), M, K, N, B, 0, rt ? 1 : 0, 4);
  std::vector<uint8_t> want = to_physical(dst, want_logical, 0xA5);
  auto r = be.tryExecute(req);
  check((bool)r && r->has_value(), name);
  if (!r || !r->has_value()) {
    if (!r) std::printf("     error %s: %s\n", stringifyTargetModelKernelErrorCode(r.error().code), r.error().detail.c_str());
    return;
  }
  const TargetModelOneDNNResult &res = **r;
  check(res.destination.key == dst && res.destination.storage == want, "  gemm bytes equal the formal lane, template bytes kept");
  check(res.evidence.matmulInvocations == 1 && res.evidence.reorderInvocations <= 1 &&
            res.evidence.formalFusedMultiplyAdds == 0 && !res.evidence.evidenceDigest.empty() &&
            !res.evidence.implementation.empty(),
        "  gemm evidence as the caller validates it");
}

}  // namespace

int main() {
  auto made = HipTargetModelBackend::create(0);
  if (!made) {
    std::printf("FAIL create: %s\n", made.error().detail.c_str());
    return 2;
  }
  HipTargetModelBackend &be = **made;
  std::mt19937 rng(20260803);
  const auto budget = FormalNumericWorkBudget::create(1u << 24, 1u << 30);

  // ---- GEMM through TargetModelOneDNNBackend::tryExecute
  gemm_case(be, rng, LogicalFormat::F32, LogicalFormat::F32, 1, 48, 70, 96, false, false, "gemm f32 Cx 48x70x96");
  gemm_case(be, rng, LogicalFormat::BF16, LogicalFormat::BF16, 1, 33, 129, 65, false, true, "gemm bf16 Cx rhs Transpose");
  gemm_case(be, rng, LogicalFormat::F16, LogicalFormat::F32, 3, 17, 40, 130, true, false, "gemm f16->f32 NCx batch 3 + psum");

  // ---- elementwise Square on bf16 Cx, and binary Add on f32 NCx (IEEE-exact
  // operations, so the bytes must match; the transcendental ops are checked
  // within tolerance by the Python parity suite)
  {
    PhysicalTensorDescriptor d = desc(LogicalFormat::BF16, PhysicalTensorLayout::Cx, {37, 200});
    auto x = random_logical(d, rng);
    TargetModelElementwiseRequest req{FormalElementwiseOperation{TargetElementwiseOperation::Square, {d}, d},
                                      TargetModelNumericOperands{{{d, to_physical(d, x, 0)}},
                                                                 {d, std::vector<uint8_t>(*d.getStorageBytes(), 0x5A)}}};
    std::vector<uint8_t> wl(x.size());
    oracle_elementwise((int)TargetElementwiseOperation::Square, (int)LogicalFormat::BF16, x.data(), nullptr, wl.data(),
                       (int64_t)d.getElementCount());
    auto r = be.execute(req, budget);
    check((bool)r, "elementwise Square bf16 Cx");
    if (r) {
      check(r->destination.storage == to_physical(d, wl, 0x5A), "  elementwise bytes equal the managed lane");
      check(r->evidence.scalarEvaluations == d.getElementCount() && !r->evidence.environmentDigest.empty(),
            "  elementwise evidence: one evaluation per element");
    }
    // budget: one element short
    auto small = FormalNumericWorkBudget::create(d.getElementCount() - 1, 1);
    auto rb = be.execute(req, small);
    check(!rb && rb.error().code == TargetModelKernelErrorCode::WorkBudgetExceeded, "elementwise over budget fails");
  }
  {
    PhysicalTensorDescriptor d = desc(LogicalFormat::F32, PhysicalTensorLayout::NCx, {2, 9, 130});
    auto x = random_logical(d, rng), y = random_logical(d, rng);
    TargetModelElementwiseRequest req{FormalElementwiseOperation{TargetElementwiseOperation::Add, {d, d}, d},
                                      TargetModelNumericOperands{{{d, to_physical(d, x, 0)}, {d, to_physical(d, y, 0)}},
                                                                 {d, std::vector<uint8_t>(*d.getStorageBytes(), 0x11)}}};
    std::vector<uint8_t> wl(x.size());
    oracle_elementwise((int)TargetElementwiseOperation::Add, (int)LogicalFormat::F32, x.data(), y.data(), wl.data(),
                       (int64_t)d.getElementCount());
    auto r = be.execute(req, budget);
    check((bool)r && r->destination.storage == to_physical(d, wl, 0x11), "elementwise Add f32 NCx");
  }

  // ---- convert F32 -> BF16 (route 167) on Cx
  {
    PhysicalTensorDescriptor s = desc(LogicalFormat::F32, PhysicalTensorLayout::Cx, {21, 300});
    PhysicalTensorDescriptor d = desc(LogicalFormat::BF16, PhysicalTensorLayout::Cx, {21, 300});
    auto x = random_logical(s, rng, 1e3f);
    TargetModelConvertRequest req{FormalConvertOperation{167, s, d},
                                  TargetModelNumericOperands{{{s, to_physical(s, x, 0)}},
                                                             {d, std::vector<uint8_t>(*d.getStorageBytes(), 0x77)}}};
    std::vector<uint8_t> wl(d.getElementCount() * 2);
    oracle_convert(167, 0, x.data(), wl.data(), (int64_t)s.getElementCount());
    auto r = be.execute(req, budget);
    check((bool)r && r->destination.storage == to_physical(d, wl, 0x77), "convert F32->BF16 (route 167) Cx");
    // route/format mismatch: BF16 descriptors with the F32->BF16 route
    TargetModelConvertRequest bad{FormalConvertOperation{167, d, d},
                                  TargetModelNumericOperands{{{d, std::vector<uint8_t>(*d.getStorageBytes(), 0)}},
                                                             {d, std::vector<uint8_t>(*d.getStorageBytes(), 0)}}};
    auto rb = be.execute(bad, budget);
    check(!rb && rb.error().code == TargetModelKernelErrorCode::InvalidCommandField, "convert with mismatched route fails");
  }

  // ---- reduce Sum over Trailing0 (F32, NCx)
  {
    PhysicalTensorDescriptor in = desc(LogicalFormat::F32, PhysicalTensorLayout::NCx, {2, 3, 5, 70});
    PhysicalTensorDescriptor out = desc(LogicalFormat::F32, PhysicalTensorLayout::NCx, {2, 3, 5, 1});
    auto x = random_logical(in, rng);
    TargetModelReduceRequest req{FormalReduceOperation{TargetReduceOperation::Sum, in, out, TargetReduceDimension::Trailing0},
                                 TargetModelNumericOperands{{{in, to_physical(in, x, 0)}},
                                                            {out, std::vector<uint8_t>(*out.getStorageBytes(), 0x33)}}};
    std::vector<uint8_t> wl(out.getElementCount() * 4);
    const auto s = s64(in);
    oracle_reduce(0, 0, (int)LogicalFormat::F32, s.data(), (int)s.size(), x.data(), wl.data());
    auto r = be.execute(req, budget);
    check((bool)r && r->destination.storage == to_physical(out, wl, 0x33) &&
              r->evidence.scalarEvaluations == in.getElementCount(),
          "reduce Sum Trailing0 f32 NCx (evaluations = input elements)");
  }

  // ---- bad requests fail with no output
  {
    PhysicalTensorDescriptor d = desc(LogicalFormat::F32, PhysicalTensorLayout::Cx, {4, 64});
    TargetModelElementwiseRequest req{FormalElementwiseOperation{TargetElementwiseOperation::Abs, {d}, d},
                                      TargetModelNumericOperands{{{d, std::vector<uint8_t>(7, 0)}},
                                                                 {d, std::vector<uint8_t>(*d.getStorageBytes(), 0)}}};
    auto r = be.execute(req, budget);
    check(!r && r.error().code == TargetModelKernelErrorCode::InvalidCommandField, "short input storage fails");
    PhysicalTensorDescriptor i8 = desc(LogicalFormat::I8, PhysicalTensorLayout::Cx, {4, 128});
    TargetModelGemmRequest g{FormalGemmOperation{i8, i8, i8, 4, 128, 4, 1, TargetGemmOrientation::Normal,
                                                 TargetGemmOrientation::Normal, std::nullopt},
                             TargetModelNumericOperands{{{i8, std::vector<uint8_t>(*i8.getStorageBytes(), 0)},
                                                         {i8, std::vector<uint8_t>(*i8.getStorageBytes(), 0)}},
                                                        {i8, std::vector<uint8_t>(*i8.getStorageBytes(), 0)}}};
    auto rg = be.tryExecute(g);
    check(!rg && rg.error().code == TargetModelKernelErrorCode::UnsupportedCommand, "I8 formal GEMM is unsupported, as in the reference");
  }

  std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "PASSED", failures);
  return failures ? 1 : 0;
}
