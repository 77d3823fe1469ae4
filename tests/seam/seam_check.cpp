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
  TargetModelGemmRequest req{FormalGemmOperation{lhs, rhs, dst, M, K, N, B, *getCanonicalFormalGemmGeometry(batched ? 3 : 2),
                                                 TargetGemmOrientation::Normal,
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
  check(!res.flags.any(), "  gemm flags empty, as the managed lane returns them");
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
    TargetModelConvertRequest req{FormalConvertOperation{167, s, d, TargetConvertParameter::roundingMode(
                                                                     TargetRoundingMode::NearestEven)},
                                  TargetModelNumericOperands{{{s, to_physical(s, x, 0)}},
                                                             {d, std::vector<uint8_t>(*d.getStorageBytes(), 0x77)}}};
    std::vector<uint8_t> wl(d.getElementCount() * 2);
    oracle_convert(167, 0, x.data(), wl.data(), (int64_t)s.getElementCount());
    auto r = be.execute(req, budget);
    check((bool)r && r->destination.storage == to_physical(d, wl, 0x77), "convert F32->BF16 (route 167) Cx");
    // route/format mismatch: BF16 descriptors with the F32->BF16 route
    TargetModelConvertRequest bad{FormalConvertOperation{167, d, d, std::nullopt},
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

  // ---- the managed lane's domain (ManagedReferenceTargetModel.cpp:137-458):
  // each refusal fails with ManagedReferenceBackendFailure and the
  // reference's message, and returns no output
  {
    auto refused = [&](const auto &r, const char *message, const char *name) {
      const bool ok = !r && r.error().code == TargetModelKernelErrorCode::ManagedReferenceBackendFailure &&
                      r.error().detail == std::string("managed-reference tensor: ") + message;
      check(ok, name);
      if (!ok && !r) std::printf("     got %s: %s\n", stringifyTargetModelKernelErrorCode(r.error().code),
                                 r.error().detail.c_str());
    };
    auto set_f32 = [](std::vector<uint8_t> &v, size_t i, uint32_t bits) { std::memcpy(&v[4 * i], &bits, 4); };
    PhysicalTensorDescriptor f = desc(LogicalFormat::F32, PhysicalTensorLayout::Cx, {6, 70});
    PhysicalTensorDescriptor b = desc(LogicalFormat::BF16, PhysicalTensorLayout::Cx, {6, 70});
    auto tmpl = [](const PhysicalTensorDescriptor &d) { return std::vector<uint8_t>(*d.getStorageBytes(), 0x3C); };
    auto x = random_logical(f, rng);
    // convert: a TowardZero parameter; a zero-point parameter
    {
      TargetModelConvertRequest r{FormalConvertOperation{167, f, b, TargetConvertParameter::roundingMode(
                                                                        TargetRoundingMode::TowardZero)},
                                  TargetModelNumericOperands{{{f, to_physical(f, x, 0)}}, {b, tmpl(b)}}};
      refused(be.execute(r, budget), "convert is not nearest-even", "convert TowardZero is refused");
      r.operation.parameter = TargetConvertParameter::zeroPoint(3);
      refused(be.execute(r, budget), "convert is not nearest-even", "convert with a zero point is refused");
    }
    // convert: an integer route, and one layout to another
    {
      PhysicalTensorDescriptor i32 = desc(LogicalFormat::I32, PhysicalTensorLayout::Cx, {6, 70});
      TargetModelConvertRequest r{FormalConvertOperation{149, i32, f, std::nullopt},
                                  TargetModelNumericOperands{{{i32, std::vector<uint8_t>(*i32.getStorageBytes(), 0)}},
                                                             {f, tmpl(f)}}};
      refused(be.execute(r, budget), "convert is outside the F16/BF16/F32 same-shape domain",
              "convert I32->F32 is outside the managed domain");
      PhysicalTensorDescriptor bt = desc(LogicalFormat::BF16, PhysicalTensorLayout::Tensor, {6, 70});
      TargetModelConvertRequest r2{FormalConvertOperation{167, f, bt, std::nullopt},
                                   TargetModelNumericOperands{{{f, to_physical(f, x, 0)}}, {bt, tmpl(bt)}}};
      refused(be.execute(r2, budget), "convert is outside the F16/BF16/F32 same-shape domain",
              "convert Cx -> Tensor layout is outside the managed domain");
    }
    // convert: a NaN input
    {
      auto xn = x;
      set_f32(xn, 131, 0x7fc00000u);
      TargetModelConvertRequest r{FormalConvertOperation{167, f, b, std::nullopt},
                                  TargetModelNumericOperands{{{f, to_physical(f, xn, 0)}}, {b, tmpl(b)}}};
      refused(be.execute(r, budget), "input value is outside the non-NaN domain", "convert of a NaN is refused");
    }
    // elementwise: NaN result (Sqrt of a negative), NaN input (Add), an
    // operation outside the managed set, an arity mismatch
    {
      TargetModelElementwiseRequest r{FormalElementwiseOperation{TargetElementwiseOperation::Sqrt, {f}, f},
                                      TargetModelNumericOperands{{{f, to_physical(f, x, 0)}}, {f, tmpl(f)}}};
      refused(be.execute(r, budget), "result value is outside the non-NaN domain", "Sqrt of a negative is refused");
      auto xa = x, xb = x;  // xa = |x|
      for (size_t i = 0; i < f.getElementCount(); ++i) {
        float v;
        std::memcpy(&v, &x[4 * i], 4);
        v = v < 0 ? -v : v;
        std::memcpy(&xa[4 * i], &v, 4);
      }
      set_f32(xb, 17, 0xffc00000u);
      TargetModelElementwiseRequest r2{FormalElementwiseOperation{TargetElementwiseOperation::Add, {f, f}, f},
                                       TargetModelNumericOperands{{{f, to_physical(f, xa, 0)}, {f, to_physical(f, xb, 0)}},
                                                                  {f, tmpl(f)}}};
      refused(be.execute(r2, budget), "input value is outside the non-NaN domain", "Add with a NaN input is refused");
      TargetModelElementwiseRequest r3{FormalElementwiseOperation{TargetElementwiseOperation::Eq, {f, f}, f},
                                       TargetModelNumericOperands{{{f, to_physical(f, xa, 0)}, {f, to_physical(f, xa, 0)}},
                                                                  {f, tmpl(f)}}};
      refused(be.execute(r3, budget), "elementwise operation is not in the managed domain", "Eq is refused");
      TargetModelElementwiseRequest r4{FormalElementwiseOperation{TargetElementwiseOperation::Add, {f}, f},
                                       TargetModelNumericOperands{{{f, to_physical(f, xa, 0)}}, {f, tmpl(f)}}};
      refused(be.execute(r4, budget), "elementwise input arity does not match semantics", "unary Add is refused");
      // and the positive counterpart: the same Sqrt on |x| succeeds with empty flags
      TargetModelElementwiseRequest r5{FormalElementwiseOperation{TargetElementwiseOperation::Sqrt, {f}, f},
                                       TargetModelNumericOperands{{{f, to_physical(f, xa, 0)}}, {f, tmpl(f)}}};
      auto ok = be.execute(r5, budget);
      check((bool)ok && !ok->flags.any(), "Sqrt of |x| succeeds with empty flags");
    }
    // reduce: a BF16 Sum, an accumulator that meets +inf and -inf, a NaN input to Max
    {
      PhysicalTensorDescriptor in = desc(LogicalFormat::BF16, PhysicalTensorLayout::NCx, {2, 3, 4, 40});
      PhysicalTensorDescriptor out = desc(LogicalFormat::BF16, PhysicalTensorLayout::NCx, {2, 3, 4, 1});
      TargetModelReduceRequest r{FormalReduceOperation{TargetReduceOperation::Sum, in, out, TargetReduceDimension::Trailing0},
                                 TargetModelNumericOperands{{{in, std::vector<uint8_t>(*in.getStorageBytes(), 0)}},
                                                            {out, tmpl(out)}}};
      refused(be.execute(r, budget), "reduce requires F32 sum or F16/BF16/F32 max/min", "BF16 Sum is refused");
      PhysicalTensorDescriptor fi = desc(LogicalFormat::F32, PhysicalTensorLayout::NCx, {2, 3, 4, 40});
      PhysicalTensorDescriptor fo = desc(LogicalFormat::F32, PhysicalTensorLayout::NCx, {2, 3, 4, 1});
      auto xi = random_logical(fi, rng);
      set_f32(xi, 45, 0x7f800000u);
      set_f32(xi, 77, 0xff800000u);  // same row (40..79) as index 45
      TargetModelReduceRequest r2{FormalReduceOperation{TargetReduceOperation::Sum, fi, fo, TargetReduceDimension::Trailing0},
                                  TargetModelNumericOperands{{{fi, to_physical(fi, xi, 0)}}, {fo, tmpl(fo)}}};
      refused(be.execute(r2, budget), "reduce accumulator left the non-NaN domain", "Sum of +inf and -inf is refused");
      auto xm = random_logical(fi, rng);
      set_f32(xm, 300, 0x7fc00001u);
      TargetModelReduceRequest r3{FormalReduceOperation{TargetReduceOperation::Max, fi, fo, TargetReduceDimension::Trailing0},
                                  TargetModelNumericOperands{{{fi, to_physical(fi, xm, 0)}}, {fo, tmpl(fo)}}};
      refused(be.execute(r3, budget), "input value is outside the non-NaN domain", "Max over a NaN is refused");
    }
    // GEMM: axes other than the canonical ones
    {
      PhysicalTensorDescriptor l = desc(LogicalFormat::F32, PhysicalTensorLayout::Cx, {8, 64});
      PhysicalTensorDescriptor d = desc(LogicalFormat::F32, PhysicalTensorLayout::Cx, {8, 8});
      PhysicalTensorDescriptor rr = desc(LogicalFormat::F32, PhysicalTensorLayout::Cx, {64, 8});
      FormalGemmGeometry axes = *getCanonicalFormalGemmGeometry(2);
      std::swap(axes.lhsMDimension, axes.lhsContractingDimension);
      TargetModelGemmRequest g{FormalGemmOperation{l, rr, d, 8, 64, 8, 1, axes, TargetGemmOrientation::Normal,
                                                   TargetGemmOrientation::Normal, std::nullopt},
                               TargetModelNumericOperands{{{l, std::vector<uint8_t>(*l.getStorageBytes(), 0)},
                                                           {rr, std::vector<uint8_t>(*rr.getStorageBytes(), 0)}},
                                                          {d, tmpl(d)}}};
      auto rg = be.tryExecute(g);
      check(!rg && rg.error().code == TargetModelKernelErrorCode::InvalidCommandField,
            "GEMM with non-canonical axes is refused");
    }
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
    TargetModelGemmRequest g{FormalGemmOperation{i8, i8, i8, 4, 128, 4, 1, *getCanonicalFormalGemmGeometry(2),
                                                 TargetGemmOrientation::Normal,
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
