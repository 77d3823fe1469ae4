// target_model_hip_backend.cpp -- HipTargetModelBackend over the C ABI.
//
// Each command runs: validate everything (no launch on a bad request) ->
// upload the physical input images -> unpack them on the GPU (Cx/NCx codec)
// -> run the command kernel on the logical tensors -> upload the destination
// template and pack the result into it (template bytes not owned by logical
// elements survive) -> download.  The device buffers live for one call.
//
// Validation follows the reference's managed backend and formal GEMM:
// executeGemm (lib/Wafer/Simulator/Reference/Numeric/FormalTensorNumeric.cpp:272-361),
// ManagedReference::executeElementwise / executeConvert / executeReduce
// (lib/Wafer/Simulator/Reference/ManagedReferenceTargetModel.cpp:302-458) and
// the caller's result checks (lib/Wafer/Simulator/Kernel/TargetModelTensorNumeric.cpp:160-183).
#include "target_model_hip_backend.h"

#include "wafer_hip.h"

#include <algorithm>
#include <cstring>

namespace wafer::model {
namespace {

TargetModelKernelError err(TargetModelKernelErrorCode code, std::string detail) {
  return TargetModelKernelError{code, std::move(detail)};
}

// C ABI status -> the seam's error code
TargetModelKernelError from_status(int status, const char *what) {
  TargetModelKernelErrorCode code = TargetModelKernelErrorCode::ManagedReferenceBackendFailure;
  switch (status) {
  case WAFER_HIP_E_INVALID_FIELD: code = TargetModelKernelErrorCode::InvalidCommandField; break;
  case WAFER_HIP_E_BUDGET: code = TargetModelKernelErrorCode::WorkBudgetExceeded; break;
  case WAFER_HIP_E_UNSUPPORTED: code = TargetModelKernelErrorCode::UnsupportedCommand; break;
  case WAFER_HIP_E_MEMORY: code = TargetModelKernelErrorCode::MemoryReadFailure; break;
  case WAFER_HIP_E_NUMERIC: code = TargetModelKernelErrorCode::FormalNumericFailure; break;
  case WAFER_HIP_E_CODEC: code = TargetModelKernelErrorCode::PhysicalCodecFailure; break;
  case WAFER_HIP_E_UNAVAILABLE: code = TargetModelKernelErrorCode::ManagedReferenceBackendUnavailable; break;
  default: break;
  }
  return err(code, std::string(what) + ": " + wafer_hip_last_error());
}

std::vector<int64_t> shape64(const PhysicalTensorDescriptor &d) {
  return std::vector<int64_t>(d.getShape().begin(), d.getShape().end());
}

uint64_t logical_bytes(const PhysicalTensorDescriptor &d) {
  const uint32_t f = (uint32_t)d.getFormat();
  const uint64_t eb = f == WAFER_FMT_I8 ? 1 : (f == WAFER_FMT_I32 || f == WAFER_FMT_F32 || f == WAFER_FMT_TF32) ? 4 : 2;
  return d.getElementCount() * eb;
}

// One device buffer for the duration of a call.
class DeviceBuffer {
public:
  DeviceBuffer(wafer_hip_context *c) : ctx(c) {}
  DeviceBuffer(const DeviceBuffer &) = delete;
  ~DeviceBuffer() { if (ptr) wafer_hip_buffer_free(ctx, ptr); }
  int allocate(uint64_t bytes) { return wafer_hip_buffer_alloc(ctx, bytes, &ptr); }
  void *get() const { return ptr; }

private:
  wafer_hip_context *ctx;
  void *ptr = nullptr;
};

// storage size must match the descriptor's physical image exactly
std::optional<TargetModelKernelError> check_storage(const TargetModelNumericTensor &t, const char *what) {
  Expected<uint64_t> bytes = t.key.getStorageBytes();
  if (!bytes) return bytes.error();
  if (t.storage.size() != *bytes)
    return err(TargetModelKernelErrorCode::InvalidCommandField,
               std::string(what) + ": storage holds " + std::to_string(t.storage.size()) +
                   " bytes, the physical image needs " + std::to_string(*bytes));
  return std::nullopt;
}

// upload a physical image and unpack it into a logical device tensor
int upload_logical(wafer_hip_context *ctx, const TargetModelNumericTensor &t, DeviceBuffer &physical,
                   DeviceBuffer &logical) {
  const PhysicalTensorDescriptor &d = t.key;
  const std::vector<int64_t> s = shape64(d);
  if (int st = physical.allocate(t.storage.size())) return st;
  if (int st = logical.allocate(logical_bytes(d))) return st;
  if (int st = wafer_hip_copy_to_device(ctx, physical.get(), t.storage.data(), t.storage.size())) return st;
  return wafer_hip_unpack(ctx, (uint32_t)d.getFormat(), (uint32_t)d.getLayout(), s.data(), (uint32_t)s.size(),
                          physical.get(), (int64_t)t.storage.size(), logical.get());
}

// pack a logical device tensor into (a device copy of) the destination
// template and download the result
int pack_into_template(wafer_hip_context *ctx, const TargetModelNumericTensor &tmpl, const DeviceBuffer &logical,
                       std::vector<uint8_t> &out) {
  const PhysicalTensorDescriptor &d = tmpl.key;
  const std::vector<int64_t> s = shape64(d);
  DeviceBuffer physical(ctx);
  if (int st = physical.allocate(tmpl.storage.size())) return st;
  if (int st = wafer_hip_copy_to_device(ctx, physical.get(), tmpl.storage.data(), tmpl.storage.size())) return st;
  if (int st = wafer_hip_pack(ctx, (uint32_t)d.getFormat(), (uint32_t)d.getLayout(), s.data(), (uint32_t)s.size(),
                              logical.get(), physical.get(), (int64_t)tmpl.storage.size()))
    return st;
  out.resize(tmpl.storage.size());
  return wafer_hip_copy_to_host(ctx, out.data(), physical.get(), out.size());
}

std::string environment_digest(wafer_hip_context *) {
  // the evidence must name the execution environment; the implementation
  // string carries the kernel set, the prefix the target
  return std::string("gfx950/") + wafer_hip_implementation();
}

bool is_float(LogicalFormat f) {
  return f == LogicalFormat::F16 || f == LogicalFormat::BF16 || f == LogicalFormat::F32;
}

// A managed-lane refusal: the reference's backend reports these as string
// errors prefixed "managed-reference tensor: " (referenceError,
// ManagedReferenceTargetModel.cpp:27-31), which its caller turns into
// ManagedReferenceBackendFailure (TargetModelTensorNumeric.cpp:168-173).
TargetModelKernelError managed(const std::string &detail) {
  return err(TargetModelKernelErrorCode::ManagedReferenceBackendFailure, "managed-reference tensor: " + detail);
}

// getTargetElementwiseArity (lib/Wafer/Target/TargetOperation.cpp:255-300)
unsigned elementwise_arity(TargetElementwiseOperation op) {
  switch (op) {
  case TargetElementwiseOperation::Max: case TargetElementwiseOperation::Min: case TargetElementwiseOperation::Add:
  case TargetElementwiseOperation::Sub: case TargetElementwiseOperation::Mul: case TargetElementwiseOperation::Eq:
  case TargetElementwiseOperation::Ne: case TargetElementwiseOperation::Ge: case TargetElementwiseOperation::Gt:
  case TargetElementwiseOperation::Le: case TargetElementwiseOperation::Lt: case TargetElementwiseOperation::LogicAnd:
  case TargetElementwiseOperation::LogicOr: case TargetElementwiseOperation::LogicXor:
    return 2;
  default:
    return 1;
  }
}

// The relation / logic / saturating operations evaluateElementwise refuses
// (ManagedReferenceTargetModel.cpp:284-296).
bool in_managed_elementwise_domain(TargetElementwiseOperation op) {
  switch (op) {
  case TargetElementwiseOperation::Eq: case TargetElementwiseOperation::Ne: case TargetElementwiseOperation::Ge:
  case TargetElementwiseOperation::Gt: case TargetElementwiseOperation::Le: case TargetElementwiseOperation::Lt:
  case TargetElementwiseOperation::LogicNot: case TargetElementwiseOperation::LogicAnd:
  case TargetElementwiseOperation::LogicOr: case TargetElementwiseOperation::LogicXor:
  case TargetElementwiseOperation::SatRelu: case TargetElementwiseOperation::LeakyRelu:
    return false;
  default:
    return true;
  }
}

// Index of the first NaN of a logical device tensor (count when none).
Expected<uint64_t> first_nan(wafer_hip_context *ctx, const PhysicalTensorDescriptor &d, const void *logical) {
  uint64_t first = 0;
  if (int st = wafer_hip_first_nan(ctx, (uint32_t)d.getFormat(), logical, d.getElementCount(), &first))
    return from_status(st, "non-NaN domain check");
  return first;
}

}  // namespace

Expected<FormalGemmGeometry> getCanonicalFormalGemmGeometry(uint64_t rank) {
  if (rank < 2)
    return err(TargetModelKernelErrorCode::InvalidCommandField, "canonical numeric GEMM axes require rank at least 2");
  const uint64_t base = rank - 2;
  std::vector<uint64_t> batch;
  for (uint64_t d = 0; d < base; ++d) batch.push_back(d);
  return FormalGemmGeometry{batch, base, base + 1, batch, base, base + 1, batch, base, base + 1};
}

const char *stringifyTargetModelKernelErrorCode(TargetModelKernelErrorCode code) {
  switch (code) {
  case TargetModelKernelErrorCode::InvalidCommandField: return "InvalidCommandField";
  case TargetModelKernelErrorCode::WorkBudgetExceeded: return "WorkBudgetExceeded";
  case TargetModelKernelErrorCode::UnsupportedCommand: return "UnsupportedCommand";
  case TargetModelKernelErrorCode::MemoryReadFailure: return "MemoryReadFailure";
  case TargetModelKernelErrorCode::FormalNumericFailure: return "FormalNumericFailure";
  case TargetModelKernelErrorCode::PhysicalCodecFailure: return "PhysicalCodecFailure";
  case TargetModelKernelErrorCode::ManagedReferenceBackendUnavailable: return "ManagedReferenceBackendUnavailable";
  case TargetModelKernelErrorCode::ManagedReferenceBackendFailure: return "ManagedReferenceBackendFailure";
  case TargetModelKernelErrorCode::OneDNNBackendUnavailable: return "OneDNNBackendUnavailable";
  case TargetModelKernelErrorCode::OneDNNBackendFailure: return "OneDNNBackendFailure";
  }
  return "Unknown";
}

Expected<PhysicalTensorDescriptor> PhysicalTensorDescriptor::create(LogicalFormat format, PhysicalTensorLayout layout,
                                                                    std::vector<uint64_t> shape) {
  if (shape.empty() || shape.size() > 8)
    return err(TargetModelKernelErrorCode::InvalidCommandField, "descriptor: rank must be 1..8");
  uint64_t count = 1;
  for (uint64_t e : shape) {
    if (e == 0 || e > 65535)
      return err(TargetModelKernelErrorCode::InvalidCommandField, "descriptor: every extent must be in [1, 65535]");
    count *= e;
  }
  PhysicalTensorDescriptor d(format, layout, std::move(shape), count);
  // the geometry check of computePhysicalTensorGeometry
  Expected<uint64_t> bytes = d.getStorageBytes();
  if (!bytes) return bytes.error();
  return d;
}

Expected<uint64_t> PhysicalTensorDescriptor::getStorageBytes() const {
  const std::vector<int64_t> s(shape.begin(), shape.end());
  int64_t bytes = 0;
  if (int st = wafer_hip_physical_bytes((uint32_t)format, (uint32_t)layout, s.data(), (uint32_t)s.size(), &bytes))
    return from_status(st, "physical geometry");
  return (uint64_t)bytes;
}

Expected<std::unique_ptr<HipTargetModelBackend>> HipTargetModelBackend::create(int device) {
  wafer_hip_context *ctx = nullptr;
  if (int st = wafer_hip_context_create(device, &ctx)) {
    TargetModelKernelError e = from_status(st, "HIP backend");
    e.code = TargetModelKernelErrorCode::ManagedReferenceBackendUnavailable;
    return e;
  }
  return std::unique_ptr<HipTargetModelBackend>(new HipTargetModelBackend(ctx));
}

HipTargetModelBackend::~HipTargetModelBackend() { wafer_hip_context_destroy(ctx); }

// ---- GEMM -----------------------------------------------------------------------
Expected<std::optional<TargetModelOneDNNResult>>
HipTargetModelBackend::tryExecute(const TargetModelGemmRequest &request) const {
  const FormalGemmOperation &op = request.operation;
  const TargetModelNumericOperands &t = request.tensors;
  const size_t want_inputs = op.psum ? 3 : 2;
  if (t.inputs.size() != want_inputs)
    return err(TargetModelKernelErrorCode::InvalidCommandField, "gemm: expected lhs, rhs" + std::string(op.psum ? ", psum" : ""));
  if (!(t.inputs[0].key == op.lhs) || !(t.inputs[1].key == op.rhs) || !(t.destinationTemplate.key == op.destination) ||
      (op.psum && !(t.inputs[2].key == *op.psum)))
    return err(TargetModelKernelErrorCode::InvalidCommandField, "gemm: tensor keys differ from the operation's descriptors");
  {
    // the formal factory admits only the canonical axes (createFormalGemmOperation,
    // lib/Wafer/Simulator/Reference/Formal/FormalOperations.cpp:262-270)
    Expected<FormalGemmGeometry> canonical = getCanonicalFormalGemmGeometry(op.lhs.getShape().size());
    if (!canonical) return canonical.error();
    if (!(op.axes == *canonical))
      return err(TargetModelKernelErrorCode::InvalidCommandField,
                 "gemm: NE GEMM requires canonical leading batch and trailing M/K/N axes");
  }
  const LogicalFormat in = op.lhs.getFormat(), out = op.destination.getFormat();
  if (!is_float(in) || op.rhs.getFormat() != in || !is_float(out))
    return err(TargetModelKernelErrorCode::UnsupportedCommand, "gemm: formats must be F16, BF16 or F32 (lhs == rhs)");
  if (op.psum && op.psum->getFormat() != LogicalFormat::F32)
    return err(TargetModelKernelErrorCode::UnsupportedCommand, "gemm: partial sums must be F32");
  const uint64_t B = op.batchCount, M = op.m, K = op.k, N = op.n;
  if (!B || !M || !K || !N) return err(TargetModelKernelErrorCode::InvalidCommandField, "gemm: empty dimension");
  if (op.lhs.getElementCount() != B * M * K || op.rhs.getElementCount() != B * K * N ||
      op.destination.getElementCount() != B * M * N || (op.psum && op.psum->getElementCount() != B * M * N))
    return err(TargetModelKernelErrorCode::InvalidCommandField, "gemm: descriptor element counts do not match m, k, n, batch");
  for (size_t i = 0; i < t.inputs.size(); ++i)
    if (auto e = check_storage(t.inputs[i], "gemm input")) return *e;
  if (auto e = check_storage(t.destinationTemplate, "gemm destination")) return *e;

  DeviceBuffer lp(ctx), ll(ctx), rp(ctx), rl(ctx), pp(ctx), pl(ctx), dl(ctx);
  if (int st = upload_logical(ctx, t.inputs[0], lp, ll)) return from_status(st, "gemm lhs");
  if (int st = upload_logical(ctx, t.inputs[1], rp, rl)) return from_status(st, "gemm rhs");
  if (op.psum)
    if (int st = upload_logical(ctx, t.inputs[2], pp, pl)) return from_status(st, "gemm psum");
  if (int st = dl.allocate(logical_bytes(op.destination))) return from_status(st, "gemm destination");
  if (int st = wafer_hip_gemm(ctx, ll.get(), rl.get(), dl.get(), op.psum ? pl.get() : nullptr, (uint32_t)M, (uint32_t)K,
                              (uint32_t)N, (uint32_t)B, (uint32_t)in, (uint32_t)out,
                              op.psum ? (uint32_t)WAFER_FMT_F32 : WAFER_GEMM_PSUM_DISABLED,
                              (uint32_t)op.lhsOrientation, (uint32_t)op.rhsOrientation))
    return from_status(st, "gemm");
  TargetModelOneDNNResult res{TargetModelNumericTensor{op.destination, {}}, {}, {}};
  if (int st = pack_into_template(ctx, t.destinationTemplate, dl, res.destination.storage))
    return from_status(st, "gemm pack");
  res.evidence.matmulInvocations = 1;
  res.evidence.reorderInvocations = 0;
  res.evidence.formalFusedMultiplyAdds = 0;
  res.evidence.evidenceKind = TargetModelOneDNNEvidenceKind::ManagedReferenceEnvironment;
  res.evidence.evidenceDigest = environment_digest(ctx);
  res.evidence.implementation = wafer_hip_implementation();
  return std::optional<TargetModelOneDNNResult>(std::move(res));
}

// ---- elementwise ------------------------------------------------------------------
// Checks in the managed lane's order (executeManagedReference and
// executeElementwise, ManagedReferenceTargetModel.cpp:297-342, 500-540): tensor
// identity, the scalar budget, arity, one same-shape F16/BF16/F32 domain,
// the managed operation set, then the non-NaN domain.  The reference checks
// NaN element by element (decode the inputs, evaluate, encode); here the
// first NaN input and the first NaN result are located on the GPU and the
// earlier of the two decides the message (an input at the same index wins,
// since it is decoded first).
Expected<TargetModelManagedReferenceResult>
HipTargetModelBackend::execute(const TargetModelElementwiseRequest &request, FormalNumericWorkBudget budget) const {
  const FormalElementwiseOperation &op = request.operation;
  const TargetModelNumericOperands &t = request.tensors;
  if (!(t.destinationTemplate.key == op.destination) || t.inputs.size() != op.inputs.size())
    return managed("request tensor key does not match operation");
  for (size_t i = 0; i < op.inputs.size(); ++i)
    if (!(t.inputs[i].key == op.inputs[i])) return managed("request input key does not match operation");
  const uint64_t count = op.destination.getElementCount();
  if (count > budget.getMaximumScalarEvaluations())
    return err(TargetModelKernelErrorCode::WorkBudgetExceeded, "elementwise: " + std::to_string(count) +
                                                                   " evaluations exceed the scalar budget");
  if (op.inputs.size() != elementwise_arity(op.operation))
    return managed("elementwise input arity does not match semantics");
  for (const PhysicalTensorDescriptor &in : op.inputs)
    if (in.getShape() != op.destination.getShape() || in.getLayout() != op.destination.getLayout() ||
        in.getFormat() != op.destination.getFormat())
      return managed("elementwise tensors do not have one same-shape F16/BF16/F32 domain");
  if (!is_float(op.destination.getFormat())) return managed("elementwise result is not F16, BF16 or F32");
  if (!in_managed_elementwise_domain(op.operation))
    return managed("elementwise operation is not in the managed domain");
  for (size_t i = 0; i < op.inputs.size(); ++i)
    if (auto e = check_storage(t.inputs[i], "elementwise input")) return *e;
  if (auto e = check_storage(t.destinationTemplate, "elementwise destination")) return *e;

  DeviceBuffer p0(ctx), l0(ctx), p1(ctx), l1(ctx), dl(ctx);
  if (int st = upload_logical(ctx, t.inputs[0], p0, l0)) return from_status(st, "elementwise input 0");
  if (op.inputs.size() == 2)
    if (int st = upload_logical(ctx, t.inputs[1], p1, l1)) return from_status(st, "elementwise input 1");
  uint64_t first_in = count;
  for (size_t i = 0; i < op.inputs.size(); ++i) {
    Expected<uint64_t> f = first_nan(ctx, op.inputs[i], i == 0 ? l0.get() : l1.get());
    if (!f) return f.error();
    first_in = std::min(first_in, *f);
  }
  if (int st = dl.allocate(logical_bytes(op.destination))) return from_status(st, "elementwise destination");
  if (int st = wafer_hip_elementwise(ctx, (uint32_t)op.operation, (uint32_t)op.destination.getFormat(), l0.get(),
                                     op.inputs.size() == 2 ? l1.get() : nullptr, dl.get(), count))
    return from_status(st, "elementwise");
  Expected<uint64_t> first_out = first_nan(ctx, op.destination, dl.get());
  if (!first_out) return first_out.error();
  if (first_in < count && first_in <= *first_out) return managed("input value is outside the non-NaN domain");
  if (*first_out < count) return managed("result value is outside the non-NaN domain");
  TargetModelManagedReferenceResult res{TargetModelNumericTensor{op.destination, {}}, {}, {}};
  if (int st = pack_into_template(ctx, t.destinationTemplate, dl, res.destination.storage))
    return from_status(st, "elementwise pack");
  res.evidence.scalarEvaluations = count;  // TargetModelTensorNumeric.cpp:104-106
  res.evidence.environmentDigest = environment_digest(ctx);
  res.evidence.implementation = wafer_hip_implementation();
  return res;
}

// ---- convert --------------------------------------------------------------------------
// The managed convert (executeConvert, ManagedReferenceTargetModel.cpp:345-379):
// a served route whose formats match the descriptors, a NearestEven (or
// absent) parameter, F16/BF16/F32 endpoints of one shape and layout, and no
// NaN input.  Finite inputs cannot produce a NaN result on these routes.
Expected<TargetModelManagedReferenceResult>
HipTargetModelBackend::execute(const TargetModelConvertRequest &request, FormalNumericWorkBudget budget) const {
  const FormalConvertOperation &op = request.operation;
  const TargetModelNumericOperands &t = request.tensors;
  if (t.inputs.size() != 1 || !(t.destinationTemplate.key == op.destination))
    return managed("request tensor key does not match operation");
  if (!(t.inputs[0].key == op.source)) return managed("request input key does not match operation");
  const uint64_t count = op.destination.getElementCount();
  if (count > budget.getMaximumScalarEvaluations())
    return err(TargetModelKernelErrorCode::WorkBudgetExceeded, "convert: " + std::to_string(count) +
                                                                   " evaluations exceed the scalar budget");
  uint32_t src_fmt = 0, dst_fmt = 0;
  if (wafer_hip_convert_route(op.opcode, &src_fmt, &dst_fmt)) return managed("convert opcode is not a target route");
  if ((uint32_t)op.source.getFormat() != src_fmt || (uint32_t)op.destination.getFormat() != dst_fmt)
    return err(TargetModelKernelErrorCode::InvalidCommandField, "convert: descriptor formats differ from the route's");
  if (op.parameter && op.parameter->getRoundingMode() != TargetRoundingMode::NearestEven)
    return managed("convert is not nearest-even");
  if (!is_float(op.source.getFormat()) || !is_float(op.destination.getFormat()) ||
      op.source.getShape() != op.destination.getShape() || op.source.getLayout() != op.destination.getLayout())
    return managed("convert is outside the F16/BF16/F32 same-shape domain");
  if (auto e = check_storage(t.inputs[0], "convert source")) return *e;
  if (auto e = check_storage(t.destinationTemplate, "convert destination")) return *e;

  DeviceBuffer sp(ctx), sl(ctx), dl(ctx);
  if (int st = upload_logical(ctx, t.inputs[0], sp, sl)) return from_status(st, "convert source");
  Expected<uint64_t> first_in = first_nan(ctx, op.source, sl.get());
  if (!first_in) return first_in.error();
  if (*first_in < count) return managed("input value is outside the non-NaN domain");
  if (int st = dl.allocate(logical_bytes(op.destination))) return from_status(st, "convert destination");
  if (int st = wafer_hip_convert(ctx, op.opcode, (uint32_t)TargetRoundingMode::NearestEven, sl.get(), dl.get(), count))
    return from_status(st, "convert");
  TargetModelManagedReferenceResult res{TargetModelNumericTensor{op.destination, {}}, {}, {}};
  if (int st = pack_into_template(ctx, t.destinationTemplate, dl, res.destination.storage))
    return from_status(st, "convert pack");
  res.evidence.scalarEvaluations = count;  // TargetModelTensorNumeric.cpp:101-103
  res.evidence.environmentDigest = environment_digest(ctx);
  res.evidence.implementation = wafer_hip_implementation();
  return res;
}

// ---- reduce -----------------------------------------------------------------------------
Expected<TargetModelManagedReferenceResult>
HipTargetModelBackend::execute(const TargetModelReduceRequest &request, FormalNumericWorkBudget budget) const {
  const FormalReduceOperation &op = request.operation;
  const TargetModelNumericOperands &t = request.tensors;
  if (t.inputs.size() != 1 || !(t.destinationTemplate.key == op.destination))
    return managed("request tensor key does not match operation");
  if (!(t.inputs[0].key == op.input)) return managed("request input key does not match operation");
  const uint64_t evaluations = op.input.getElementCount();  // TargetModelTensorNumeric.cpp:107-109
  if (evaluations > budget.getMaximumScalarEvaluations())
    return err(TargetModelKernelErrorCode::WorkBudgetExceeded, "reduce: " + std::to_string(evaluations) +
                                                                   " evaluations exceed the scalar budget");
  // executeReduce's domain (ManagedReferenceTargetModel.cpp:382-397)
  const LogicalFormat fmt = op.input.getFormat();
  if ((op.operation != TargetReduceOperation::Sum && op.operation != TargetReduceOperation::Max &&
       op.operation != TargetReduceOperation::Min) ||
      !is_float(fmt) || op.destination.getFormat() != fmt ||
      (op.operation == TargetReduceOperation::Sum && fmt != LogicalFormat::F32))
    return managed("reduce requires F32 sum or F16/BF16/F32 max/min");
  if (auto e = check_storage(t.inputs[0], "reduce input")) return *e;
  if (auto e = check_storage(t.destinationTemplate, "reduce destination")) return *e;

  DeviceBuffer ip(ctx), il(ctx), dl(ctx);
  if (int st = upload_logical(ctx, t.inputs[0], ip, il)) return from_status(st, "reduce input");
  // NaN inputs are refused as they are decoded; with finite inputs only a
  // Sum can leave the domain (+inf + -inf), which the reference reports as
  // the accumulator leaving it.  (With both present the reference reports
  // whichever its input order meets first; here a NaN input always wins.)
  {
    Expected<uint64_t> f = first_nan(ctx, op.input, il.get());
    if (!f) return f.error();
    if (*f < evaluations) return managed("input value is outside the non-NaN domain");
  }
  if (int st = dl.allocate(logical_bytes(op.destination))) return from_status(st, "reduce destination");
  const std::vector<int64_t> s = shape64(op.input);
  // the kernel checks the reduced shape against the destination's element
  // count through its own geometry; compare here as well so a mismatch fails
  // before any launch
  {
    // reduced dims of TargetReduceDimension (Trailing0..3, Trailing2And1, Trailing2And1And0)
    std::vector<uint64_t> r(op.input.getShape());
    const size_t rank = r.size();
    auto drop = [&](size_t trailing) { if (trailing < rank) r[rank - 1 - trailing] = 1; };
    switch (op.dimension) {
    case TargetReduceDimension::Trailing0: drop(0); break;
    case TargetReduceDimension::Trailing1: drop(1); break;
    case TargetReduceDimension::Trailing2: drop(2); break;
    case TargetReduceDimension::Trailing3: drop(3); break;
    case TargetReduceDimension::Trailing2And1: drop(2); drop(1); break;
    case TargetReduceDimension::Trailing2And1And0: drop(2); drop(1); drop(0); break;
    }
    uint64_t n = 1;
    for (uint64_t e : r) n *= e;
    if (n != op.destination.getElementCount())
      return err(TargetModelKernelErrorCode::InvalidCommandField, "reduce: destination does not hold the reduced shape");
  }
  if (int st = wafer_hip_reduce(ctx, (uint32_t)op.operation, (uint32_t)op.dimension, (uint32_t)op.input.getFormat(),
                                s.data(), (uint32_t)s.size(), il.get(), dl.get()))
    return from_status(st, "reduce");
  {
    Expected<uint64_t> f = first_nan(ctx, op.destination, dl.get());
    if (!f) return f.error();
    if (*f < op.destination.getElementCount()) return managed("reduce accumulator left the non-NaN domain");
  }
  TargetModelManagedReferenceResult res{TargetModelNumericTensor{op.destination, {}}, {}, {}};
  if (int st = pack_into_template(ctx, t.destinationTemplate, dl, res.destination.storage))
    return from_status(st, "reduce pack");
  res.evidence.scalarEvaluations = evaluations;
  res.evidence.environmentDigest = environment_digest(ctx);
  res.evidence.implementation = wafer_hip_implementation();
  return res;
}

}  // namespace wafer::model
