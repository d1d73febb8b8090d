// ExecutionPlan (the role of src/runtime/execution_plan.cpp:40-138): everything that depends only on the problem
// and the kernel is settled once in create() — capability check on the plan's device, workspace and persistent
// sizes, per-plan kernel state, the gather table of a needs_lut kernel (built on the host, uploaded on a private
// stream and waited for, so a capture running on another stream sees no foreign work), the operand footprints and
// a LaunchArgs record with every field but the pointers and the stream — so execute() checks the caller's tensors
// against precomputed values and execute_unchecked() copies that record, fills in five pointers and enqueues.
// Neither allocates or synchronizes.
#include "gpu_inference/execution_plan.h"

#include <hip/hip_runtime.h>

#include <string>

#include "gpu_inference/roctx.h"

namespace gie {
namespace {

// Makes `device` current for the lifetime of the scope and restores the caller's device afterwards.
class DeviceScope {
 public:
  explicit DeviceScope(int device) {
    GIE_HIP_CHECK(hipGetDevice(&saved_));
    if (saved_ != device) GIE_HIP_CHECK(hipSetDevice(device));
  }
  ~DeviceScope() { (void)hipSetDevice(saved_); }
  DeviceScope(const DeviceScope&) = delete;
  DeviceScope& operator=(const DeviceScope&) = delete;

 private:
  int saved_ = 0;
};

// Half-open byte ranges [a, a + an) and [b, b + bn) share a byte (empty or null ranges share none).
bool ranges_meet(const void* a, size_t an, const void* b, size_t bn) {
  if (a == nullptr || b == nullptr || an == 0 || bn == 0) return false;
  const uintptr_t lo_a = reinterpret_cast<uintptr_t>(a), lo_b = reinterpret_cast<uintptr_t>(b);
  return lo_a < lo_b + bn && lo_b < lo_a + an;
}

[[noreturn]] void bad_argument(const std::string& msg) { throw Error(StatusCode::kInvalidArgument, msg); }

// Host-to-device copy that has completed on return, issued on a stream of its own (non-blocking, so it neither
// waits for nor joins work on the legacy stream).
void upload_now(void* dst, const void* src, size_t bytes) {
  hipStream_t s = nullptr;
  GIE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  const hipError_t copied = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s);
  const hipError_t waited = copied == hipSuccess ? hipStreamSynchronize(s) : copied;
  (void)hipStreamDestroy(s);
  GIE_HIP_CHECK(waited);
}

// One operand against what the plan expects of it: a device pointer, the precision policy's storage type and the
// problem's shape, in that order.
void expect_operand(const char* role, const void* data, DataType dtype, const TensorShape& shape, DataType want_dtype,
                    const TensorShape& want_shape) {
  if (data == nullptr) bad_argument(std::string(role) + " has no device pointer");
  if (dtype != want_dtype)
    bad_argument(std::string(role) + " is " + to_string(dtype) + "; this problem stores " + to_string(want_dtype));
  if (shape != want_shape)
    bad_argument(std::string(role) + " has shape " + shape.to_string() + "; this problem needs " +
                 want_shape.to_string());
}

}  // namespace

std::shared_ptr<ExecutionPlan> ExecutionPlan::create(const ConvProblem& problem, const KernelDesc& kernel, int device) {
  RoctxRange range("gie::ExecutionPlan::create");
  validate_problem(problem);
  if (device < 0) GIE_HIP_CHECK(hipGetDevice(&device));
  DeviceScope scope(device);
  const DeviceInfo& dev = DeviceInfo::get(device);
  std::string why;
  if (!kernel.supports(problem, dev, &why))
    throw Error(StatusCode::kUnsupported,
                kernel.name + " does not run " + problem.key() + " on " + dev.name + " (" + dev.gcn_arch + "): " + why);

  std::shared_ptr<ExecutionPlan> plan(new ExecutionPlan());
  ExecutionPlan& pl = *plan;
  pl.problem_ = problem;
  pl.kernel_ = &kernel;
  pl.device_ = device;
  pl.workspace_bytes_ = kernel.workspace_bytes(problem);
  pl.persistent_bytes_ = kernel.persistent_bytes ? kernel.persistent_bytes(problem) : 0;
  if (kernel.create_state) pl.state_ = kernel.create_state(problem);
  if (kernel.needs_lut) {
    const std::vector<LutEntry> table =
        kernel.lut_chunked ? build_conv_lut_chunked(problem.p) : build_conv_lut(problem.p);
    pl.lut_bytes_ = table.size() * sizeof(LutEntry);
    pl.lut_ = DeviceBuffer(pl.lut_bytes_);
    upload_now(pl.lut_.data(), table.data(), pl.lut_bytes_);
  }
  const Conv2DParams& p = problem.p;
  const size_t es = dtype_size(problem.dtype());
  pl.x_bytes_ = size_t(p.input_shape().numel()) * es;
  pl.w_bytes_ = size_t(p.weight_shape().numel()) * es;
  pl.y_bytes_ = size_t(p.output_shape().numel()) * es;
  pl.bias_bytes_ = problem.has_bias ? size_t(p.out_channels) * es : 0;
  pl.proto_.problem = &pl.problem_;
  pl.proto_.dev = &dev;
  pl.proto_.plan_state = pl.state_.get();
  pl.proto_.plan_data = pl.lut_.data();
  return plan;
}

ExecutionPlan::~ExecutionPlan() = default;

void ExecutionPlan::execute(const ConstTensorRef& x, const ConstTensorRef& w, const ConstTensorRef* bias,
                            const TensorRef& y, void* workspace, size_t workspace_bytes, hipStream_t stream,
                            hipEvent_t* stage_events, int only_stage) const {
  const Conv2DParams& p = problem_.p;
  const DataType dt = problem_.dtype();
  expect_operand("input x", x.data, x.dtype, x.shape, dt, p.input_shape());
  expect_operand("weights w", w.data, w.dtype, w.shape, dt, p.weight_shape());
  expect_operand("output y", y.data, y.dtype, y.shape, dt, p.output_shape());
  const bool bias_given = bias != nullptr && bias->data != nullptr;
  if (problem_.has_bias && bias == nullptr) bad_argument("the problem adds a bias but no bias tensor was passed");
  if (!problem_.has_bias && bias_given) bad_argument("a bias tensor was passed but the problem adds no bias");
  const void* b = nullptr;
  if (problem_.has_bias) {
    expect_operand("bias", bias->data, bias->dtype, bias->shape, dt, p.bias_shape());
    b = bias->data;
  }

  // y is written while x, w and bias are read: no in-place convolution
  if (ranges_meet(y.data, y_bytes_, x.data, x_bytes_) || ranges_meet(y.data, y_bytes_, w.data, w_bytes_) ||
      ranges_meet(y.data, y_bytes_, b, bias_bytes_))
    bad_argument("output y overlaps an input (in-place convolution is not supported)");

  if (workspace_bytes_ > 0) {
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
      bad_argument("workspace must start on a 256-byte boundary (its buffers take 16-byte vector accesses)");
    if (workspace == nullptr || workspace_bytes < workspace_bytes_)
      throw Error(StatusCode::kWorkspaceTooSmall, kernel_->name + " needs " + std::to_string(workspace_bytes_) +
                                                      " workspace bytes; " + std::to_string(workspace_bytes) +
                                                      " were given");
    if (ranges_meet(workspace, workspace_bytes_, x.data, x_bytes_) ||
        ranges_meet(workspace, workspace_bytes_, w.data, w_bytes_) ||
        ranges_meet(workspace, workspace_bytes_, y.data, y_bytes_))
      bad_argument("workspace overlaps a tensor");
  }
  int current = 0;
  GIE_HIP_CHECK(hipGetDevice(&current));
  if (current != device_)
    bad_argument("plan belongs to device " + std::to_string(device_) + " but device " + std::to_string(current) +
                 " is current");
  execute_unchecked(x.data, w.data, b, y.data, workspace, workspace_bytes, stream, stage_events, only_stage);
}

void ExecutionPlan::execute_unchecked(const void* x, const void* w, const void* bias, void* y, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream, hipEvent_t* stage_events,
                                      int only_stage) const {
  RoctxRange range(kernel_->name.c_str());
  LaunchArgs la = proto_;
  la.x = x;
  la.w = w;
  la.bias = problem_.has_bias ? bias : nullptr;
  la.y = y;
  la.workspace = workspace;
  la.workspace_bytes = workspace_bytes;
  la.stream = stream;
  la.stage_events = stage_events;
  la.only_stage = only_stage;
  kernel_->launch(la);
}

}  // namespace gie
