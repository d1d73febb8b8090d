// An ExecutionPlan binds one ConvProblem to one concrete kernel and owns all one-time setup (capability check,
// device tables). Creating a plan may allocate and synchronize; execute() only launches work.
// (The reference's include/gpu_inference/execution_plan.h, on HIP streams/events.)
#pragma once

#include <hip/hip_runtime_api.h>

#include <memory>

#include "gpu_inference/kernel_registry.h"

namespace gie {

class ExecutionPlan {
 public:
  // Throws gie::Error(kUnsupported) if `kernel` cannot run `problem` on the device.
  static std::shared_ptr<ExecutionPlan> create(const ConvProblem& problem, const KernelDesc& kernel, int device = -1);
  ~ExecutionPlan();
  ExecutionPlan(const ExecutionPlan&) = delete;
  ExecutionPlan& operator=(const ExecutionPlan&) = delete;

  // Validates arguments (shapes, dtypes, null pointers, aliasing, workspace size) and launches asynchronously
  // on `stream`. Never synchronizes the device.
  // stage_events: optional, three events recorded around the repack and convolution stages (LaunchArgs).
  void execute(const ConstTensorRef& x, const ConstTensorRef& w, const ConstTensorRef* bias, const TensorRef& y,
               void* workspace, size_t workspace_bytes, hipStream_t stream, hipEvent_t* stage_events = nullptr,
               int only_stage = -1) const;

  // Raw-pointer fast path: arguments were validated once by the caller (timing loops, graph capture).
  void execute_unchecked(const void* x, const void* w, const void* bias, void* y, void* workspace,
                         size_t workspace_bytes, hipStream_t stream, hipEvent_t* stage_events = nullptr,
                         int only_stage = -1) const;

  const ConvProblem& problem() const { return problem_; }
  const KernelDesc& kernel() const { return *kernel_; }
  size_t workspace_bytes() const { return workspace_bytes_; }
  size_t persistent_bytes() const { return persistent_bytes_ + lut_bytes_; }  // plan-owned, the gather table included
  size_t lut_bytes() const { return lut_bytes_; }                             // 0 unless the kernel sets needs_lut
  int device() const { return device_; }

 private:
  ExecutionPlan() = default;
  ConvProblem problem_;
  const KernelDesc* kernel_ = nullptr;
  int device_ = 0;
  size_t workspace_bytes_ = 0;
  size_t persistent_bytes_ = 0;
  DeviceBuffer lut_;  // device copy of the gather table (needs_lut kernels)
  size_t lut_bytes_ = 0;
  size_t x_bytes_ = 0, w_bytes_ = 0, y_bytes_ = 0, bias_bytes_ = 0;  // operand footprints, for the alias checks
  LaunchArgs proto_;  // everything but the pointers and the stream, filled once by create()
  std::shared_ptr<void> state_;
};

}  // namespace gie
