// Conv2D::forward / workspace_size / clear_plan_cache over a process-global plan cache
// (the reference's conv2d.cpp:113-164: PlanKey, selection outside the lock, first insert wins).
#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <mutex>
#include <tuple>

#include "gpu_inference/conv2d.h"
#include "gpu_inference/dispatcher.h"
#include "gpu_inference/execution_plan.h"

namespace gie {
namespace {

struct PlanKey {
  std::string problem, backend, kernel;
  int device;
  bool autotune, retune;
  std::string cache;
  bool operator<(const PlanKey& o) const {
    return std::tie(problem, backend, kernel, device, autotune, retune, cache) <
           std::tie(o.problem, o.backend, o.kernel, o.device, o.autotune, o.retune, o.cache);
  }
};

std::mutex g_plan_mu;
std::map<PlanKey, std::shared_ptr<ExecutionPlan>>& plan_cache() {
  static std::map<PlanKey, std::shared_ptr<ExecutionPlan>> c;
  return c;
}

std::shared_ptr<ExecutionPlan> get_plan(const ConvProblem& prob, const Conv2DOptions& opt) {
  validate_problem(prob);
  int dev = 0;
  GIE_HIP_CHECK(hipGetDevice(&dev));
  PlanKey key{prob.key(), to_string(opt.backend), opt.kernel, dev, opt.autotune, opt.force_retune, opt.cache_path};
  {
    std::lock_guard<std::mutex> lock(g_plan_mu);
    auto it = plan_cache().find(key);
    if (it != plan_cache().end()) return it->second;
  }
  const DeviceInfo& di = DeviceInfo::get(dev);
  Selection sel = Dispatcher::select(prob, di, opt);
  std::shared_ptr<ExecutionPlan> plan = ExecutionPlan::create(prob, *sel.kernel, dev);
  std::lock_guard<std::mutex> lock(g_plan_mu);
  return plan_cache().emplace(key, plan).first->second;
}

}  // namespace

void Conv2D::forward(const ConstTensorRef& input, const ConstTensorRef& weights, const ConstTensorRef* bias,
                     const ConvProblem& problem, const TensorRef& output, void* workspace, size_t workspace_bytes,
                     hipStream_t stream, const Conv2DOptions& options) {
  auto plan = get_plan(problem, options);
  plan->execute(input, weights, bias, output, workspace, workspace_bytes, stream);
}

size_t Conv2D::workspace_size(const ConvProblem& problem, const Conv2DOptions& options) {
  return get_plan(problem, options)->workspace_bytes();
}

void Conv2D::clear_plan_cache() {
  std::lock_guard<std::mutex> lock(g_plan_mu);
  plan_cache().clear();
}

}  // namespace gie
