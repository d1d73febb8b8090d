// hipGraph capture/replay of a sequence of asynchronous launches (typically a chain of
// ExecutionPlan::execute_unchecked calls) — the reference's CudaGraphExecutor (cuda_graph.h) on HIP graphs.
// Graphs remove per-launch host cost and inter-kernel gaps for small, launch-bound layers.
#pragma once

#include <hip/hip_runtime_api.h>

#include <functional>

#include "gpu_inference/error.h"

namespace gie {

class HipGraphExecutor {
 public:
  using Enqueue = std::function<void(hipStream_t)>;  // must not allocate, synchronize or memset

  HipGraphExecutor() = default;
  ~HipGraphExecutor();
  HipGraphExecutor(const HipGraphExecutor&) = delete;
  HipGraphExecutor& operator=(const HipGraphExecutor&) = delete;

  // Runs `enqueue` once eagerly (lazy initialization is illegal during capture), then captures and instantiates.
  void capture(const Enqueue& enqueue);
  // Re-captures and updates the executable graph in place when the topology is unchanged; else re-instantiates.
  // Returns true if updated in place.
  bool recapture_update(const Enqueue& enqueue);
  void launch(hipStream_t stream) const;
  // Uploads the executable graph's device-side state on `stream` ahead of the first launch (hipGraphUpload), so
  // that launch does not pay for it. Addition to the reference's interface.
  void upload(hipStream_t stream) const;

  bool valid() const { return exec_ != nullptr; }
  size_t node_count() const { return nodes_; }
  double capture_us() const { return capture_us_; }
  double instantiate_us() const { return instantiate_us_; }

 private:
  void adopt(hipGraph_t g, double capture_us);  // instantiates g as the executable graph, taking ownership of it
  void reset();
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t exec_ = nullptr;
  size_t nodes_ = 0;
  double capture_us_ = 0, instantiate_us_ = 0;
};

}  // namespace gie
