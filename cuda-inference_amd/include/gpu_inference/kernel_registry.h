// Registry of concrete kernel implementations ("candidates") — the reference's operator-plugin record
// (include/gpu_inference/kernel_registry.h:26-82) with the same fields and function-pointer contract.
//
// Every launchable kernel configuration is one KernelDesc. The dispatcher filters the registry by capability,
// the cost model ranks it and the autotuner measures it. `launch` must not allocate, free or synchronize:
// it only enqueues work through the kernel C-ABI (include/gie_hip.h), so it can be captured into a hipGraph.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "gpu_inference/conv2d.h"
#include "gpu_inference/device_info.h"

namespace gie {

// Bump when kernel behaviour changes in a way that invalidates tuning results.
constexpr int kLibraryVersion = 1;

struct LaunchArgs {
  const ConvProblem* problem = nullptr;
  const DeviceInfo* dev = nullptr;
  const void* x = nullptr;
  const void* w = nullptr;
  const void* bias = nullptr;  // nullptr when !problem->has_bias
  void* y = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  void* plan_state = nullptr;       // opaque per-plan state created by KernelDesc::create_state
  hipStream_t stream = nullptr;
  // Profiling hook: >= 0 launches only that stage of a multi-launch kernel (0 = repack, 1 = main kernel,
  // 2 = split-K reduce) on a workspace a full launch has already filled; every stage is idempotent, so
  // back-to-back launches of one stage time that kernel alone. -1 (default) launches the whole chain.
  int only_stage = -1;
};

struct KernelDesc {
  std::string name;  // unique, stable; used in caches and result files
  Backend backend = Backend::kDirect;
  int version = 1;  // bump when this kernel's code changes behaviour/performance
  std::vector<std::pair<std::string, int>> params;  // tile/launch parameters
  int threads_per_block = 0;

  // Tile extents in the implicit-GEMM view (M = C_out, N = B*Ho*Wo, K = C_in*Kh*Kw).
  int tile_m = 1, tile_n = 1, tile_k = 1;
  bool uses_tensor_cores = false;  // matrix cores (MFMA)
  int launches = 1;             // kernel launches per forward call (cost model)
  double efficiency_prior = 0;  // compute-ceiling fraction for a family the cost model has no measured profile of
  double (*extra_traffic_bytes)(const ConvProblem&) = nullptr;  // DRAM bytes beyond compulsory X/W/Y
  const void* function = nullptr;  // primary __global__ function, may be null (occupancy via blocks_per_cu)

  bool (*supports)(const ConvProblem&, const DeviceInfo&, std::string* why) = nullptr;
  size_t (*workspace_bytes)(const ConvProblem&) = nullptr;     // per-call temporary memory
  size_t (*dynamic_smem_bytes)(const ConvProblem&) = nullptr;  // LDS per workgroup
  int64_t (*num_blocks)(const ConvProblem&) = nullptr;         // workgroups of the main kernel
  double (*tile_efficiency)(const ConvProblem&) = nullptr;
  std::shared_ptr<void> (*create_state)(const ConvProblem&) = nullptr;
  size_t (*persistent_bytes)(const ConvProblem&) = nullptr;
  void (*launch)(const LaunchArgs&) = nullptr;
  // Resident workgroups per CU of the main kernel (MI355X-specific addition; null -> 1).
  int (*blocks_per_cu)(const ConvProblem&) = nullptr;

  std::string describe() const;
};

const std::vector<KernelDesc>& kernel_registry();
// TESTING ONLY: mutable access so tests can inject deliberately faulty kernels.
std::vector<KernelDesc>& kernel_registry_for_testing();
const KernelDesc* find_kernel(const std::string& name);
std::vector<const KernelDesc*> kernels_for_backend(Backend b);

}  // namespace gie
