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
  const void* plan_data = nullptr;  // device copy of the plan's gather table when the kernel sets needs_lut
  void* plan_state = nullptr;       // opaque per-plan state created by KernelDesc::create_state
  hipStream_t stream = nullptr;
  // Optional stage events (the reference's hook): families with a repack stage record events[0] before it,
  // events[1] after it and events[2] after the convolution (before any split-K reduce).
  hipEvent_t* stage_events = nullptr;
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
  bool needs_lut = false;    // the plan builds the gather table (build_conv_lut*) and passes it as plan_data
  bool lut_chunked = false;  // ... one entry per 8 consecutive k (build_conv_lut_chunked, C % 8 == 0)
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

// Records stage event i of a full launch when the caller passed stage events (LaunchArgs::stage_events).
inline void record_stage_event(const LaunchArgs& la, int i) {
  if (la.stage_events != nullptr && la.only_stage < 0) GIE_HIP_CHECK(hipEventRecord(la.stage_events[i], la.stream));
}

const std::vector<KernelDesc>& kernel_registry();
// TESTING ONLY: mutable access so tests can inject deliberately faulty kernels.
std::vector<KernelDesc>& kernel_registry_for_testing();
const KernelDesc* find_kernel(const std::string& name);
std::vector<const KernelDesc*> kernels_for_backend(Backend b);

// Gather table for implicit-GEMM kernels that walk the reduction index k in (c, r, s) order (the reference's
// kernel_registry.h:86-96 format, 16 bytes per entry). No kernel of this library reads one — every family here
// keeps its tap offsets in registers — but a kernel registered with needs_lut gets it built and uploaded once per
// plan, as in the reference.
struct alignas(16) LutEntry {
  int32_t c_off;  // channel displacement: c * H * W elements (per k), 8 * chunk elements (chunked)
  int32_t r_off;  // filter-row displacement r * dilation_h
  int32_t s_off;  // filter-column displacement s * dilation_w
  int32_t pad_;   // zero
};
// One entry per k = (c * KH + r) * KW + s, k < C * KH * KW.
std::vector<LutEntry> build_conv_lut(const Conv2DParams& p);
// One entry per chunk q of 8 consecutive k in tap-major order (q = (r * KW + s) * C/8 + c/8); C % 8 == 0 or it
// throws kInvalidArgument.
std::vector<LutEntry> build_conv_lut_chunked(const Conv2DParams& p);

}  // namespace gie
