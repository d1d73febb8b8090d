// GPU capability and peak-rate queries (the reference's include/gpu_inference/device_info.h on HIP).
//
// Peaks are spec-derived estimates (CU count x clock x per-architecture throughput; HBM from the product
// table), not measurements; perf_model.h's measure_ceilings() gives measured ones. Field names follow the
// reference: `sm_count` is the compute-unit count, `warp_size` the wavefront width (64 on CDNA),
// `smem_*` the LDS limits.
#pragma once

#include <hip/hip_runtime_api.h>

#include <string>

namespace gie {

struct DeviceInfo {
  int device = 0;
  std::string name;
  std::string gcn_arch;  // e.g. "gfx950:sramecc+:xnack-"
  int cc_major = 0, cc_minor = 0;
  int sm_count = 0;  // compute units
  size_t global_mem_bytes = 0;
  size_t l2_bytes = 0;
  size_t smem_per_block_default = 0;  // LDS per workgroup without opt-in
  size_t smem_per_block_optin = 0;    // LDS per workgroup with hipFuncAttributeMaxDynamicSharedMemorySize
  size_t smem_per_sm = 0;             // LDS per CU
  int regs_per_sm = 0;
  int max_threads_per_sm = 0;
  int max_threads_per_block = 0;
  int max_blocks_per_sm = 0;
  int warp_size = 64;
  int max_sm_clock_khz = 0;
  int mem_clock_khz = 0;
  int mem_bus_bits = 0;
  int driver_version = 0;
  int runtime_version = 0;

  int cc() const { return cc_major * 10 + cc_minor; }
  bool is_gfx950() const { return gcn_arch.rfind("gfx950", 0) == 0; }
  // Matrix-core (MFMA) availability of the element types this library's kernels use.
  bool supports_fp16_tensor_cores() const;
  bool supports_bf16_tensor_cores() const;
  bool supports_tf32_tensor_cores() const { return false; }  // gfx950 has no xf32 MFMA
  bool supports_cp_async() const { return is_gfx950(); }     // direct global->LDS loads

  // Theoretical estimates (TFLOP/s, GB/s) -- NOT measurements.
  double est_peak_fp32_tflops() const;
  double est_peak_fp16_tc_tflops() const;  // dense MFMA, FP32 accumulate
  double est_peak_bw_gbs() const;

  std::string describe() const;

  // Queried once per device and cached (thread-safe).
  static const DeviceInfo& get(int device);
  static const DeviceInfo& current();
};

}  // namespace gie
