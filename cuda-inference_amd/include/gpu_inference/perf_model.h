// Roofline-style analytical performance model (the reference's include/gpu_inference/perf_model.h), with
// MI355X ceilings: dense FP16/BF16 MFMA, HBM3E bandwidth and the measured launch cost.
//
// FLOP counts are exact; byte counts are compulsory-traffic lower bounds; time estimates use theoretical
// (DeviceInfo) or measured (measure_ceilings) ceilings. The model ranks/prunes autotuning candidates only.
#pragma once

#include <map>
#include <string>

#include "gpu_inference/kernel_registry.h"

namespace gie {

struct DeviceCeilings {
  double fp32_tflops = 0;     // vector FP32 FMA ceiling
  double fp16_tc_tflops = 0;  // dense FP16 MFMA ceiling
  double bw_gbs = 0;          // achievable HBM bandwidth
  double launch_overhead_us = 4.0;
  bool measured = false;
  std::string source;
};

DeviceCeilings theoretical_ceilings(const DeviceInfo& dev);
// Runs (or loads cached) microbenchmarks on `device`; cached in $GIE_CEILING_DIR (default
// ~/.cache/gpu_inference). Allocates ~1 GiB briefly.
DeviceCeilings measure_ceilings(int device, bool use_cache = true);
bool load_cached_ceilings(int device, DeviceCeilings* out);

enum class Bound { kCompute, kBandwidth, kLaunch };
const char* to_string(Bound b);

struct ProblemModel {
  double flops = 0;
  double input_bytes = 0, weight_bytes = 0, output_bytes = 0, bias_bytes = 0;
  double compulsory_bytes = 0;       // read X, W, bias once + write Y once
  double im2col_bytes = 0;           // size of an explicit unrolled matrix
  double im2col_extra_traffic = 0;   // write + read of that matrix
  double unfused_extra_traffic = 0;  // extra read+write of Y per separate elementwise op
  double arithmetic_intensity = 0;   // flops / compulsory_bytes
  double unrolled_blowup = 0;
};
ProblemModel analyze_problem(const ConvProblem& prob);

struct Estimate {
  double time_us = 0;
  double compute_us = 0, memory_us = 0, launch_us = 0;
  Bound bound = Bound::kCompute;
  double tile_efficiency = 1.0;
  double wave_efficiency = 1.0;  // workgroup load balance over CUs
  int blocks_per_sm = 0;
};

Estimate roofline_estimate(const ConvProblem& prob, const DeviceCeilings& c, bool tensor_cores);
Estimate estimate_kernel(const ConvProblem& prob, const KernelDesc& k, const DeviceInfo& dev,
                         const DeviceCeilings& c);
double backend_efficiency_prior(const KernelDesc& k);

void set_model_calibration(const std::map<std::string, double>& scale_by_backend);
std::map<std::string, double> get_model_calibration();

}  // namespace gie
