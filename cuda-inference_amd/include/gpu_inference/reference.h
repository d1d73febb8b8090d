// Reference convolutions and error metrics (the reference's include/gpu_inference/reference.h).
//
// Reference precision policy:
//  * the reference consumes exactly the values the kernel consumes (inputs quantized to the storage type);
//  * products and sums accumulate in double; bias is added, ReLU applied, then one rounding to float;
//  * alongside y it emits scale[i] = sqrt(sum_k (x_k*w_k)^2 + (sum_k x_k*w_k)^2 + bias^2), the magnitude the
//    tolerance model scales with.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>
#include <vector>

#include "gpu_inference/conv2d.h"

namespace gie {

struct ReferenceOutput {
  std::vector<float> y;
  std::vector<float> scale;
};

// Nested-loop CPU implementation (double accumulation, OpenMP over outputs).
void cpu_conv2d_reference(const ConvProblem& prob, const float* x, const float* w, const float* bias,
                          ReferenceOutput* out);

// GPU reference with double accumulation (one thread per output) reading the same device tensors the
// optimized kernels read. d_y / d_scale are float[numel(Y)].
void gpu_conv2d_reference(const ConvProblem& prob, const void* x, const void* w, const void* bias, float* d_y,
                          float* d_scale, hipStream_t stream);

// |err_i| <= c_acc*u_acc*sqrt(K)*scale_i + c_out*u_out*|ref_i| + c_inter*u_out*scale_i + c_in*u_in*scale_i + floor
struct TolerancePolicy {
  double c_acc = 8.0;
  double c_out = 1.0;
  double c_inter = 0.0;
  double c_in = 0.0;
  double u_in = 0.00048828125;
  double u_acc = 5.9604644775390625e-08;
  double u_out = 5.9604644775390625e-08;
  double abs_floor = 1e-30;
  int64_t k = 1;
  static TolerancePolicy for_problem(const ConvProblem& prob, bool intermediate_rounding = false);
  double tol(double ref, double scale) const;
  std::string describe() const;
};

struct ErrorMetrics {
  int64_t n = 0;
  double max_abs = 0, mean_abs = 0, rms = 0;
  double max_rel = 0;
  double frac_over_tol = 0;
  int64_t over_tol = 0, nan_count = 0, inf_count = 0;
  double worst_tol_ratio = 0;
  double rel_l2 = 0;  // ||test - ref|| / ||ref|| (benchmark gate)
  bool passed() const { return n > 0 && nan_count == 0 && inf_count == 0 && over_tol == 0; }
  std::string summary() const;
};

ErrorMetrics compare_outputs(const float* test, const float* ref, const float* scale, int64_t n,
                             const TolerancePolicy& tol);

float quantize_to(Precision p, float v);
float round_to_tf32(float v);
uint16_t float_to_half_bits(float v);
uint16_t float_to_bf16_bits(float v);
float half_bits_to_float(uint16_t h);
float bf16_bits_to_float(uint16_t h);
std::vector<float> download_as_float(const void* d_ptr, DataType dt, int64_t n);

}  // namespace gie
