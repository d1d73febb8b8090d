// Deterministic synthetic data and device-buffer helpers for tests, the autotuner and the benchmark
// (the reference's include/gpu_inference/testing.h).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "gpu_inference/conv2d.h"
#include "gpu_inference/reference.h"

namespace gie {

// SplitMix64: seeds reproduce identical data on every platform.
class Rng {
 public:
  explicit Rng(uint64_t seed) : s_(seed) {}
  uint64_t next_u64();
  double uniform();  // [0, 1)
  float uniform(float lo, float hi);
  float normal();    // Irwin-Hall (sum of 12 uniforms - 6)

 private:
  uint64_t s_;
};

enum class Distribution { kUniform, kNormal, kSparseSigned, kPositive };
const char* to_string(Distribution d);

// kReference: weights * sqrt(3/K), bias ~ U(-1,1) (the reference's make_conv_data);
// kBenchmark: weights * 1/sqrt(K), bias ~ U(-0.1,0.1) (the benchmark configurations).
enum class Scaling { kReference, kBenchmark };

struct ConvData {
  ConvProblem prob;
  std::vector<float> hx, hw, hb;  // values the reference consumes (quantized)
  DeviceBuffer dx, dw, db, dy;    // device tensors in the storage dtype

  ConstTensorRef x_ref() const;
  ConstTensorRef w_ref() const;
  ConstTensorRef b_ref() const;
  TensorRef y_ref();
};

// The seeded values of make_conv_data with no device work (same draw order and quantization): what the
// reference consumes, and for kTf32 the unrounded FP32 values the device receives (raw_x, raw_w; empty otherwise).
struct HostConvData {
  std::vector<float> hx, hw, hb;
  std::vector<float> raw_x, raw_w;
};
HostConvData make_host_conv_data(const ConvProblem& prob, uint64_t seed, Distribution dist = Distribution::kUniform,
                                 Scaling scaling = Scaling::kReference);

ConvData make_conv_data(const ConvProblem& prob, uint64_t seed, Distribution dist = Distribution::kUniform,
                        Scaling scaling = Scaling::kReference);
DeviceBuffer upload_as(const std::vector<float>& v, DataType dt);

}  // namespace gie
