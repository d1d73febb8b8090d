// Seeded synthetic data (the reference's testing.cu: SplitMix64, draw order x -> w -> bias, quantize to the
// storage type, poison y with NaN bits) plus the benchmark scaling of BASELINE's configurations.
#include "gpu_inference/testing.h"

#include <hip/hip_runtime.h>

#include <cmath>

namespace gie {

uint64_t Rng::next_u64() {
  uint64_t z = (s_ += 0x9e3779b97f4a7c15ULL);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}
double Rng::uniform() { return double(next_u64() >> 11) * (1.0 / 9007199254740992.0); }
float Rng::uniform(float lo, float hi) { return lo + float(uniform()) * (hi - lo); }
float Rng::normal() {
  double s = 0;
  for (int i = 0; i < 12; ++i) s += uniform();
  return float(s - 6.0);
}

const char* to_string(Distribution d) {
  switch (d) {
    case Distribution::kUniform: return "uniform";
    case Distribution::kNormal: return "normal";
    case Distribution::kSparseSigned: return "sparse_signed";
    case Distribution::kPositive: return "positive";
  }
  return "?";
}

ConstTensorRef ConvData::x_ref() const { return {dx.data(), prob.dtype(), prob.p.input_shape()}; }
ConstTensorRef ConvData::w_ref() const { return {dw.data(), prob.dtype(), prob.p.weight_shape()}; }
ConstTensorRef ConvData::b_ref() const { return {db.data(), prob.dtype(), prob.p.bias_shape()}; }
TensorRef ConvData::y_ref() { return {dy.data(), prob.dtype(), prob.p.output_shape()}; }

DeviceBuffer upload_as(const std::vector<float>& v, DataType dt) {
  DeviceBuffer buf(v.size() * dtype_size(dt));
  if (dt == DataType::kFloat32) {
    GIE_HIP_CHECK(hipMemcpy(buf.data(), v.data(), v.size() * 4, hipMemcpyHostToDevice));
  } else {
    std::vector<uint16_t> raw(v.size());
    for (size_t i = 0; i < v.size(); ++i)
      raw[i] = dt == DataType::kFloat16 ? float_to_half_bits(v[i]) : float_to_bf16_bits(v[i]);
    GIE_HIP_CHECK(hipMemcpy(buf.data(), raw.data(), raw.size() * 2, hipMemcpyHostToDevice));
  }
  return buf;
}

namespace {
float draw(Rng& rng, Distribution d) {
  switch (d) {
    case Distribution::kUniform: return rng.uniform(-1.f, 1.f);
    case Distribution::kNormal: return rng.normal();
    case Distribution::kSparseSigned: return rng.uniform() < 0.7 ? 0.f : rng.uniform(-2.f, 2.f);
    case Distribution::kPositive: return rng.uniform(0.f, 1.f);
  }
  return 0.f;
}
}  // namespace

HostConvData make_host_conv_data(const ConvProblem& prob, uint64_t seed, Distribution dist, Scaling scaling) {
  validate_problem(prob);
  const Conv2DParams& p = prob.p;
  Rng rng(seed);
  std::vector<float> rx(size_t(p.input_shape().numel())), rw(size_t(p.weight_shape().numel())),
      rb(size_t(p.out_channels));
  for (auto& v : rx) v = draw(rng, dist);
  const float k = float(p.gemm_k());
  const float wscale = scaling == Scaling::kBenchmark ? 1.0f / std::sqrt(k) : std::sqrt(3.0f / k);
  for (auto& v : rw) v = draw(rng, dist) * wscale;
  const float blim = scaling == Scaling::kBenchmark ? 0.1f : 1.0f;
  for (auto& v : rb) v = rng.uniform(-blim, blim);

  HostConvData h;
  const bool half_storage = prob.dtype() != DataType::kFloat32;
  h.hx.resize(rx.size());
  h.hw.resize(rw.size());
  h.hb.resize(rb.size());
  for (size_t i = 0; i < rx.size(); ++i) h.hx[i] = quantize_to(prob.precision, rx[i]);
  for (size_t i = 0; i < rw.size(); ++i) h.hw[i] = quantize_to(prob.precision, rw[i]);
  for (size_t i = 0; i < rb.size(); ++i) h.hb[i] = half_storage ? quantize_to(prob.precision, rb[i]) : rb[i];
  if (prob.precision == Precision::kTf32) {
    h.raw_x = std::move(rx);
    h.raw_w = std::move(rw);
  }
  return h;
}

ConvData make_conv_data(const ConvProblem& prob, uint64_t seed, Distribution dist, Scaling scaling) {
  HostConvData h = make_host_conv_data(prob, seed, dist, scaling);
  ConvData d;
  d.prob = prob;
  const DataType dt = prob.dtype();
  const bool tf32 = prob.precision == Precision::kTf32;
  d.dx = upload_as(tf32 ? h.raw_x : h.hx, dt);
  d.dw = upload_as(tf32 ? h.raw_w : h.hw, dt);
  d.db = upload_as(h.hb, dt);
  d.dy = DeviceBuffer(size_t(prob.p.output_shape().numel()) * dtype_size(dt));
  GIE_HIP_CHECK(hipMemset(d.dy.data(), 0xFF, d.dy.size()));  // NaN bits: unwritten outputs fail comparisons
  GIE_HIP_CHECK(hipDeviceSynchronize());
  d.hx = std::move(h.hx);
  d.hw = std::move(h.hw);
  d.hb = std::move(h.hb);
  return d;
}

}  // namespace gie
