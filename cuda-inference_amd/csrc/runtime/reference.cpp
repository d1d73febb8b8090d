// Reference convolutions, tolerance model and error metrics (the reference's cpu_reference.cpp and
// reference.cu:95-200). The library's CPU reference and the oracle under oracle/ are independent
// implementations of the same definition; tests cross-check them.
#include "gpu_inference/reference.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <sstream>

#include "gie_hip.h"

#ifdef _OPENMP
#include <omp.h>
#endif

namespace gie {

void cpu_conv2d_reference(const ConvProblem& prob, const float* x, const float* w, const float* bias,
                          ReferenceOutput* out) {
  validate_problem(prob);
  const Conv2DParams& p = prob.p;
  const int OH = p.out_h(), OW = p.out_w();
  const int64_t total = int64_t(p.batch) * p.out_channels * OH * OW;
  out->y.assign(size_t(total), 0.f);
  out->scale.assign(size_t(total), 0.f);
  const bool relu = prob.activation == Activation::kReLU;
  const bool use_bias = prob.has_bias && bias != nullptr;
#pragma omp parallel for schedule(static)
  for (int64_t idx = 0; idx < total; ++idx) {
    const int64_t plane = int64_t(OH) * OW;
    const int b = int(idx / (plane * p.out_channels));
    const int o = int((idx / plane) % p.out_channels);
    const int oh = int((idx % plane) / OW), ow = int(idx % OW);
    double acc = 0.0, sumsq = 0.0;
    for (int c = 0; c < p.in_channels; ++c) {
      const float* xc = x + (int64_t(b) * p.in_channels + c) * p.in_h * p.in_w;
      const float* wc = w + (int64_t(o) * p.in_channels + c) * p.kernel_h * p.kernel_w;
      for (int r = 0; r < p.kernel_h; ++r) {
        const int ih = oh * p.stride_h - p.pad_h + r * p.dilation_h;
        if (ih < 0 || ih >= p.in_h) continue;
        for (int s = 0; s < p.kernel_w; ++s) {
          const int iw = ow * p.stride_w - p.pad_w + s * p.dilation_w;
          if (iw < 0 || iw >= p.in_w) continue;
          const double prod = double(xc[int64_t(ih) * p.in_w + iw]) * double(wc[r * p.kernel_w + s]);
          acc += prod;
          sumsq += prod * prod;
        }
      }
    }
    sumsq += acc * acc;
    if (use_bias) {
      acc += double(bias[o]);
      sumsq += double(bias[o]) * double(bias[o]);
    }
    if (relu && acc < 0.0) acc = 0.0;
    out->y[size_t(idx)] = float(acc);
    out->scale[size_t(idx)] = float(std::sqrt(sumsq));
  }
}

void gpu_conv2d_reference(const ConvProblem& prob, const void* x, const void* w, const void* bias, float* d_y,
                          float* d_scale, hipStream_t stream) {
  validate_problem(prob);
  if (prob.precision == Precision::kTf32)
    throw Error(StatusCode::kUnsupported, "the GPU reference has no TF32 multiplier rounding on this device");
  const Conv2DParams& p = prob.p;
  gie_conv_geom g{p.batch, p.in_channels, p.in_h, p.in_w, p.out_channels, p.kernel_h, p.kernel_w,
                  p.stride_h, p.stride_w, p.pad_h, p.pad_w, p.out_h(), p.out_w(), p.in_channels,
                  prob.activation == Activation::kReLU ? 1 : 0};
  const int dtype = prob.precision == Precision::kFp16 ? GIE_HIP_FP16
                    : prob.precision == Precision::kBf16 ? GIE_HIP_BF16
                                                         : GIE_HIP_FP32;
  check_kernel_status(gie_hip_reference_conv(dtype, &g, x, w, prob.has_bias ? bias : nullptr, d_y, d_scale, stream),
                      "GPU reference convolution");
}

// ---- storage rounding (IEEE-754 round to nearest even, from the format definitions) ----
namespace {
uint32_t f2u(float v) {
  uint32_t u;
  std::memcpy(&u, &v, 4);
  return u;
}
float u2f(uint32_t u) {
  float v;
  std::memcpy(&v, &u, 4);
  return v;
}
}  // namespace

uint16_t float_to_half_bits(float v) {
  const uint32_t x = f2u(v);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int exp = int((x >> 23) & 0xffu);
  const uint32_t mant = x & 0x7fffffu;
  if (exp == 0xff) return uint16_t(sign | (mant ? 0x7e00u : 0x7c00u));
  const int e = exp - 112;  // rebias 127 -> 15
  if (e >= 31) return uint16_t(sign | 0x7c00u);
  if (e > 0) {
    const uint32_t keep = mant >> 13, drop = mant & 0x1fffu;
    const uint32_t up = (drop > 0x1000u || (drop == 0x1000u && (keep & 1u))) ? 1u : 0u;
    return uint16_t(sign + ((uint32_t(e) << 10) | keep) + up);
  }
  const int shift = 126 - exp;  // value = (1.mant) * 2^(exp-127) = full * 2^(-24 - shift)... in units of 2^-24
  if (shift > 24 || (exp == 0 && mant == 0)) return uint16_t(sign);
  const uint32_t full = exp ? (mant | 0x800000u) : mant;
  const uint32_t keep = full >> shift, drop = full & ((1u << shift) - 1u), half = 1u << (shift - 1);
  const uint32_t up = (drop > half || (drop == half && (keep & 1u))) ? 1u : 0u;
  return uint16_t(sign | (keep + up));
}

float half_bits_to_float(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  if (exp == 0x1f) return u2f(sign | 0x7f800000u | (mant << 13));
  if (exp == 0) {
    const float mag = float(mant) * 5.9604644775390625e-08f;  // mant * 2^-24
    return sign ? -mag : mag;
  }
  return u2f(sign | ((exp + 112) << 23) | (mant << 13));
}

uint16_t float_to_bf16_bits(float v) {
  const uint32_t x = f2u(v);
  if ((x & 0x7fffffffu) > 0x7f800000u) return uint16_t((x >> 16) | 0x40u);
  return uint16_t((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

float bf16_bits_to_float(uint16_t h) { return u2f(uint32_t(h) << 16); }

float round_to_tf32(float v) {
  uint32_t bits = f2u(v);
  if ((bits & 0x7f800000u) == 0x7f800000u) return v;
  bits += 0x1000u;  // round to nearest, ties away from zero
  bits &= 0xffffe000u;
  return u2f(bits);
}

float quantize_to(Precision p, float v) {
  switch (p) {
    case Precision::kFp32: return v;
    case Precision::kTf32: return round_to_tf32(v);
    case Precision::kFp16: return half_bits_to_float(float_to_half_bits(v));
    case Precision::kBf16: return bf16_bits_to_float(float_to_bf16_bits(v));
  }
  return v;
}

std::vector<float> download_as_float(const void* d_ptr, DataType dt, int64_t n) {
  std::vector<float> out(static_cast<size_t>(n));
  if (dt == DataType::kFloat32) {
    GIE_HIP_CHECK(hipMemcpy(out.data(), d_ptr, size_t(n) * 4, hipMemcpyDeviceToHost));
  } else {
    std::vector<uint16_t> raw(static_cast<size_t>(n));
    GIE_HIP_CHECK(hipMemcpy(raw.data(), d_ptr, size_t(n) * 2, hipMemcpyDeviceToHost));
    for (int64_t i = 0; i < n; ++i)
      out[size_t(i)] = dt == DataType::kFloat16 ? half_bits_to_float(raw[size_t(i)]) : bf16_bits_to_float(raw[size_t(i)]);
  }
  return out;
}

// ---- tolerance and metrics ----
TolerancePolicy TolerancePolicy::for_problem(const ConvProblem& prob, bool intermediate_rounding) {
  TolerancePolicy t;
  t.k = prob.p.gemm_k();
  switch (prob.precision) {
    case Precision::kFp32: t.u_out = 5.9604644775390625e-08; t.abs_floor = 1e-30; break;
    case Precision::kTf32: t.u_out = 5.9604644775390625e-08; t.abs_floor = 1e-30; t.c_in = 8.0; break;
    case Precision::kFp16: t.u_out = 4.8828125e-04; t.abs_floor = 3.0e-8; break;
    case Precision::kBf16: t.u_out = 3.90625e-03; t.abs_floor = 1e-30; break;
  }
  if (intermediate_rounding) t.c_inter = 1.0;
  return t;
}

double TolerancePolicy::tol(double ref, double scale) const {
  return c_acc * u_acc * std::sqrt(double(k)) * scale + c_out * u_out * std::fabs(ref) + c_inter * u_out * scale +
         c_in * u_in * scale + abs_floor;
}

std::string TolerancePolicy::describe() const {
  std::ostringstream os;
  os << "tol_i = " << c_acc << "*2^-24*sqrt(K=" << k << ")*scale_i + " << c_out << "*u_out(" << u_out << ")*|ref_i| + "
     << c_inter << "*u_out*scale_i + " << abs_floor;
  return os.str();
}

ErrorMetrics compare_outputs(const float* test, const float* ref, const float* scale, int64_t n,
                             const TolerancePolicy& tol) {
  ErrorMetrics m;
  m.n = n;
  double sum_abs = 0, sum_sq = 0, ref_sq = 0;
  for (int64_t i = 0; i < n; ++i) ref_sq += double(ref[i]) * double(ref[i]);
  const double rel_floor = std::max(1e-3 * std::sqrt(ref_sq / double(std::max<int64_t>(n, 1))), 1e-30);
  for (int64_t i = 0; i < n; ++i) {
    const double t = test[i];
    if (std::isnan(t)) { ++m.nan_count; continue; }
    if (std::isinf(t)) { ++m.inf_count; continue; }
    const double err = std::fabs(t - double(ref[i]));
    sum_abs += err;
    sum_sq += err * err;
    m.max_abs = std::max(m.max_abs, err);
    m.max_rel = std::max(m.max_rel, err / std::max(std::fabs(double(ref[i])), rel_floor));
    const double ti = tol.tol(ref[i], scale[i]);
    m.worst_tol_ratio = std::max(m.worst_tol_ratio, err / ti);
    if (err > ti) ++m.over_tol;
  }
  m.mean_abs = n ? sum_abs / double(n) : 0;
  m.rms = n ? std::sqrt(sum_sq / double(n)) : 0;
  m.frac_over_tol = n ? double(m.over_tol) / double(n) : 0;
  m.rel_l2 = ref_sq > 0 ? std::sqrt(sum_sq / ref_sq) : std::sqrt(sum_sq);
  return m;
}

std::string ErrorMetrics::summary() const {
  std::ostringstream os;
  os << "max_abs=" << max_abs << " mean_abs=" << mean_abs << " rms=" << rms << " max_rel=" << max_rel
     << " rel_l2=" << rel_l2 << " over_tol=" << over_tol << "/" << n << " worst_tol_ratio=" << worst_tol_ratio
     << " nan=" << nan_count << " inf=" << inf_count;
  return os.str();
}

}  // namespace gie
