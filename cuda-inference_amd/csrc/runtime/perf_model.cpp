// Roofline cost model (the reference's perf_model.cpp structure: compulsory traffic, tile and wave efficiency,
// per-family efficiency prior, launch overhead) + measured ceilings from the HIP microbenchmarks in
// csrc/kernels/ceilings.hip (the reference's ceilings.cu role), cached per GPU as JSON.
#include "gpu_inference/perf_model.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <map>
#include <mutex>

#include "gie_hip.h"
#include "gpu_inference/json_lite.h"
#include "gpu_inference/tensor.h"
#include "gpu_inference/timing.h"

namespace gie {
namespace {

std::mutex g_cal_mu;
std::map<std::string, double>& cal_map() {
  static std::map<std::string, double> m;
  return m;
}

double bytes_per_us(const DeviceCeilings& c) { return c.bw_gbs * 1e3; }
double flops_per_us(double tflops) { return tflops * 1e6; }

Bound classify(double compute_us, double memory_us, double launch_us) {
  if (launch_us >= compute_us && launch_us >= memory_us) return Bound::kLaunch;
  return compute_us >= memory_us ? Bound::kCompute : Bound::kBandwidth;
}

std::string ceiling_path(int device) {
  const DeviceInfo& d = DeviceInfo::get(device);
  std::string dir;
  if (const char* p = std::getenv("GIE_CEILING_DIR")) dir = p;
  else dir = std::string(std::getenv("HOME") ? std::getenv("HOME") : ".") + "/.cache/gpu_inference";
  std::string arch = d.gcn_arch;
  for (char& c : arch)
    if (c == ':' || c == '/' || c == ' ') c = '_';
  return dir + "/ceilings_" + arch + "_cu" + std::to_string(d.sm_count) + "_hip" + std::to_string(d.runtime_version) +
         ".json";
}

}  // namespace

void set_model_calibration(const std::map<std::string, double>& m) {
  std::lock_guard<std::mutex> lock(g_cal_mu);
  cal_map() = m;
}
std::map<std::string, double> get_model_calibration() {
  std::lock_guard<std::mutex> lock(g_cal_mu);
  return cal_map();
}

const char* to_string(Bound b) {
  switch (b) {
    case Bound::kCompute: return "compute";
    case Bound::kBandwidth: return "bandwidth";
    case Bound::kLaunch: return "launch";
  }
  return "?";
}

DeviceCeilings theoretical_ceilings(const DeviceInfo& dev) {
  DeviceCeilings c;
  c.fp32_tflops = dev.est_peak_fp32_tflops();
  c.fp16_tc_tflops = dev.est_peak_fp16_tc_tflops();
  c.bw_gbs = dev.est_peak_bw_gbs();
  c.launch_overhead_us = 4.0;
  c.measured = false;
  c.source = "theoretical estimate from CU count, max clock and CDNA throughput tables";
  return c;
}

bool load_cached_ceilings(int device, DeviceCeilings* out) {
  try {
    const json::Value v = json::parse_file(ceiling_path(device));
    const json::Value* f = v.find("fp16_mfma_tflops");
    const json::Value* b = v.find("bw_gbs");
    const json::Value* l = v.find("launch_overhead_us");
    if (!f || !b || !l) return false;
    out->fp16_tc_tflops = f->as_double();
    out->bw_gbs = b->as_double();
    out->launch_overhead_us = l->as_double();
    out->fp32_tflops = DeviceInfo::get(device).est_peak_fp32_tflops();
    out->measured = true;
    out->source = "measured (cached " + ceiling_path(device) + ")";
    return out->fp16_tc_tflops > 0 && out->bw_gbs > 0;
  } catch (const Error&) {
    return false;
  }
}

DeviceCeilings measure_ceilings(int device, bool use_cache) {
  DeviceCeilings c;
  if (use_cache && load_cached_ceilings(device, &c)) return c;
  int prev = 0;
  GIE_HIP_CHECK(hipGetDevice(&prev));
  GIE_HIP_CHECK(hipSetDevice(device));
  struct Restore {
    int d;
    ~Restore() { (void)hipSetDevice(d); }
  } restore{prev};
  const DeviceInfo& dev = DeviceInfo::get(device);
  c = theoretical_ceilings(dev);
  hipStream_t s;
  GIE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  struct SG {
    hipStream_t s;
    ~SG() { (void)hipStreamDestroy(s); }
  } sg{s};
  TimingOptions to;
  to.warmup_iters = 3;
  to.samples = 10;
  {  // matrix cores: 8 workgroups per CU, 4 independent MFMA chains per wave
    DeviceBuffer sink(size_t(dev.sm_count) * 8 * 4);
    const int blocks = dev.sm_count * 8, iters = 2048;
    const TimingStats t = time_stream_work(
        [&](hipStream_t st) {
          check_kernel_status(gie_hip_ceiling_mfma(blocks, iters, static_cast<float*>(sink.data()), st), "mfma ceiling");
        },
        s, to);
    const double flops = double(blocks) * 4.0 * iters * 4.0 * 16384.0;
    c.fp16_tc_tflops = flops / (t.median_us * 1e6);
  }
  {  // HBM: copy a buffer well beyond L2 + the 256 MiB Infinity Cache
    const size_t bytes = size_t(1) << 29;
    DeviceBuffer a(bytes), b(bytes);
    GIE_HIP_CHECK(hipMemsetAsync(a.data(), 0, bytes, s));
    const TimingStats t = time_stream_work(
        [&](hipStream_t st) { check_kernel_status(gie_hip_ceiling_copy(a.data(), b.data(), bytes, st), "copy ceiling"); },
        s, to);
    c.bw_gbs = 2.0 * double(bytes) / (t.median_us * 1e3);
  }
  {  // launch cost: back-to-back empty kernels on one stream
    const TimingStats t = time_stream_work(
        [&](hipStream_t st) { check_kernel_status(gie_hip_ceiling_empty(st), "empty kernel"); }, s, to);
    c.launch_overhead_us = t.median_us;
  }
  c.measured = true;
  c.source = "measured on " + dev.name;
  if (use_cache) {
    try {
      json::Value v = json::Value::object();
      v["device"] = dev.name;
      v["gcn_arch"] = dev.gcn_arch;
      v["fp16_mfma_tflops"] = c.fp16_tc_tflops;
      v["bw_gbs"] = c.bw_gbs;
      v["launch_overhead_us"] = c.launch_overhead_us;
      const std::string path = ceiling_path(device);
      const size_t slash = path.find_last_of('/');
      if (slash != std::string::npos) {
        const std::string cmd = "mkdir -p '" + path.substr(0, slash) + "'";
        if (std::system(cmd.c_str()) != 0) throw Error(StatusCode::kIo, "cannot create " + path.substr(0, slash));
      }
      json::write_file(path, v);
    } catch (const Error&) {
      // an unwritable cache directory only costs a re-measurement next time
    }
  }
  return c;
}

ProblemModel analyze_problem(const ConvProblem& prob) {
  const Conv2DParams& p = prob.p;
  const double esz = double(dtype_size(prob.dtype()));
  ProblemModel m;
  m.flops = double(p.flops());
  m.input_bytes = double(p.input_shape().numel()) * esz;
  m.weight_bytes = double(p.weight_shape().numel()) * esz;
  m.output_bytes = double(p.output_shape().numel()) * esz;
  m.bias_bytes = prob.has_bias ? double(p.out_channels) * esz : 0.0;
  m.compulsory_bytes = m.input_bytes + m.weight_bytes + m.output_bytes + m.bias_bytes;
  m.im2col_bytes = double(p.batch) * double(p.gemm_k()) * double(p.out_h()) * double(p.out_w()) * esz;
  m.im2col_extra_traffic = 2.0 * m.im2col_bytes;
  m.unfused_extra_traffic = 2.0 * m.output_bytes;
  m.arithmetic_intensity = m.flops / m.compulsory_bytes;
  m.unrolled_blowup = m.im2col_bytes / m.input_bytes;
  return m;
}

Estimate roofline_estimate(const ConvProblem& prob, const DeviceCeilings& c, bool tensor_cores) {
  const ProblemModel m = analyze_problem(prob);
  Estimate e;
  e.compute_us = m.flops / flops_per_us(tensor_cores ? c.fp16_tc_tflops : c.fp32_tflops);
  e.memory_us = m.compulsory_bytes / bytes_per_us(c);
  e.launch_us = c.launch_overhead_us;
  e.time_us = std::max(e.compute_us, e.memory_us);
  e.bound = classify(e.compute_us, e.memory_us, e.launch_us);
  if (e.bound == Bound::kLaunch) e.time_us = e.launch_us;
  return e;
}

double backend_efficiency_prior(const KernelDesc& k) {
  if (k.efficiency_prior > 0) return k.efficiency_prior;
  switch (k.backend) {
    case Backend::kDirect: return 0.05;
    case Backend::kSimtTiled: return 0.40;
    case Backend::kImplicitGemm: return 0.55;
    case Backend::kTensorCore: return 0.30;
    case Backend::kIm2colGemm: return 0.60;
    default: return 0.1;
  }
}

Estimate estimate_kernel(const ConvProblem& prob, const KernelDesc& k, const DeviceInfo& dev, const DeviceCeilings& c) {
  const ProblemModel m = analyze_problem(prob);
  Estimate e;
  if (k.tile_efficiency) {
    e.tile_efficiency = k.tile_efficiency(prob);
  } else {
    const auto pad = [](int64_t v, int64_t t) { return double(v) / double(((v + t - 1) / t) * t); };
    e.tile_efficiency = pad(prob.p.gemm_m(), k.tile_m) * pad(prob.p.gemm_n(), k.tile_n) * pad(prob.p.gemm_k(), k.tile_k);
  }
  const int64_t blocks = k.num_blocks ? std::max<int64_t>(k.num_blocks(prob), 1) : 1;
  e.blocks_per_sm = k.blocks_per_cu ? std::max(k.blocks_per_cu(prob), 1) : 1;
  const double slots = double(dev.sm_count) * e.blocks_per_sm;
  e.wave_efficiency = double(blocks) / (std::ceil(double(blocks) / slots) * slots);
  // a workgroup occupies one CU: below one workgroup per CU the idle CUs are lost too
  const double cu_fill = std::min(1.0, double(blocks) / double(std::max(dev.sm_count, 1)));

  const double peak = k.uses_tensor_cores ? c.fp16_tc_tflops : c.fp32_tflops;
  const double eff = backend_efficiency_prior(k) * std::max(e.tile_efficiency, 1e-3) *
                     std::max(std::min(e.wave_efficiency, cu_fill), 1e-3);
  e.compute_us = m.flops / (flops_per_us(peak) * eff);

  double traffic = m.compulsory_bytes;
  if (k.extra_traffic_bytes) traffic += k.extra_traffic_bytes(prob);
  e.memory_us = traffic / bytes_per_us(c);
  e.launch_us = c.launch_overhead_us * k.launches;
  e.bound = classify(e.compute_us, e.memory_us, e.launch_us);
  e.time_us = std::max(e.compute_us, e.memory_us) + e.launch_us;
  {
    std::lock_guard<std::mutex> lock(g_cal_mu);
    auto it = cal_map().find(to_string(k.backend));
    if (it != cal_map().end()) {
      e.compute_us *= it->second;
      e.memory_us *= it->second;
      e.time_us = std::max(e.compute_us, e.memory_us) + e.launch_us;
    }
  }
  return e;
}

}  // namespace gie
