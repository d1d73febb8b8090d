// Analytical cost model for MI355X (the role of src/runtime/perf_model.cpp:47-174) and the ceiling
// microbenchmarks that calibrate it (csrc/kernels/ceilings.hip).
//
// Model of one forward call of kernel k on problem P:
//   compute = FLOPs / (MFMA peak x family MFMA efficiency x tile efficiency x wave efficiency)
//   memory  = (compulsory bytes + the kernel's extra traffic) / (HBM bandwidth x family HBM efficiency)
//   fixed   = launches x dispatch cost + the family's cost of filling and draining a launch
//   time    = max(compute, memory) + fixed      (reported as launch_us; "launch"-bound when it dominates)
// * Family efficiencies are not guesses per backend: each is what that kernel family reached on an MI355X in the
//   library's benchmark protocol (per-call time, inputs resident in HBM), listed in kFamilies with the measurement.
// * Wave efficiency follows how gfx950 places workgroups: dispatch deals them round-robin to the 8 XCDs, and each
//   XCD's 32 CUs hold blocks_per_cu of them at a time, so a launch runs in ceil(ceil(blocks / 8) / (32 x occ))
//   waves and the last wave's empty slots are lost.
// * The dispatch cost is the measured gap of back-to-back launches on one stream (measure_ceilings), 1.5 us
//   before any measurement.
// The model only orders candidates for problems nothing has been measured on; the autotuner decides by timing.
#include "gpu_inference/perf_model.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <map>
#include <mutex>
#include <system_error>

#include "gie_hip.h"
#include "gpu_inference/json_lite.h"
#include "gpu_inference/tensor.h"
#include "gpu_inference/timing.h"

namespace gie {
namespace {

constexpr double kDefaultDispatchUs = 1.5;
constexpr int kXcds = 8;

struct FamilyProfile {
  const char* prefix;
  double mfma_eff;  // steady-state fraction of the dense MFMA peak (the FP32 vector peak for f32_)
  double hbm_eff;   // fraction of HBM bandwidth reached when bandwidth-bound
  double fill_us;   // fixed cost of a launch: workgroup set-up, pipeline fill, epilogue drain of the last wave
};

// Fitted to per-call times of each family's best entry on one MI355X (256 CUs), inputs resident in HBM, kernel
// arguments in device memory (HIP's default), the reference harness's protocol (median of 30 samples of >= 1 ms):
//   L2 = 32x256x14x14 -> 256 3x3 fp16, L3 = 64x256x28x28 -> 1024 1x1 fp16, L4 = 64x3x224x224 -> 64 7x7/2 fp16,
//   L5 = 8x512x7x7 -> 512 3x3 bf16.
// Where in-kernel clocks split a launch into its steady state and its fixed part (set-up, first loads, epilogue
// drain), mfma_eff is the steady state's share of the MFMA peak and fill_us the fixed part; otherwise the
// efficiency alone carries the measurement.
constexpr FamilyProfile kFamilies[] = {
    {"slab_", 0.66, 0.45, 2.5},     // L2 9.1 us (split form: steps at 0.66 of peak, ~3.7 us of set-up, first slice
                                    // and epilogue per unit); the other forms share the profile and the tuner
    {"band_", 0.27, 0.45, 5.0},     // L2 18.9 us including the weight repack launch
    {"halo_", 0.37, 0.40, 10.0},    // L2 23.3 us including the repack launch, L5 24.7 us at split 4
    {"mfma_", 0.22, 0.35, 8.0},     // L2 25.7 us, L3 87 us, L4 145 us, L5 26.0 us at split 4
    {"pw_", 0.30, 0.48, 2.0},       // L3 37.2-39.6 us (weight-stationary streaming form; shared tiles, 128-byte
                                    // device-scope runs) = 3.3-3.5 TB/s of compulsory traffic
    {"stem_", 0.28, 0.69, 2.0},     // L4 26.6-26.8 us (128-byte device-scope output runs) = 4.6 TB/s
    {"narrow_", 0.084, 0.30, 2.0},  // L5 15.0 us (123 TFLOP/s)
    {"stack_", 0.33, 0.40, 4.1},    // L5 9.6 us at split 2 (6.7 conv + 2.8 reduce), 10.2 at split 1
    {"deep_", 0.44, 0.40, 2.9},     // L5 6.6 us: steps at 0.44 of peak, ~4.2 us of set-up, first stage and
                                    // partial-tile exchange per unit
    {"f32_", 0.30, 0.35, 2.0},      // FP32 / TF32 vector kernels: not benchmarked, assumed
};

const FamilyProfile* profile_of(const std::string& name) {
  for (const FamilyProfile& f : kFamilies)
    if (name.compare(0, std::strlen(f.prefix), f.prefix) == 0) return &f;
  return nullptr;
}

std::mutex g_scale_mu;
std::map<std::string, double>& backend_scale() {
  static std::map<std::string, double> m;
  return m;
}

Bound bound_of(double compute_us, double memory_us, double launch_us) {
  if (launch_us >= std::max(compute_us, memory_us)) return Bound::kLaunch;
  return compute_us >= memory_us ? Bound::kCompute : Bound::kBandwidth;
}

// Fraction of the computed tile volume that is real work in the implicit-GEMM view.
double padded_fraction(const ConvProblem& prob, const KernelDesc& k) {
  const auto frac = [](int64_t v, int64_t tile) {
    tile = std::max<int64_t>(tile, 1);
    return double(v) / double(((v + tile - 1) / tile) * tile);
  };
  return frac(prob.p.gemm_m(), k.tile_m) * frac(prob.p.gemm_n(), k.tile_n) * frac(prob.p.gemm_k(), k.tile_k);
}

std::string ceiling_file(int device) {
  const DeviceInfo& d = DeviceInfo::get(device);
  std::string dir;
  if (const char* env = std::getenv("GIE_CEILING_DIR")) dir = env;
  else dir = std::string(std::getenv("HOME") ? std::getenv("HOME") : ".") + "/.cache/gpu_inference";
  std::string arch = d.gcn_arch;
  for (char& c : arch)
    if (c == ':' || c == '/' || c == ' ') c = '_';
  return dir + "/ceilings_" + arch + "_cu" + std::to_string(d.sm_count) + "_hip" + std::to_string(d.runtime_version) +
         ".json";
}

class ScopedDevice {
 public:
  explicit ScopedDevice(int device) {
    GIE_HIP_CHECK(hipGetDevice(&saved_));
    GIE_HIP_CHECK(hipSetDevice(device));
  }
  ~ScopedDevice() { (void)hipSetDevice(saved_); }

 private:
  int saved_ = 0;
};

class ScopedStream {
 public:
  ScopedStream() { GIE_HIP_CHECK(hipStreamCreateWithFlags(&s_, hipStreamNonBlocking)); }
  ~ScopedStream() { (void)hipStreamDestroy(s_); }
  hipStream_t get() const { return s_; }

 private:
  hipStream_t s_ = nullptr;
};

}  // namespace

void set_model_calibration(const std::map<std::string, double>& scale_by_backend) {
  std::lock_guard<std::mutex> lock(g_scale_mu);
  backend_scale() = scale_by_backend;
}

std::map<std::string, double> get_model_calibration() {
  std::lock_guard<std::mutex> lock(g_scale_mu);
  return backend_scale();
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
  c.launch_overhead_us = kDefaultDispatchUs;
  c.measured = false;
  c.source = "spec estimate (CU count x clock x CDNA per-CU rates; HBM from the product table)";
  return c;
}

bool load_cached_ceilings(int device, DeviceCeilings* out) {
  try {
    const std::string path = ceiling_file(device);
    const json::Value v = json::parse_file(path);
    const json::Value* mfma = v.find("fp16_mfma_tflops");
    const json::Value* bw = v.find("bw_gbs");
    const json::Value* launch = v.find("launch_overhead_us");
    if (mfma == nullptr || bw == nullptr || launch == nullptr) return false;
    DeviceCeilings c;
    c.fp16_tc_tflops = mfma->as_double();
    c.bw_gbs = bw->as_double();
    c.launch_overhead_us = launch->as_double();
    c.fp32_tflops = DeviceInfo::get(device).est_peak_fp32_tflops();
    c.measured = true;
    c.source = "measured, cached in " + path;
    if (c.fp16_tc_tflops <= 0 || c.bw_gbs <= 0) return false;
    *out = c;
    return true;
  } catch (const Error&) {
    return false;
  }
}

DeviceCeilings measure_ceilings(int device, bool use_cache) {
  DeviceCeilings c;
  if (use_cache && load_cached_ceilings(device, &c)) return c;
  ScopedDevice scope(device);
  const DeviceInfo& dev = DeviceInfo::get(device);
  c = theoretical_ceilings(dev);
  ScopedStream stream;
  TimingOptions to;
  to.warmup_iters = 3;
  to.samples = 10;
  {
    // MFMA: 8 workgroups per CU, each wave running 4 independent 16x16x32 fp16 chains (16384 FLOP per MFMA)
    const int blocks = dev.sm_count * 8, iters = 2048;
    DeviceBuffer sink(size_t(blocks) * 4);
    const TimingStats t = time_stream_work(
        [&](hipStream_t s) {
          check_kernel_status(gie_hip_ceiling_mfma(blocks, iters, static_cast<float*>(sink.data()), s),
                              "MFMA ceiling");
        },
        stream.get(), to);
    c.fp16_tc_tflops = double(blocks) * 4.0 * iters * 4.0 * 16384.0 / (t.median_us * 1e6);
  }
  {
    // HBM: a 512 MiB copy, twice the 256 MiB Infinity Cache, read + write counted
    const size_t bytes = size_t(512) << 20;
    DeviceBuffer src(bytes), dst(bytes);
    GIE_HIP_CHECK(hipMemsetAsync(src.data(), 0, bytes, stream.get()));
    const TimingStats t = time_stream_work(
        [&](hipStream_t s) {
          check_kernel_status(gie_hip_ceiling_copy(src.data(), dst.data(), bytes, s), "copy ceiling");
        },
        stream.get(), to);
    c.bw_gbs = 2.0 * double(bytes) / (t.median_us * 1e3);
  }
  {
    // dispatch: back-to-back empty kernels on one stream
    const TimingStats t = time_stream_work(
        [&](hipStream_t s) { check_kernel_status(gie_hip_ceiling_empty(s), "empty kernel"); }, stream.get(), to);
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
      const std::string path = ceiling_file(device);
      std::error_code ec;
      std::filesystem::create_directories(std::filesystem::path(path).parent_path(), ec);
      if (!ec) json::write_file(path, v);
    } catch (const Error&) {
      // an unwritable cache only costs a measurement next time
    }
  }
  return c;
}

ProblemModel analyze_problem(const ConvProblem& prob) {
  const Conv2DParams& p = prob.p;
  const double es = double(dtype_size(prob.dtype()));
  ProblemModel m;
  m.flops = double(p.flops());
  m.input_bytes = es * double(p.input_shape().numel());
  m.weight_bytes = es * double(p.weight_shape().numel());
  m.output_bytes = es * double(p.output_shape().numel());
  m.bias_bytes = prob.has_bias ? es * double(p.out_channels) : 0.0;
  m.compulsory_bytes = m.input_bytes + m.weight_bytes + m.output_bytes + m.bias_bytes;
  // an explicit unrolled matrix has one row of C*Kh*Kw taps per output pixel
  m.im2col_bytes = es * double(p.gemm_k()) * double(p.gemm_n());
  m.im2col_extra_traffic = 2.0 * m.im2col_bytes;  // written once, read once
  m.unfused_extra_traffic = 2.0 * m.output_bytes;  // a separate bias/ReLU pass reads and writes Y again
  m.arithmetic_intensity = m.flops / m.compulsory_bytes;
  m.unrolled_blowup = m.im2col_bytes / m.input_bytes;
  return m;
}

Estimate roofline_estimate(const ConvProblem& prob, const DeviceCeilings& c, bool tensor_cores) {
  const ProblemModel m = analyze_problem(prob);
  Estimate e;
  e.compute_us = m.flops / ((tensor_cores ? c.fp16_tc_tflops : c.fp32_tflops) * 1e6);
  e.memory_us = m.compulsory_bytes / (c.bw_gbs * 1e3);
  e.launch_us = c.launch_overhead_us;
  e.bound = bound_of(e.compute_us, e.memory_us, e.launch_us);
  e.time_us = e.bound == Bound::kLaunch ? e.launch_us : std::max(e.compute_us, e.memory_us);
  return e;
}

double backend_efficiency_prior(const KernelDesc& k) {
  if (const FamilyProfile* f = profile_of(k.name)) return f->mfma_eff;
  if (k.efficiency_prior > 0) return k.efficiency_prior;
  return 0.10;  // a kernel outside the measured families
}

Estimate estimate_kernel(const ConvProblem& prob, const KernelDesc& k, const DeviceInfo& dev, const DeviceCeilings& c) {
  const ProblemModel m = analyze_problem(prob);
  const FamilyProfile* fam = profile_of(k.name);
  const double mfma_eff = backend_efficiency_prior(k);
  const double hbm_eff = fam ? fam->hbm_eff : 0.35;

  Estimate e;
  e.tile_efficiency = k.tile_efficiency ? k.tile_efficiency(prob) : padded_fraction(prob, k);
  const int64_t blocks = k.num_blocks ? std::max<int64_t>(k.num_blocks(prob), 1) : 1;
  e.blocks_per_sm = k.blocks_per_cu ? std::max(k.blocks_per_cu(prob), 1) : 1;
  const int xcds = (dev.sm_count >= kXcds && dev.sm_count % kXcds == 0) ? kXcds : 1;
  const int64_t slots = int64_t(dev.sm_count / xcds) * e.blocks_per_sm;  // resident workgroups per XCD
  const int64_t per_xcd = (blocks + xcds - 1) / xcds;
  const int64_t waves = (per_xcd + slots - 1) / slots;
  e.wave_efficiency = double(blocks) / double(waves * slots * xcds);

  const double peak_tflops = k.uses_tensor_cores ? c.fp16_tc_tflops : c.fp32_tflops;
  const double rate = peak_tflops * 1e6 * mfma_eff * std::max(e.tile_efficiency, 1e-3) *
                      std::max(e.wave_efficiency, 1e-3);  // FLOP per us
  e.compute_us = m.flops / rate;
  const double traffic = m.compulsory_bytes + (k.extra_traffic_bytes ? k.extra_traffic_bytes(prob) : 0.0);
  e.memory_us = traffic / (c.bw_gbs * 1e3 * hbm_eff);
  // resident workgroups overlap each other's set-up, so only the launch's first fill and last drain are exposed
  e.launch_us = c.launch_overhead_us * std::max(k.launches, 1) + (fam ? fam->fill_us : 2.0);
  {
    std::lock_guard<std::mutex> lock(g_scale_mu);
    const auto it = backend_scale().find(to_string(k.backend));
    if (it != backend_scale().end()) {
      e.compute_us *= it->second;
      e.memory_us *= it->second;
    }
  }
  e.bound = bound_of(e.compute_us, e.memory_us, e.launch_us);
  e.time_us = std::max(e.compute_us, e.memory_us) + e.launch_us;
  return e;
}

}  // namespace gie
