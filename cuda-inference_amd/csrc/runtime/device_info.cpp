// DeviceInfo on hipGetDeviceProperties, with CDNA peak tables (the reference's device_info.cpp keeps NVIDIA ones).
#include "gpu_inference/device_info.h"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <sstream>

#include "gpu_inference/error.h"

namespace gie {
namespace {

int attr(hipDeviceAttribute_t a, int dev) {
  int v = 0;
  GIE_HIP_CHECK(hipDeviceGetAttribute(&v, a, dev));
  return v;
}

bool arch_is(const std::string& arch, const char* prefix) { return arch.rfind(prefix, 0) == 0; }

// Dense FP16 MFMA FLOP per clock per CU (FP32 accumulate), from AMD's CDNA product specifications.
int fp16_mfma_flops_per_clk_cu(const std::string& arch) {
  if (arch_is(arch, "gfx950")) return 4096;  // MI355X: 2516.6 TFLOP/s at 256 CUs x 2.4 GHz
  if (arch_is(arch, "gfx942")) return 2048;  // MI300X
  if (arch_is(arch, "gfx90a")) return 1024;  // MI250X
  return 0;
}

// Vector FP32 FLOP per clock per CU.
int fp32_flops_per_clk_cu(const std::string& arch) {
  if (arch_is(arch, "gfx950") || arch_is(arch, "gfx942") || arch_is(arch, "gfx90a")) return 256;
  return 128;
}

// HBM peak by product (GB/s); the memory-clock formula under-reports HBM3E on ROCm.
double hbm_peak_gbs(const std::string& arch) {
  if (arch_is(arch, "gfx950")) return 8000.0;
  if (arch_is(arch, "gfx942")) return 5300.0;
  if (arch_is(arch, "gfx90a")) return 3276.8;
  return 0.0;
}

}  // namespace

bool DeviceInfo::supports_fp16_tensor_cores() const { return fp16_mfma_flops_per_clk_cu(gcn_arch) > 0; }
bool DeviceInfo::supports_bf16_tensor_cores() const { return fp16_mfma_flops_per_clk_cu(gcn_arch) > 0; }

double DeviceInfo::est_peak_fp32_tflops() const {
  return double(sm_count) * fp32_flops_per_clk_cu(gcn_arch) * double(max_sm_clock_khz) * 1e3 / 1e12;
}

double DeviceInfo::est_peak_fp16_tc_tflops() const {
  return double(sm_count) * fp16_mfma_flops_per_clk_cu(gcn_arch) * double(max_sm_clock_khz) * 1e3 / 1e12;
}

double DeviceInfo::est_peak_bw_gbs() const {
  const double t = hbm_peak_gbs(gcn_arch);
  if (t > 0) return t;
  return 2.0 * double(mem_clock_khz) * 1e3 * (double(mem_bus_bits) / 8.0) / 1e9;
}

std::string DeviceInfo::describe() const {
  std::ostringstream os;
  os << name << " (" << gcn_arch << ", " << sm_count << " CUs @ " << max_sm_clock_khz / 1000 << " MHz, "
     << global_mem_bytes / (1024 * 1024) << " MiB HBM, L2 " << l2_bytes / 1024 << " KiB, LDS/workgroup "
     << smem_per_block_default / 1024 << "/" << smem_per_block_optin / 1024 << " KiB, wave" << warp_size
     << ", HIP runtime " << runtime_version << ", driver " << driver_version << ")";
  return os.str();
}

const DeviceInfo& DeviceInfo::get(int device) {
  static std::mutex mu;
  static std::map<int, DeviceInfo> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(device);
  if (it != cache.end()) return it->second;

  DeviceInfo d;
  d.device = device;
  hipDeviceProp_t prop;
  GIE_HIP_CHECK(hipGetDeviceProperties(&prop, device));
  d.gcn_arch = prop.gcnArchName;
  // some driver stacks leave the marketing name empty: the architecture string then names the device
  d.name = prop.name[0] != '\0' ? std::string(prop.name) : "AMD GPU " + d.gcn_arch;
  d.cc_major = prop.major;
  d.cc_minor = prop.minor;
  d.global_mem_bytes = prop.totalGlobalMem;
  d.smem_per_block_default = prop.sharedMemPerBlock;
  d.warp_size = prop.warpSize;
  d.sm_count = prop.multiProcessorCount;
  d.l2_bytes = size_t(prop.l2CacheSize);
  d.smem_per_block_optin = prop.sharedMemPerBlockOptin ? prop.sharedMemPerBlockOptin : prop.sharedMemPerBlock;
  d.smem_per_sm = prop.maxSharedMemoryPerMultiProcessor;
  d.regs_per_sm = prop.regsPerMultiprocessor;
  d.max_threads_per_sm = prop.maxThreadsPerMultiProcessor;
  d.max_threads_per_block = prop.maxThreadsPerBlock;
  d.max_blocks_per_sm = attr(hipDeviceAttributeMaxBlocksPerMultiProcessor, device);
  d.max_sm_clock_khz = prop.clockRate;
  d.mem_clock_khz = prop.memoryClockRate;
  d.mem_bus_bits = prop.memoryBusWidth;
  GIE_HIP_CHECK(hipDriverGetVersion(&d.driver_version));
  GIE_HIP_CHECK(hipRuntimeGetVersion(&d.runtime_version));
  return cache.emplace(device, std::move(d)).first->second;
}

const DeviceInfo& DeviceInfo::current() {
  int dev = 0;
  GIE_HIP_CHECK(hipGetDevice(&dev));
  return get(dev);
}

}  // namespace gie
