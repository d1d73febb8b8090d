// The FP32 / TF32 family (conv_f32.hip: MFMA 32x32x2 f32 straight from NCHW x and OIHW w) as registry entries.
//   * FP32 entries carry the reference's FP32 backend and name stem (implicit_gemm_fp32_..., Backend::kImplicitGemm,
//     src/kernels/implicit_gemm.cu:218-268): they are the strict-FP32 GPU path.
//   * TF32 entries (mfma_tf32_..., Backend::kTensorCore) round the multiplier inputs to TF32 in the kernel, as the
//     reference's TF32 tensor-core kernels do.
//   * capability filter: the entry's precision, a gfx950 device, 32-bit offsets and grid limits
//     (gie_hip_f32_check), split <= the number of (tap, 16-channel) stages;
//   * workspace: none for split 1; split * |Y| FP32 partials otherwise (reduced by gie_hip_splitk_reduce).
// The FP32 matrix-core rate equals the vector FP32 rate on gfx950 (256 FLOP/clk/CU), so the cost model prices
// these entries against the FP32 ceiling (uses_tensor_cores = false).
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "gie_hip.h"
#include "gpu_inference/kernel_registry.h"

namespace gie {
namespace {

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

gie_conv_geom geom_of(const ConvProblem& prob) {
  const Conv2DParams& p = prob.p;
  gie_conv_geom g;
  g.batch = p.batch;
  g.in_channels = p.in_channels;
  g.in_h = p.in_h;
  g.in_w = p.in_w;
  g.out_channels = p.out_channels;
  g.kernel_h = p.kernel_h;
  g.kernel_w = p.kernel_w;
  g.stride_h = p.stride_h;
  g.stride_w = p.stride_w;
  g.pad_h = p.pad_h;
  g.pad_w = p.pad_w;
  g.out_h = p.out_h();
  g.out_w = p.out_w();
  g.c_pad = p.in_channels;
  g.relu = prob.activation == Activation::kReLU ? 1 : 0;
  return g;
}

int dtype_of(Precision p) { return p == Precision::kTf32 ? GIE_HIP_TF32 : GIE_HIP_FP32; }

template <int Config, int Split, Precision P>
struct Fns {
  static int tile_m() { return gie_hip_f32_config_tile_m(Config); }
  static bool supports(const ConvProblem& prob, const DeviceInfo& dev, std::string* why) {
    auto no = [&](const std::string& m) {
      if (why) *why = m;
      return false;
    };
    if (prob.precision != P) return no(std::string("kernel is ") + to_string(P) + " only");
    if (!dev.is_gfx950()) return no("needs gfx950 matrix cores (v_mfma_f32_32x32x2_f32); device is " + dev.gcn_arch);
    const gie_conv_geom g = geom_of(prob);
    int stages = 0;
    if (gie_hip_f32_check(Config, &g, &stages) != GIE_HIP_OK)
      return no("offsets exceed 32 bits or the grid exceeds its limits");
    if (Split > 1 && stages < 2 * Split) return no("reduction too short for this split-K factor");
    if (workspace(prob) > dev.global_mem_bytes / 4) return no("workspace exceeds a quarter of device memory");
    return true;
  }
  static size_t workspace(const ConvProblem& prob) {
    return Split > 1 ? align256(size_t(Split) * size_t(prob.p.output_shape().numel()) * 4) : 0;
  }
  static size_t lds(const ConvProblem&) { return size_t(2) * 16 * ((tile_m() + 32) + (128 + 32)) * 4; }
  static int64_t blocks(const ConvProblem& prob) {
    const int64_t n = int64_t(prob.p.batch) * prob.p.out_h() * prob.p.out_w();
    return (n + 127) / 128 * ((prob.p.out_channels + tile_m() - 1) / tile_m()) * Split;
  }
  static double extra_traffic(const ConvProblem& prob) {
    // each 128-pixel tile re-reads the weights and each filter tile the activations from L2 (not HBM); split-K
    // writes and re-reads the FP32 partials
    return Split > 1 ? 2.0 * Split * double(prob.p.output_shape().numel()) * 4.0 : 0.0;
  }
  static int occupancy(const ConvProblem&) { return 2; }
  static void launch(const LaunchArgs& la) {
    const ConvProblem& prob = *la.problem;
    const gie_conv_geom g = geom_of(prob);
    float* part = Split > 1 ? static_cast<float*>(la.workspace) : nullptr;
    const auto stage = [&](int k) { return la.only_stage < 0 || la.only_stage == k; };
    // stage 1: the convolution (no repack stage); stage 2: the split-K reduce
    if (stage(1)) {
      check_kernel_status(gie_hip_conv_f32(Config, dtype_of(P), &g, la.x, la.w, la.bias, la.y, part, Split, la.stream),
                          "FP32 MFMA convolution");
    }
    if (Split > 1 && stage(2)) {
      check_kernel_status(gie_hip_splitk_reduce(dtype_of(P), part, la.bias, la.y, prob.p.output_shape().numel(), Split,
                                                prob.p.out_channels, g.out_h * g.out_w, g.relu, la.stream),
                          "split-K reduce");
    }
  }
};

template <int Config, int Split, Precision P>
KernelDesc make_entry() {
  using F = Fns<Config, Split, P>;
  const int bm = gie_hip_f32_config_tile_m(Config);
  KernelDesc k;
  const std::string tile = std::to_string(bm) + "x128x16";
  if (P == Precision::kFp32) {
    k.name = "implicit_gemm_fp32_" + tile + "_mfma_sk" + std::to_string(Split);
    k.backend = Backend::kImplicitGemm;
  } else {
    k.name = std::string("mfma_") + to_string(P) + "_" + tile + "_sk" + std::to_string(Split);
    k.backend = Backend::kTensorCore;
  }
  k.version = 1;
  k.params = {{"block_m", bm}, {"block_n", 128}, {"block_k", 16}, {"stages", 2}, {"split_k", Split}};
  k.threads_per_block = 256;
  k.tile_m = bm;
  k.tile_n = 128;
  k.tile_k = 16;
  k.uses_tensor_cores = false;  // priced against the FP32 ceiling, which the FP32 MFMA rate equals
  k.launches = 1 + (Split > 1 ? 1 : 0);
  k.supports = &F::supports;
  k.workspace_bytes = &F::workspace;
  k.dynamic_smem_bytes = &F::lds;
  k.num_blocks = &F::blocks;
  k.extra_traffic_bytes = &F::extra_traffic;
  k.blocks_per_cu = &F::occupancy;
  k.launch = &F::launch;
  return k;
}

template <Precision P>
void add_precision(std::vector<KernelDesc>& out) {
  out.push_back(make_entry<0, 1, P>());
  out.push_back(make_entry<1, 1, P>());
  out.push_back(make_entry<0, 2, P>());
  out.push_back(make_entry<1, 2, P>());
  out.push_back(make_entry<0, 4, P>());
  out.push_back(make_entry<1, 4, P>());
  out.push_back(make_entry<0, 8, P>());
  out.push_back(make_entry<1, 8, P>());
}

}  // namespace

void register_f32_family(std::vector<KernelDesc>& out) {
  add_precision<Precision::kFp32>(out);
  add_precision<Precision::kTf32>(out);
}

}  // namespace gie
