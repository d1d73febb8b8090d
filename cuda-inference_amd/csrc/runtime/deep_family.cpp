// The gfx950 deep family (3x3 stride-1 MFMA convolution over small images with a long reduction, conv_deep.hip) as
// registry entries, in the role of the reference's tcmma registration (src/kernels/tensor_core_mma.cu:264-395):
//   * one launch per call: the whole reduction of a (16-filter block, image) tile runs in one workgroup, so there is
//     no split-K, no reduce launch and no workspace;
//   * capability filter: fp16/bf16, a gfx950 device, 3x3 / stride 1 / padding 1, in_channels % 128 == 0, in_h <= 8,
//     in_w <= 7, offsets within 32 bits (gie_hip_deep_check);
//   * the kernel reads w by 16-byte loads and x by 16-byte loads from 4-byte boundaries: a caller whose w is not
//     16-byte aligned or whose x is not 4-byte aligned runs the implicit-GEMM entry of the same precision.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <vector>

#include "gie_hip.h"
#include "gpu_inference/kernel_registry.h"

namespace gie {
namespace {

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

const KernelDesc& fallback_of(Precision p) {
  const KernelDesc* k = find_kernel(std::string("mfma_") + to_string(p) + "_128x128x64_w4x2_s3_sk1");
  if (!k) throw Error(StatusCode::kInternal, "deep family: implicit-GEMM fallback entry is missing");
  return *k;
}

template <Precision P>
struct Fns {
  static bool supports(const ConvProblem& prob, const DeviceInfo& dev, std::string* why) {
    auto no = [&](const std::string& m) {
      if (why) *why = m;
      return false;
    };
    if (prob.precision != P) return no(std::string("kernel is ") + to_string(P) + " only");
    if (!dev.is_gfx950()) return no("needs gfx950 matrix cores (v_mfma_f32_16x16x32); device is " + dev.gcn_arch);
    const gie_conv_geom g = geom_of(prob);
    int lds = 0;
    if (gie_hip_deep_check(&g, &lds) != GIE_HIP_OK)
      return no("deep kernel: 3x3 filter, stride 1, padding 1, in_channels % 128 == 0, in_h <= 8, in_w <= 7, "
                "offsets within 32 bits");
    if (size_t(lds) > dev.smem_per_block_optin)
      return no("needs " + std::to_string(lds / 1024) + " KiB LDS (limit " +
                std::to_string(dev.smem_per_block_optin / 1024) + " KiB)");
    std::string fw;
    if (!fallback_of(P).supports(prob, dev, &fw)) return no("unaligned-pointer fallback cannot run it: " + fw);
    return true;
  }
  static size_t workspace(const ConvProblem& prob) { return fallback_of(P).workspace_bytes(prob); }
  static size_t lds(const ConvProblem& prob) {
    const gie_conv_geom g = geom_of(prob);
    int bytes = 0;
    return gie_hip_deep_check(&g, &bytes) == GIE_HIP_OK ? size_t(bytes) : 0;
  }
  static int64_t blocks(const ConvProblem& prob) {  // (16-filter block, image), padded to 8 XCD ranges
    const int64_t units = int64_t(prob.p.batch) * ((prob.p.out_channels + 15) / 16);
    return (units + 7) / 8 * 8;
  }
  static double extra_traffic(const ConvProblem&) { return 0.0; }
  static int occupancy(const ConvProblem&) { return 1; }
  // useful output positions of the 8 x 8 tile (pitch 8, four 16-position blocks) times the filter padding
  static double tile_efficiency(const ConvProblem& prob) {
    const Conv2DParams& p = prob.p;
    const double pos = double(p.out_h()) * p.out_w() / 64.0;
    const double o = double(p.out_channels) / double(((p.out_channels + 15) / 16) * 16);
    return std::min(1.0, pos) * o;
  }
  static void launch(const LaunchArgs& la) {
    const ConvProblem& prob = *la.problem;
    const gie_conv_geom g = geom_of(prob);
    if ((reinterpret_cast<uintptr_t>(la.w) & 15u) || (reinterpret_cast<uintptr_t>(la.x) & 3u)) {
      fallback_of(P).launch(la);
      return;
    }
    if (la.only_stage < 0 || la.only_stage == 1)
      check_kernel_status(gie_hip_conv_deep(P == Precision::kFp16 ? GIE_HIP_FP16 : GIE_HIP_BF16, &g, la.x, la.w,
                                            la.bias, la.y, la.stream),
                          "deep MFMA convolution (NCHW / OIHW direct, whole reduction per workgroup)");
  }
};

template <Precision P>
KernelDesc make_entry() {
  KernelDesc k;
  k.name = std::string("deep_") + to_string(P) + "_3x3_16x8r8_k32x4_ld";
  k.backend = Backend::kTensorCore;
  k.version = 1;
  k.params = {{"block_m", 16}, {"rows", 8}, {"pitch", 8}, {"block_k", 32}, {"kernel_h", 3}, {"kernel_w", 3},
              {"stages", 2}, {"slices_per_step", 4}, {"split_k", 1}};
  k.threads_per_block = 512;
  k.tile_m = 16;
  k.tile_n = 64;
  k.tile_k = 32 * 9;
  k.uses_tensor_cores = true;
  k.launches = 1;
  k.supports = &Fns<P>::supports;
  k.workspace_bytes = &Fns<P>::workspace;
  k.dynamic_smem_bytes = &Fns<P>::lds;
  k.num_blocks = &Fns<P>::blocks;
  k.extra_traffic_bytes = &Fns<P>::extra_traffic;
  k.blocks_per_cu = &Fns<P>::occupancy;
  k.tile_efficiency = &Fns<P>::tile_efficiency;
  k.launch = &Fns<P>::launch;
  return k;
}

}  // namespace

void register_deep_family(std::vector<KernelDesc>& out) {
  out.push_back(make_entry<Precision::kFp16>());
  out.push_back(make_entry<Precision::kBf16>());
}

}  // namespace gie
