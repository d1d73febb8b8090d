// The gfx950 narrow family (3x3 filter, stride 1, padding 1, few output pixels and a long reduction,
// conv_narrow.hip) as a registry entry: one launch straight from NCHW x and OIHW w, no repack and no split-K
// partials (the reference runs the same layer through its tcmma registration, src/kernels/tensor_core_mma.cu:264-395).
//   * capability filter: fp16/bf16, a gfx950 device, that filter geometry, in_channels % 128 == 0, the images one
//     32-pixel block touches fit LDS (gie_hip_narrow_check);
//   * the kernel reads x and w with 16-byte loads; caller tensors that are not aligned for that run the
//     implicit-GEMM entry of the same precision instead, so the workspace is that entry's.
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

int dtype_of(Precision p) { return p == Precision::kFp16 ? GIE_HIP_FP16 : GIE_HIP_BF16; }

// the entry that runs the problem when the caller's pointers are not 16-byte aligned
const KernelDesc& fallback_of(Precision p) {
  const KernelDesc* k = find_kernel(std::string("mfma_") + to_string(p) + "_128x128x64_w4x2_s3_sk1");
  if (!k) throw Error(StatusCode::kInternal, "pointwise family: implicit-GEMM fallback entry is missing");
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
    if (!dev.is_gfx950()) return no("needs gfx950 matrix cores (v_mfma_f32_32x32x16); device is " + dev.gcn_arch);
    const gie_conv_geom g = geom_of(prob);
    if (gie_hip_narrow_check(&g, nullptr) != GIE_HIP_OK)
      return no("narrow kernel: 3x3 filter, stride 1, padding 1, in_channels % 128 == 0, the images of a 32-pixel block within LDS");
    std::string fw;
    if (!fallback_of(P).supports(prob, dev, &fw)) return no("unaligned-pointer fallback cannot run it: " + fw);
    if (workspace(prob) > dev.global_mem_bytes / 4) return no("workspace exceeds a quarter of device memory");
    return true;
  }
  static size_t workspace(const ConvProblem& prob) { return fallback_of(P).workspace_bytes(prob); }
  static size_t lds(const ConvProblem& prob) {
    const gie_conv_geom g = geom_of(prob);
    int bytes = 0;
    return gie_hip_narrow_check(&g, &bytes) == GIE_HIP_OK ? size_t(bytes) : 0;
  }
  static int64_t blocks(const ConvProblem& prob) {  // tiles of 32 filters x 32 pixels, padded to 8 XCD ranges
    const Conv2DParams& p = prob.p;
    const int64_t tiles = (int64_t(p.batch) * p.out_h() * p.out_w() + 31) / 32 * ((p.out_channels + 31) / 32);
    return (tiles + 7) / 8 * 8;
  }
  static double extra_traffic(const ConvProblem&) { return 0.0; }  // X, W read and Y written once from HBM
  static int occupancy(const ConvProblem&) { return 1; }
  static void launch(const LaunchArgs& la) {
    const ConvProblem& prob = *la.problem;
    if ((reinterpret_cast<uintptr_t>(la.x) & 15u) || (reinterpret_cast<uintptr_t>(la.y) & 1u) ||
        (reinterpret_cast<uintptr_t>(la.w) & 15u) || (reinterpret_cast<uintptr_t>(la.bias) & 1u)) {
      fallback_of(P).launch(la);
      return;
    }
    if (la.only_stage >= 0 && la.only_stage != 1) return;  // one stage: the convolution itself
    const gie_conv_geom g = geom_of(prob);
    check_kernel_status(gie_hip_conv_narrow(dtype_of(P), &g, la.x, la.w, la.bias, la.y, la.stream),
                        "narrow MFMA convolution (3x3, whole reduction per workgroup)");
  }
};

template <Precision P>
KernelDesc make_entry() {
  using F = Fns<P>;
  KernelDesc k;
  k.name = std::string("narrow_") + to_string(P) + "_3x3_32x32x16_k8w";
  k.backend = Backend::kTensorCore;
  k.version = 1;
  k.params = {{"block_m", 32}, {"block_n", 32}, {"block_k", 16}, {"kernel_h", 3}, {"kernel_w", 3},
              {"stages", 1},   {"split_k", 1}};
  k.threads_per_block = 512;
  k.tile_m = 32;
  k.tile_n = 32;
  k.tile_k = 16;
  k.uses_tensor_cores = true;
  k.launches = 1;
  k.supports = &F::supports;
  k.workspace_bytes = &F::workspace;
  k.dynamic_smem_bytes = &F::lds;
  k.num_blocks = &F::blocks;
  k.extra_traffic_bytes = &F::extra_traffic;
  k.blocks_per_cu = &F::occupancy;
  k.launch = &F::launch;
  return k;
}

}  // namespace

void register_narrow_family(std::vector<KernelDesc>& out) {
  out.push_back(make_entry<Precision::kFp16>());
  out.push_back(make_entry<Precision::kBf16>());
}

}  // namespace gie
