// The gfx950 stem family (7x7 filter, stride 2, padding 3, in_channels <= 4, conv_stem.hip) as a registry
// entry: one launch straight from NCHW, no repack and no channel padding (the reference runs the same layer
// through its tcmma registration, src/kernels/tensor_core_mma.cu:264-395).
//   * capability filter: fp16/bf16, a gfx950 device, that filter geometry, in_w % 16 == 0, 32-bit offsets
//     (gie_hip_stem_check);
//   * the kernel reads x rows and w with 16-byte loads and writes y with 16-byte stores; caller tensors that are not
//     aligned for that run the implicit-GEMM entry of the same precision instead, so the workspace is that entry's.
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
    if (gie_hip_stem_check(&g, nullptr) != GIE_HIP_OK)
      return no("stem kernel: 7x7 filter, stride 2, padding 3, in_channels <= 4, in_w % 16 == 0, 32-bit offsets");
    std::string fw;
    if (!fallback_of(P).supports(prob, dev, &fw)) return no("unaligned-pointer fallback cannot run it: " + fw);
    if (workspace(prob) > dev.global_mem_bytes / 4) return no("workspace exceeds a quarter of device memory");
    return true;
  }
  static size_t workspace(const ConvProblem& prob) { return fallback_of(P).workspace_bytes(prob); }
  static size_t lds(const ConvProblem& prob) {
    const gie_conv_geom g = geom_of(prob);
    int bytes = 0;
    return gie_hip_stem_check(&g, &bytes) == GIE_HIP_OK ? size_t(bytes) : 0;
  }
  static int64_t blocks(const ConvProblem& prob) {  // persistent: one workgroup per CU and 64-filter group
    const Conv2DParams& p = prob.p;
    const int64_t tiles = int64_t(p.batch) * ((p.out_h() + 3) / 4);  // 4-row tiles (2 for wide rows)
    return std::min<int64_t>((tiles + 7) / 8 * 8, 256) * ((p.out_channels + 63) / 64);
  }
  static double extra_traffic(const ConvProblem&) { return 0.0; }  // X, W read and Y written once from HBM
  static int occupancy(const ConvProblem&) { return 1; }
  static void launch(const LaunchArgs& la) {
    const ConvProblem& prob = *la.problem;
    if ((reinterpret_cast<uintptr_t>(la.x) & 15u) || (reinterpret_cast<uintptr_t>(la.y) & 15u) ||
        (reinterpret_cast<uintptr_t>(la.w) & 15u) || (reinterpret_cast<uintptr_t>(la.bias) & 1u)) {
      fallback_of(P).launch(la);
      return;
    }
    if (la.only_stage >= 0 && la.only_stage != 1) return;  // one stage: the convolution itself
    const gie_conv_geom g = geom_of(prob);
    check_kernel_status(gie_hip_conv_stem(dtype_of(P), &g, la.x, la.w, la.bias, la.y, la.stream),
                        "stem MFMA convolution (7x7 stride 2, direct NCHW)");
  }
};

template <Precision P>
KernelDesc make_entry() {
  using F = Fns<P>;
  KernelDesc k;
  k.name = std::string("stem_") + to_string(P) + "_7x7s2_64x32x16_wreg";
  k.backend = Backend::kTensorCore;
  k.version = 2;  // 2: device-scope output stores
  k.params = {{"block_m", 64}, {"block_n", 32}, {"block_k", 16}, {"kernel_h", 7}, {"kernel_w", 7},
              {"stages", 1},   {"split_k", 1}};
  k.threads_per_block = 512;
  k.tile_m = 64;
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

void register_stem_family(std::vector<KernelDesc>& out) {
  out.push_back(make_entry<Precision::kFp16>());
  out.push_back(make_entry<Precision::kBf16>());
}

}  // namespace gie
