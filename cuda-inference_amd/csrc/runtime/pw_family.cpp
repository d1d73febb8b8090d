// The gfx950 pointwise family (1x1 convolution straight from NCHW, conv_pw.hip) as registry entries (the role
// of the reference's tcmma registration, src/kernels/tensor_core_mma.cu:264-395, for the 1x1 case): one launch,
// no repack of either operand. Two forms per precision:
//   * tiled (pw_<p>_1x1_128x128x32_s4_sk1): 128 filters x 128 pixels per workgroup, any C % 8 == 0;
//   * streaming (pw_<p>_1x1_256x64x16_s4_wreg): 256 filters x C <= 256 held in registers per workgroup, one
//     8-wave workgroup per CU streaming a range of 64-pixel blocks (gie_hip_pws_check).
//   * capability filter: fp16/bf16, a gfx950 device, 1x1 filter, stride 1, no padding, C % 8 == 0 and
//     H*W % 8 == 0 (16-byte chunks of filters and channel rows), 32-bit offsets (gie_hip_pw_check);
//   * the kernels read x and w with 16-byte accesses; caller tensors that are only 2-byte aligned run the
//     implicit-GEMM entry of the same precision instead, so the workspace is that entry's (repacked X and W, the
//     reference's tcmma layout for the same problem).
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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <Precision P, bool Stream>
struct Fns {
  static bool supports(const ConvProblem& prob, const DeviceInfo& dev, std::string* why) {
    auto no = [&](const std::string& m) {
      if (why) *why = m;
      return false;
    };
    if (prob.precision != P) return no(std::string("kernel is ") + to_string(P) + " only");
    if (!dev.is_gfx950()) return no("needs gfx950 matrix cores (v_mfma_f32_32x32x16); device is " + dev.gcn_arch);
    const Conv2DParams& p = prob.p;
    if (p.kernel_h != 1 || p.kernel_w != 1 || p.stride_h != 1 || p.stride_w != 1 || p.pad_h != 0 || p.pad_w != 0)
      return no("pointwise kernel: 1x1 filter, stride 1, no padding only");
    const gie_conv_geom g = geom_of(prob);
    if (gie_hip_pw_check(&g, nullptr) != GIE_HIP_OK)
      return no("needs in_channels % 8 == 0 and in_h*in_w % 8 == 0 (16-byte rows), offsets within 32 bits");
    if (Stream && gie_hip_pws_check(&g, nullptr) != GIE_HIP_OK)
      return no("streaming form holds 256 filters x in_channels in registers: needs in_channels <= 256");
    std::string fw;
    if (!fallback_of(P).supports(prob, dev, &fw)) return no("unaligned-pointer fallback cannot run it: " + fw);
    if (workspace(prob) > dev.global_mem_bytes / 4) return no("workspace exceeds a quarter of device memory");
    return true;
  }
  static size_t workspace(const ConvProblem& prob) { return fallback_of(P).workspace_bytes(prob); }
  static size_t lds(const ConvProblem& prob) {
    if (!Stream) return 64 * 1024;
    const gie_conv_geom g = geom_of(prob);
    int bytes = 0;
    return gie_hip_pws_check(&g, &bytes) == GIE_HIP_OK ? size_t(bytes) : 0;
  }
  static int64_t blocks(const ConvProblem& prob) {
    const Conv2DParams& p = prob.p;
    if (Stream) {  // one workgroup per CU: 256-filter blocks x pixel ranges of 64-pixel blocks
      const int64_t n_ob = (p.out_channels + 255) / 256;
      const int64_t n_blk = (int64_t(p.batch) * p.in_h * p.in_w + 63) / 64;
      return n_ob * std::max<int64_t>(1, std::min<int64_t>(n_blk, std::max<int64_t>(1, 256 / n_ob)));
    }
    const int64_t tiles = int64_t(p.batch) * ((int64_t(p.in_h) * p.in_w + 127) / 128);
    return (tiles + 7) / 8 * 8 * ((p.out_channels + 127) / 128);
  }
  static double extra_traffic(const ConvProblem&) { return 0.0; }  // X, W read and Y written once from HBM
  static int occupancy(const ConvProblem&) { return Stream ? 1 : 2; }
  static void launch(const LaunchArgs& la) {
    const ConvProblem& prob = *la.problem;
    const bool y_ok = Stream ? (reinterpret_cast<uintptr_t>(la.y) & 7u) == 0 : aligned16(la.y);
    if (!aligned16(la.x) || !aligned16(la.w) || !y_ok) {
      fallback_of(P).launch(la);
      return;
    }
    if (la.only_stage >= 0 && la.only_stage != 1) return;  // one stage: the convolution itself
    const gie_conv_geom g = geom_of(prob);
    if (Stream)
      check_kernel_status(gie_hip_conv_pws(dtype_of(P), &g, la.x, la.w, la.bias, la.y, la.stream),
                          "pointwise MFMA convolution (weight-stationary streaming)");
    else
      check_kernel_status(gie_hip_conv_pw(dtype_of(P), &g, la.x, la.w, la.bias, la.y, la.stream),
                          "pointwise MFMA convolution (direct NCHW)");
  }
};

template <Precision P, bool Stream>
KernelDesc make_entry() {
  using F = Fns<P, Stream>;
  KernelDesc k;
  k.name = std::string("pw_") + to_string(P) + (Stream ? "_1x1_256x64x16_s4_wreg" : "_1x1_128x128x32_s4_sk1");
  k.backend = Backend::kTensorCore;
  k.version = 1;
  if (Stream)
    k.params = {{"block_m", 256}, {"block_n", 64}, {"block_k", 16}, {"kernel_h", 1}, {"kernel_w", 1},
                {"stages", 4},    {"split_k", 1}};
  else
    k.params = {{"block_m", 128}, {"block_n", 128}, {"block_k", 32}, {"kernel_h", 1}, {"kernel_w", 1},
                {"stages", 4},    {"split_k", 1}};
  k.threads_per_block = Stream ? 512 : 256;
  k.tile_m = Stream ? 256 : 128;
  k.tile_n = Stream ? 64 : 128;
  k.tile_k = Stream ? 16 : 32;
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

void register_pw_family(std::vector<KernelDesc>& out) {
  out.push_back(make_entry<Precision::kFp16, true>());
  out.push_back(make_entry<Precision::kBf16, true>());
  out.push_back(make_entry<Precision::kFp16, false>());
  out.push_back(make_entry<Precision::kBf16, false>());
}

}  // namespace gie
