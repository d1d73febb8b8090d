// The gfx950 slab family (3x3 stride-1 MFMA convolution straight from NCHW x and OIHW w, conv_slab.hip) as
// registry entries, in the role of the reference's tcmma registration (src/kernels/tensor_core_mma.cu:264-395):
//   * one launch per call (two with split-K: the slab kernel writes FP32 partials, splitk_reduce.hip finishes);
//     there is no repack of either operand, so split 1 needs no workspace;
//   * capability filter: fp16/bf16, a gfx950 device, 3x3 / stride 1 / padding 1, in_channels % 8 == 0, rows that
//     fit the entry's pitch, 32-bit offsets (gie_hip_slab_check), split <= the number of channel slices;
//   * the kernel reads the weights by 16-byte loads and, for even rows, the activations by 4-byte loads: a caller
//     whose w is not 16-byte aligned, or whose x the configuration cannot load, runs the implicit-GEMM entry of the
//     same precision (y may have any 2-byte alignment).
// Workspace = [split * |Y| FP32 partials | 256-B align] for split > 1, else 0.
#include <hip/hip_runtime.h>

#include <algorithm>
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

int dtype_of(Precision p) { return p == Precision::kFp16 ? GIE_HIP_FP16 : GIE_HIP_BF16; }

struct Entry {
  int config;
  int split;
  Precision precision;
  gie_slab_config info;
};

std::vector<Entry>& entries() {
  static std::vector<Entry> e;
  return e;
}

const KernelDesc& fallback_of(Precision p) {
  const KernelDesc* k = find_kernel(std::string("mfma_") + to_string(p) + "_128x128x64_w4x2_s3_sk1");
  if (!k) throw Error(StatusCode::kInternal, "slab family: implicit-GEMM fallback entry is missing");
  return *k;
}

int slices_of(const ConvProblem& prob, const Entry& en) {
  return (prob.p.in_channels + en.info.tile_k - 1) / en.info.tile_k;
}

template <int I>
struct Fns {
  static const Entry& e() { return entries()[I]; }
  static bool supports(const ConvProblem& prob, const DeviceInfo& dev, std::string* why) {
    auto no = [&](const std::string& m) {
      if (why) *why = m;
      return false;
    };
    const Entry& en = e();
    if (prob.precision != en.precision) return no(std::string("kernel is ") + to_string(en.precision) + " only");
    if (!dev.is_gfx950()) return no("needs gfx950 matrix cores (v_mfma_f32_16x16x32); device is " + dev.gcn_arch);
    const gie_conv_geom g = geom_of(prob);
    int lds = 0;
    if (gie_hip_slab_check(en.config, &g, &lds) != GIE_HIP_OK)
      return no("slab kernel: 3x3 filter, stride 1, padding 1, in_channels % 8 == 0, in_w + 1 <= " +
                std::to_string(en.info.pitch) + ", offsets within 32 bits");
    if (en.split > slices_of(prob, en)) return no("split-K factor exceeds the channel slices");
    if (size_t(lds) > dev.smem_per_block_optin)
      return no("needs " + std::to_string(lds / 1024) + " KiB LDS (limit " +
                std::to_string(dev.smem_per_block_optin / 1024) + " KiB)");
    std::string fw;
    if (!fallback_of(en.precision).supports(prob, dev, &fw))
      return no("unaligned-weight fallback cannot run it: " + fw);
    if (workspace(prob) > dev.global_mem_bytes / 4) return no("workspace exceeds a quarter of device memory");
    return true;
  }
  static size_t own_workspace(const ConvProblem& prob) {
    return e().split > 1 ? align256(size_t(e().split) * size_t(prob.p.output_shape().numel()) * 4) : 0;
  }
  static size_t workspace(const ConvProblem& prob) {
    return std::max(own_workspace(prob), fallback_of(e().precision).workspace_bytes(prob));
  }
  static size_t lds(const ConvProblem& prob) {
    const gie_conv_geom g = geom_of(prob);
    int bytes = 0;
    return gie_hip_slab_check(e().config, &g, &bytes) == GIE_HIP_OK ? size_t(bytes) : 0;
  }
  static int64_t blocks(const ConvProblem& prob) {  // (split, image, slab of rows, 32-filter block)
    const Entry& en = e();
    const Conv2DParams& p = prob.p;
    const int64_t slabs = (p.out_h() + en.info.rows - 1) / en.info.rows;
    return int64_t(en.split) * p.batch * slabs * ((p.out_channels + 31) / 32);
  }
  static double extra_traffic(const ConvProblem& prob) {  // FP32 partials written and read back
    return e().split > 1 ? 2.0 * e().split * double(prob.p.output_shape().numel()) * 4.0 : 0.0;
  }
  // the full and pipelined forms hold ~300-400 VGPR+AGPR per lane (one workgroup per CU), the split form two waves
  // per SIMD of at most 256 (one workgroup per CU); the lean form 256 at most (two workgroups)
  static int occupancy(const ConvProblem&) { return e().info.workgroups_per_cu; }
  // Useful output positions per step-equivalent: every slab of rows runs the step sequence of the widest
  // configuration (224 positions x 32 filters), whatever its own rows x pitch, because a step's time is set by its
  // loads and waits more than by its MFMA count; times the filter and channel padding.
  static double tile_efficiency(const ConvProblem& prob) {
    const Entry& en = e();
    const Conv2DParams& p = prob.p;
    const int64_t slabs = (p.out_h() + en.info.rows - 1) / en.info.rows;
    const double pos = double(p.out_h()) * p.out_w() / (double(slabs) * 224.0);
    const double o = double(p.out_channels) / double(((p.out_channels + 31) / 32) * 32);
    const double c = double(p.in_channels) / double(((p.in_channels + 31) / 32) * 32);
    return std::min(1.0, pos) * o * c;
  }
  static void launch(const LaunchArgs& la) {
    const Entry& en = e();
    const ConvProblem& prob = *la.problem;
    const gie_conv_geom g = geom_of(prob);
    float* part = en.split > 1 ? static_cast<float*>(la.workspace) : nullptr;
    const int dt = dtype_of(prob.precision);
    const auto stage = [&](int k) { return la.only_stage < 0 || la.only_stage == k; };
    // w not 16-byte aligned, or an x alignment whose load form this configuration lacks: the kernel refuses the
    // call before launching anything and the implicit-GEMM entry runs it instead
    if (reinterpret_cast<uintptr_t>(la.w) & 15u) {
      fallback_of(en.precision).launch(la);
      return;
    }
    if (stage(1)) {
      const int rc = gie_hip_conv_slab(en.config, dt, &g, la.x, la.w, la.bias, la.y, part, en.split, la.stream);
      if (rc == GIE_HIP_EUNSUPPORTED) {
        fallback_of(en.precision).launch(la);
        return;
      }
      check_kernel_status(rc, "slab MFMA convolution (NCHW / OIHW direct)");
    }
    if (en.split > 1 && stage(2))
      check_kernel_status(gie_hip_splitk_reduce(dt, part, la.bias, la.y, prob.p.output_shape().numel(), en.split,
                                                prob.p.out_channels, g.out_h * g.out_w, g.relu, la.stream),
                          "split-K reduce");
  }
};

constexpr int kMaxEntries = 128;

template <int I>
void fill_fns(int idx, KernelDesc& k) {
  if constexpr (I < kMaxEntries) {
    if (idx == I) {
      k.supports = &Fns<I>::supports;
      k.workspace_bytes = &Fns<I>::workspace;
      k.dynamic_smem_bytes = &Fns<I>::lds;
      k.num_blocks = &Fns<I>::blocks;
      k.extra_traffic_bytes = &Fns<I>::extra_traffic;
      k.blocks_per_cu = &Fns<I>::occupancy;
      k.tile_efficiency = &Fns<I>::tile_efficiency;
      k.launch = &Fns<I>::launch;
      return;
    }
    fill_fns<I + 1>(idx, k);
  }
}

}  // namespace

void register_slab_family(std::vector<KernelDesc>& out) {
  std::vector<Entry>& es = entries();
  es.clear();
  const int n = gie_hip_slab_config_count();
  for (Precision prec : {Precision::kFp16, Precision::kBf16}) {
    for (int ci = 0; ci < n; ++ci) {
      gie_slab_config info;
      check_kernel_status(gie_hip_slab_config_get(ci, &info), "slab config query");
      for (int split : {1, 2, 4, 8}) es.push_back({ci, split, prec, info});
    }
  }
  if (es.size() > size_t(kMaxEntries)) throw Error(StatusCode::kInternal, "too many slab registry entries");
  for (size_t i = 0; i < es.size(); ++i) {
    const Entry& en = es[i];
    KernelDesc k;
    k.name = std::string("slab_") + to_string(en.precision) + "_3x3_" + std::to_string(en.info.tile_m) + "x" +
             std::to_string(en.info.rows) + "r" + std::to_string(en.info.pitch) + "_k" +
             std::to_string(en.info.tile_k) + "_s" + std::to_string(en.info.stages) +
             (en.info.form == 1 ? "_l" : en.info.form == 2 ? "_p" : en.info.form == 3 ? "_ld" : "") +
             (en.info.workgroups_per_cu > 1 ? "_o" + std::to_string(en.info.workgroups_per_cu) : std::string()) + "_sk" +
             std::to_string(en.split);
    k.backend = Backend::kTensorCore;
    k.version = en.info.version;
    k.params = {{"block_m", en.info.tile_m}, {"rows", en.info.rows}, {"pitch", en.info.pitch},
                {"block_k", en.info.tile_k}, {"kernel_h", 3}, {"kernel_w", 3}, {"stages", en.info.stages},
                {"workgroups_per_cu", en.info.workgroups_per_cu}, {"form", en.info.form},
                {"split_k", en.split}};
    k.threads_per_block = en.info.threads;
    k.tile_m = en.info.tile_m;
    k.tile_n = en.info.rows * en.info.pitch;
    k.tile_k = en.info.tile_k * 9;
    k.uses_tensor_cores = true;
    k.launches = 1 + (en.split > 1 ? 1 : 0);
    fill_fns<0>(int(i), k);
    out.push_back(std::move(k));
  }
}

}  // namespace gie
