// The gfx950 band family (direct-NCHW MFMA convolution, conv_band.hip) as registry entries (the role of the
// reference's tcmma registration, src/kernels/tensor_core_mma.cu:264-395): the weight repack into 32-channel
// slices, the band kernel reading the activations as NCHW (no activation repack) with the fused epilogue, and the
// split-K reduce for split entries.
//   * capability filter: fp16/bf16, a gfx950 device, the filter size of the entry, and the geometry checks of
//     the kernel itself (band rows fit the LDS stage, 32-bit offsets) through gie_hip_band_check;
//   * workspace = [wb | 256-B align][split * |Y| FP32 partials | align], wb channel-blocked (repack_blocked.hip).
// Every launch goes through the kernel C-ABI (include/gie_hip.h); nothing here allocates or synchronizes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <vector>

#include "gie_hip.h"
#include "gpu_inference/kernel_registry.h"

namespace gie {
namespace {

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }
int c_pad_of(const ConvProblem& prob) { return (prob.p.in_channels + 31) / 32 * 32; }  // S slices of 32

struct WsLayout {
  size_t wk_off, part_off, total;
};

WsLayout ws_layout(const ConvProblem& prob, int split) {
  const Conv2DParams& p = prob.p;
  const size_t cp = size_t(c_pad_of(prob));
  WsLayout l;
  l.wk_off = 0;
  l.part_off = align256(size_t(p.out_channels) * p.kernel_h * p.kernel_w * cp * 2);
  l.total = l.part_off + (split > 1 ? align256(size_t(split) * size_t(p.output_shape().numel()) * 4) : 0);
  return l;
}

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
  g.c_pad = c_pad_of(prob);
  g.relu = prob.activation == Activation::kReLU ? 1 : 0;
  return g;
}

int dtype_of(Precision p) { return p == Precision::kFp16 ? GIE_HIP_FP16 : GIE_HIP_BF16; }

struct Entry {
  int config;
  int split;
  Precision precision;
  gie_band_config info;
};

std::vector<Entry>& entries() {
  static std::vector<Entry> e;
  return e;
}

int slices_of(const ConvProblem& prob, const Entry& en) { return (c_pad_of(prob) + en.info.tile_k - 1) / en.info.tile_k; }

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
    if (!dev.is_gfx950()) return no("needs gfx950 matrix cores (v_mfma_f32_32x32x16); device is " + dev.gcn_arch);
    const Conv2DParams& p = prob.p;
    if (p.kernel_h != en.info.kernel_h || p.kernel_w != en.info.kernel_w)
      return no("kernel is for " + std::to_string(en.info.kernel_h) + "x" + std::to_string(en.info.kernel_w) +
                " filters");
    if (en.split > 1 && slices_of(prob, en) < 2 * en.split)
      return no("reduction too short for this split-K factor");
    const gie_conv_geom g = geom_of(prob);
    int lds = 0;
    const int rc = gie_hip_band_check(en.config, &g, &lds);
    if (rc != GIE_HIP_OK)
      return no("band rows do not fit the LDS stage, or the output row is too wide (or offsets exceed 32 bits)");
    if (size_t(lds) > dev.smem_per_block_optin)
      return no("needs " + std::to_string(lds / 1024) + " KiB LDS (limit " +
                std::to_string(dev.smem_per_block_optin / 1024) + " KiB)");
    if (workspace(prob) > dev.global_mem_bytes / 4) return no("workspace exceeds a quarter of device memory");
    return true;
  }
  static size_t workspace(const ConvProblem& prob) { return ws_layout(prob, e().split).total; }
  static size_t lds(const ConvProblem& prob) {
    const gie_conv_geom g = geom_of(prob);
    int bytes = 0;
    if (gie_hip_band_check(e().config, &g, &bytes) != GIE_HIP_OK) return 0;
    return size_t(bytes);
  }
  // Useful output positions of a workgroup's tile_n-position band (rows of a power-of-two padded width, one image
  // per band), times the filter and channel padding.
  static double tile_efficiency(const ConvProblem& prob) {
    const Entry& en = e();
    const Conv2DParams& p = prob.p;
    int owp = 1;
    while (owp < p.out_w()) owp *= 2;
    const int rows = std::max(1, en.info.tile_n / owp);
    const int64_t bands = (p.out_h() + rows - 1) / rows;
    const double pos = double(p.out_h()) * p.out_w() / (double(bands) * en.info.tile_n);
    const double o = double(p.out_channels) / double(((p.out_channels + en.info.tile_m - 1) / en.info.tile_m) *
                                                     en.info.tile_m);
    const double c = double(p.in_channels) / double(((p.in_channels + en.info.tile_k - 1) / en.info.tile_k) *
                                                    en.info.tile_k);
    return std::min(1.0, pos) * o * c;
  }
  static int64_t blocks(const ConvProblem& prob) {
    // one workgroup per (32 output channels, image, band of rows); a band is tile_n / padded-row-width rows
    const Entry& en = e();
    const Conv2DParams& p = prob.p;
    int owp = 1;
    while (owp < p.out_w()) owp *= 2;
    const int rows = std::max(1, en.info.tile_n / owp);
    const int64_t bands = (p.out_h() + rows - 1) / rows;
    return int64_t((p.out_channels + en.info.tile_m - 1) / en.info.tile_m) * p.batch * bands * en.split;
  }
  static double extra_traffic(const ConvProblem& prob) {
    // the weight repack writes the padded copy of W, which the kernel reads again; split-K writes and re-reads
    // FP32 partials
    const Conv2DParams& p = prob.p;
    const double cp = c_pad_of(prob);
    const double wp = double(p.out_channels) * p.kernel_h * p.kernel_w * cp * 2.0;
    const double part = e().split > 1 ? 2.0 * e().split * double(p.output_shape().numel()) * 4.0 : 0.0;
    return 2.0 * wp + part;
  }
  static int occupancy(const ConvProblem& prob) {
    const size_t l = lds(prob);
    return l > 80 * 1024 ? 1 : 2;
  }
  static void launch(const LaunchArgs& la) {
    const Entry& en = e();
    const ConvProblem& prob = *la.problem;
    const gie_conv_geom g = geom_of(prob);
    const WsLayout l = ws_layout(prob, en.split);
    char* ws = static_cast<char*>(la.workspace);
    void* wk = ws + l.wk_off;
    float* part = en.split > 1 ? reinterpret_cast<float*>(ws + l.part_off) : nullptr;
    void* s = la.stream;
    const auto stage = [&](int k) { return la.only_stage < 0 || la.only_stage == k; };
    record_stage_event(la, 0);
    if (stage(0)) {
      check_kernel_status(gie_hip_repack_w_blocked(la.w, wk, &g, s), "channel-blocked weight repack");
    }
    record_stage_event(la, 1);
    if (stage(1)) {
      check_kernel_status(gie_hip_conv_band(en.config, dtype_of(prob.precision), &g, la.x, wk, la.bias, la.y, part,
                                          en.split, s),
                        "band MFMA convolution (direct NCHW)");
    }
    record_stage_event(la, 2);
    if (en.split > 1 && stage(2)) {
      check_kernel_status(gie_hip_splitk_reduce(dtype_of(prob.precision), part, la.bias, la.y,
                                                prob.p.output_shape().numel(), en.split, prob.p.out_channels,
                                                g.out_h * g.out_w, g.relu, s),
                          "split-K reduce");
    }
  }
};

constexpr int kMaxEntries = 96;

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

void register_band_family(std::vector<KernelDesc>& out) {
  std::vector<Entry>& es = entries();
  es.clear();
  const int n = gie_hip_band_config_count();
  for (Precision prec : {Precision::kFp16, Precision::kBf16}) {
    for (int ci = 0; ci < n; ++ci) {
      gie_band_config info;
      check_kernel_status(gie_hip_band_config_get(ci, &info), "band config query");
      for (int split : {1, 2, 4, 8}) es.push_back({ci, split, prec, info});
    }
  }
  if (es.size() > size_t(kMaxEntries)) throw Error(StatusCode::kInternal, "too many band registry entries");
  for (size_t i = 0; i < es.size(); ++i) {
    const Entry& en = es[i];
    KernelDesc k;
    k.name = std::string("band_") + to_string(en.precision) + "_" + std::to_string(en.info.kernel_h) + "x" +
             std::to_string(en.info.kernel_w) + "_" + std::to_string(en.info.tile_m) + "x" +
             std::to_string(en.info.tile_n) + "x" + std::to_string(en.info.tile_k) + "_s" +
             std::to_string(en.info.stages) + "_sk" + std::to_string(en.split);
    k.backend = Backend::kTensorCore;
    k.version = en.info.version;
    k.params = {{"block_m", en.info.tile_m}, {"block_n", en.info.tile_n}, {"block_k", en.info.tile_k},
                {"kernel_h", en.info.kernel_h}, {"kernel_w", en.info.kernel_w}, {"stages", en.info.stages},
                {"split_k", en.split}};
    k.threads_per_block = en.info.threads;
    k.tile_m = en.info.tile_m;
    k.tile_n = en.info.tile_n;
    k.tile_k = en.info.tile_k * en.info.kernel_h * en.info.kernel_w;
    k.uses_tensor_cores = true;
    k.launches = 2 + (en.split > 1 ? 1 : 0);
    fill_fns<0>(int(i), k);
    out.push_back(std::move(k));
  }
}

}  // namespace gie
