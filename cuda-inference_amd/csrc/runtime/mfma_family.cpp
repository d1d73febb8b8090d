// The gfx950 MFMA implicit-GEMM family as registry entries (the role of the reference's tcmma registration,
// src/kernels/tensor_core_mma.cu:264-395), rewritten around gfx950 limits:
//   * one fused repack dispatch (X NCHW->NHWC and W OIHW->ORSC, channels padded to a multiple of 8, so any
//     C runs: the reference needs C % 8 == 0 for this family), the MFMA kernel, and a reduce when split-K;
//   * capability filter: fp16/bf16 storage, a gfx950 MFMA device, LDS within the per-workgroup limit,
//     grid.y <= 65535, 32-bit repacked-image indexing, split needs >= 2 K tiles per slice, workspace <= 1/4 HBM;
//   * workspace = [xn | 256-B align][wk | align][split * |Y| FP32 partials | align].
// Every launch goes through the kernel C-ABI (include/gie_hip.h); nothing here allocates or synchronizes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <memory>
#include <string>
#include <vector>

#include "gie_hip.h"
#include "gpu_inference/kernel_registry.h"

namespace gie {
namespace {

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }
int c_pad_of(const ConvProblem& prob) { return (prob.p.in_channels + 7) / 8 * 8; }

struct WsLayout {
  size_t xn_off, wk_off, part_off, total;
};

WsLayout ws_layout(const ConvProblem& prob, int split) {
  const Conv2DParams& p = prob.p;
  const size_t cp = size_t(c_pad_of(prob));
  WsLayout l;
  l.xn_off = 0;
  l.wk_off = align256(size_t(p.batch) * p.in_h * p.in_w * cp * 2);
  l.part_off = l.wk_off + align256(size_t(p.out_channels) * p.kernel_h * p.kernel_w * cp * 2);
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

// Per-(config, split, precision) compile-time-free table: the registry stores one of these per entry, and the
// function pointers below look their entry up by index (KernelDesc holds plain function pointers).
struct Entry {
  int config;
  int split;
  Precision precision;
  gie_igemm_config info;
};

std::vector<Entry>& entries() {
  static std::vector<Entry> e;
  return e;
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
    const Conv2DParams& p = prob.p;
    if (size_t(en.info.lds_bytes) > dev.smem_per_block_optin)
      return no("needs " + std::to_string(en.info.lds_bytes / 1024) + " KiB LDS (limit " +
                std::to_string(dev.smem_per_block_optin / 1024) + " KiB)");
    if ((p.out_channels + en.info.tile_m - 1) / en.info.tile_m > 65535) return no("grid.y limit (65535) exceeded");
    const int cp = c_pad_of(prob);
    if (int64_t(p.in_h) * p.in_w * cp > 0x7fffffffLL) return no("repacked image exceeds 32-bit indexing");
    const int64_t kp = int64_t(p.kernel_h) * p.kernel_w * cp;
    if (kp > 0x7fffffffLL) return no("padded reduction exceeds 32-bit indexing");
    if (en.split > 1 && (kp + en.info.tile_k - 1) / en.info.tile_k < 2 * en.split)
      return no("reduction too short for this split-K factor");
    if (ws_layout(prob, en.split).total > dev.global_mem_bytes / 4)
      return no("workspace exceeds a quarter of device memory");
    return true;
  }
  static size_t workspace(const ConvProblem& prob) { return ws_layout(prob, e().split).total; }
  static size_t lds(const ConvProblem&) { return size_t(e().info.lds_bytes); }
  static int64_t blocks(const ConvProblem& prob) {
    const Entry& en = e();
    return ((prob.p.gemm_n() + en.info.tile_n - 1) / en.info.tile_n) *
           ((prob.p.gemm_m() + en.info.tile_m - 1) / en.info.tile_m) * en.split;
  }
  static double extra_traffic(const ConvProblem& prob) {
    // the repack reads X and W and writes their padded copies, which the GEMM then reads again;
    // split-K writes and re-reads FP32 partials
    const Conv2DParams& p = prob.p;
    const double cp = c_pad_of(prob);
    const double xw = double(p.input_shape().numel() + p.weight_shape().numel()) * 2.0;
    const double xwp = (double(p.batch) * p.in_h * p.in_w + double(p.out_channels) * p.kernel_h * p.kernel_w) * cp * 2.0;
    const double part = e().split > 1 ? 2.0 * e().split * double(p.output_shape().numel()) * 4.0 : 0.0;
    (void)xw;  // read once by the repack: part of the compulsory traffic already
    return 2.0 * xwp + part;
  }
  static int occupancy(const ConvProblem& prob) {
    int n = 1;
    if (gie_hip_igemm_occupancy(e().config, dtype_of(prob.precision), &n) != GIE_HIP_OK) {
      (void)hipGetLastError();
      n = 1;
    }
    return std::max(n, 1);
  }
  static void launch(const LaunchArgs& la) {
    const Entry& en = e();
    const ConvProblem& prob = *la.problem;
    const gie_conv_geom g = geom_of(prob);
    const WsLayout l = ws_layout(prob, en.split);
    char* ws = static_cast<char*>(la.workspace);
    void* xn = ws + l.xn_off;
    void* wk = ws + l.wk_off;
    float* part = en.split > 1 ? reinterpret_cast<float*>(ws + l.part_off) : nullptr;
    void* s = la.stream;
    const auto stage = [&](int k) { return la.only_stage < 0 || la.only_stage == k; };
    record_stage_event(la, 0);
    if (stage(0)) {
      check_kernel_status(gie_hip_repack_act_and_w(la.x, xn, la.w, wk, &g, s), "repack (NCHW->NHWC, OIHW->ORSC)");
    }
    record_stage_event(la, 1);
    if (stage(1)) {
      check_kernel_status(gie_hip_conv_igemm(en.config, dtype_of(prob.precision), &g, xn, wk, la.bias, la.y, part,
                                           en.split, s),
                        "MFMA implicit GEMM");
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

constexpr int kMaxEntries = 192;

template <int... Is>
struct FnTable {
  template <int I>
  static void fill(KernelDesc& k) {
    k.supports = &Fns<I>::supports;
    k.workspace_bytes = &Fns<I>::workspace;
    k.dynamic_smem_bytes = &Fns<I>::lds;
    k.num_blocks = &Fns<I>::blocks;
    k.extra_traffic_bytes = &Fns<I>::extra_traffic;
    k.blocks_per_cu = &Fns<I>::occupancy;
    k.launch = &Fns<I>::launch;
  }
};

template <int I>
void fill_fns(int idx, KernelDesc& k) {
  if constexpr (I < kMaxEntries) {
    if (idx == I) {
      FnTable<>::fill<I>(k);
      return;
    }
    fill_fns<I + 1>(idx, k);
  }
}

// Split-K factors registered for each tile configuration: long reductions over few output tiles need them
// (the reference registers sk2/4/8 variants of its small tiles, tensor_core_mma.cu:380-386).
std::vector<int> splits_for(const gie_igemm_config& c) {
  if (c.tile_m * c.tile_n <= 128 * 128) return {1, 2, 4, 8};
  return {1};
}

}  // namespace

void register_mfma_family(std::vector<KernelDesc>& out) {
  std::vector<Entry>& es = entries();
  es.clear();
  const int n = gie_hip_igemm_config_count();
  for (Precision prec : {Precision::kFp16, Precision::kBf16}) {
    for (int ci = 0; ci < n; ++ci) {
      gie_igemm_config info;
      check_kernel_status(gie_hip_igemm_config_get(ci, &info), "igemm config query");
      for (int split : splits_for(info)) es.push_back({ci, split, prec, info});
    }
  }
  if (es.size() > size_t(kMaxEntries)) throw Error(StatusCode::kInternal, "too many MFMA registry entries");
  for (size_t i = 0; i < es.size(); ++i) {
    const Entry& en = es[i];
    KernelDesc k;
    k.name = std::string("mfma_") + to_string(en.precision) + "_" + std::to_string(en.info.tile_m) + "x" +
             std::to_string(en.info.tile_n) + "x" + std::to_string(en.info.tile_k) + "_w" +
             std::to_string(en.info.waves_m) + "x" + std::to_string(en.info.waves_n) + "_s" +
             std::to_string(en.info.stages) + "_sk" + std::to_string(en.split);
    k.backend = Backend::kTensorCore;
    k.version = en.info.version;
    k.params = {{"block_m", en.info.tile_m}, {"block_n", en.info.tile_n}, {"block_k", en.info.tile_k},
                {"waves_m", en.info.waves_m}, {"waves_n", en.info.waves_n}, {"stages", en.info.stages},
                {"split_k", en.split}};
    k.threads_per_block = en.info.threads;
    k.tile_m = en.info.tile_m;
    k.tile_n = en.info.tile_n;
    k.tile_k = en.info.tile_k;
    k.uses_tensor_cores = true;
    k.launches = 2 + (en.split > 1 ? 1 : 0);
    fill_fns<0>(int(i), k);
    out.push_back(std::move(k));
  }
}

}  // namespace gie
