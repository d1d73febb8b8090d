// Implicit-GEMM convolution on gfx950 matrix cores (v_mfma_f32_16x16x32_{f16,bf16}), FP32 accumulation.
//
// GEMM view (reference naming): M = out_channels, N = batch*out_h*out_w output pixels, K = kh*kw*c_pad with k
// ordered (r, s, c) so 8 consecutive k are 8 consecutive channels of one input pixel in the NHWC repack — one
// 16-byte vector. Inside the kernel the MFMA "row" operand is the activation tile (pixels) and the "column"
// operand the weight tile (output channels): the 16x16 accumulator then gives each lane 4 consecutive output
// pixels of one output channel, which are contiguous in NCHW and leave as one 8-byte store.
//
// Workgroup: WP x WC wave64s own a TP(pixels) x TC(channels) output tile and walk K in BK slices.
//   * global -> registers with buffer loads: a lane whose row is outside the image / past the slice range /
//     past M gets an out-of-range offset and the hardware returns zeros, so the loads carry no branches and
//     the compiler's wait counting stays exact. Each thread owns fixed tile rows and one 16-byte K-chunk
//     column; the chunk's tap offset (r, s, c0) is the same for all of the thread's rows and advances without
//     division (branch-free when c_pad is a multiple of BK).
//   * PF register slots hold the next K slices in flight while LDS holds the slice being multiplied (two LDS
//     stages, unpadded rows with an xor swizzle of the 16-byte chunks so both the tile stores and the 16-row
//     fragment reads are free of bank conflicts); fragments of the next 32-wide k step are read while the
//     current one multiplies; one barrier per slice.
//   * epilogue: bias + ReLU on the FP32 accumulators, one RNE rounding, NCHW store (split == 1); or FP32
//     partials for split-K, summed by splitk_reduce.hip.
// Split-K slices follow the reference's partition rule [floor(kt*z/S), floor(kt*(z+1)/S))
// (src/kernels/tensor_core_mma.cu:112-115) and its partial layout partial[z][NCHW] (:231-234).
#include <mutex>
#include <set>
#include <utility>
#include <vector>

#include "device_common.h"

namespace gie_hip {
namespace {

struct Geom {
  int B, C, H, W, O, KH, KW, SH, SW, PH, PW, OH, OW, Cp, relu;
  int HWo;       // OH * OW
  int N;         // B * HWo output pixels
  int Kp;        // KH * KW * Cp
  int img;       // H * W * Cp elements per repacked image
  int xn_bytes;  // size of the repacked activations (buffer range)
  int wk_bytes;  // size of the repacked weights
};

// gfx9-family buffer descriptor word 3 (raw buffer, 32-bit data format): reads past num_records return 0.
constexpr int kBufferWord3 = 0x00020000;
constexpr int kOutOfRange = 0x80000000;

__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

template <int TP, int TC, int BK, int WP, int WC>
struct Shape {
  static constexpr int NT = WP * WC * 64;
  static constexpr int WTP = TP / WP, WTC = TC / WC;  // per-wave tile
  static constexpr int FP = WTP / 16, FC = WTC / 16;  // 16x16 MFMA blocks per wave
  static constexpr int LDK = BK;                      // LDS row pitch in 16-bit elements (swizzled)
  static constexpr int CPR = BK / 8;                  // 16-byte chunks per tile row
  static constexpr int LA = TP * CPR / NT, LB = TC * CPR / NT;
  static constexpr int kLds = 2 * (TP + TC) * LDK * 2;
  static_assert(TP % (WP * 16) == 0 && TC % (WC * 16) == 0, "wave tile must be a multiple of 16x16");
  static_assert(BK % 32 == 0, "BK must be a multiple of the MFMA K (32)");
  static_assert((TP * CPR) % NT == 0 && (TC * CPR) % NT == 0 && NT % CPR == 0, "chunks must divide over threads");
};

template <typename E, int TP, int TC, int BK, int WP, int WC, int PF, bool EXACT>
__global__ __launch_bounds__(WP * WC * 64) void igemm_kernel(const uint16_t* __restrict__ xn,
                                                             const uint16_t* __restrict__ wk,
                                                             const uint16_t* __restrict__ bias,
                                                             uint16_t* __restrict__ y, float* __restrict__ partial,
                                                             Geom g, int split) {
  using S = Shape<TP, TC, BK, WP, WC>;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  uint16_t* sA = reinterpret_cast<uint16_t*>(lds_raw);  // [2][TP][LDK] activations
  uint16_t* sB = sA + 2 * TP * S::LDK;                  // [2][TC][LDK] weights

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wp = wave / WC, wc = wave % WC;
  const int n0 = blockIdx.x * TP, m0 = blockIdx.y * TC;

  const int ktiles = (g.Kp + BK - 1) / BK;
  const int kt_begin = int((static_cast<long long>(ktiles) * blockIdx.z) / split);
  const int kt_end = int((static_cast<long long>(ktiles) * (blockIdx.z + 1)) / split);
  const int nk = kt_end - kt_begin;
  const int kc = tid % S::CPR;
  // chunk range of this slice set (chunks past the padded K or the slice end read as zeros)
  const int q_end = min(kt_end * S::CPR, g.Kp >> 3);

  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(xn), 0, g.xn_bytes,
                                                                      kBufferWord3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(wk), 0, g.wk_bytes,
                                                                      kBufferWord3);

  // Fixed rows of this thread: element offset of tap (0,0) channel 0 for each activation row, and the input
  // origin (hb, wb) for the bounds test; element offset of each weight row (or -1 past M).
  int a_off[S::LA], a_hb[S::LA], a_wb[S::LA];
#pragma unroll
  for (int i = 0; i < S::LA; ++i) {
    // selects, not branches: a divergent branch here makes the compiler clone the load paths below
    const int n_raw = n0 + (tid + i * S::NT) / S::CPR;
    const bool nv = n_raw < g.N;
    const int n = nv ? n_raw : 0;
    const int b = n / g.HWo;
    const int p = n - b * g.HWo;
    const int oh = p / g.OW, ow = p - (p / g.OW) * g.OW;
    const int hb = oh * g.SH - g.PH, wb = ow * g.SW - g.PW;
    a_hb[i] = nv ? hb : -0x40000000;  // an invalid row: every tap lands outside the image -> zeros
    a_wb[i] = wb;
    a_off[i] = b * g.img + (hb * g.W + wb) * g.Cp;
  }
  int b_off[S::LB];
#pragma unroll
  for (int i = 0; i < S::LB; ++i) {
    const int o = m0 + (tid + i * S::NT) / S::CPR;
    b_off[i] = o < g.O ? o * g.Kp : -1;
  }

  // K cursor of this thread's chunk column: chunk q -> tap (r, s), channel offset c0.
  int q = kt_begin * S::CPR + kc;
  const int cvec = g.Cp >> 3;
  int rs = q / cvec;
  int c0 = (q - rs * cvec) * 8;
  int r = rs / g.KW;
  int s = rs - r * g.KW;

  u32x4 ra[PF][S::LA], rb[PF][S::LB];
  // Loads the slice at the cursor into one register slot, then advances the cursor by one slice.
  auto gload = [&](u32x4(&A)[S::LA], u32x4(&B)[S::LB]) {
    // bitwise &, not &&: short-circuit evaluation would become divergent control flow around the loads
    const bool kok = q < q_end;
    const int tap = (r * g.W + s) * g.Cp + c0;
#pragma unroll
    for (int i = 0; i < S::LA; ++i) {
      const bool ok = kok & (static_cast<unsigned>(a_hb[i] + r) < static_cast<unsigned>(g.H)) &
                      (static_cast<unsigned>(a_wb[i] + s) < static_cast<unsigned>(g.W));
      A[i] = load16(xr, ok ? (a_off[i] + tap) * 2 : kOutOfRange);
    }
#pragma unroll
    for (int i = 0; i < S::LB; ++i) {
      const bool ok = kok & (b_off[i] >= 0);
      B[i] = load16(wr, ok ? (b_off[i] + q * 8) * 2 : kOutOfRange);
    }
    q += S::CPR;
    c0 += BK;
    if (EXACT) {  // c_pad % BK == 0: a slice never straddles two taps
      const bool wrap = c0 >= g.Cp;
      c0 = wrap ? c0 - g.Cp : c0;  // back to this thread's chunk column kc*8 of the next tap
      s += wrap ? 1 : 0;
      const bool wrap2 = s == g.KW;
      s = wrap2 ? 0 : s;
      r += wrap2 ? 1 : 0;
    } else {  // a slice spans several taps: recompute the tap from the chunk index (division, no branches)
      const int rs2 = q / cvec;
      c0 = (q - rs2 * cvec) * 8;
      r = rs2 / g.KW;
      s = rs2 - r * g.KW;
    }
  };
  // LDS rows are BK elements, unpadded; 16-byte chunk c of row r sits at chunk c ^ swz(r). swz takes the row's
  // position within a 256-byte bank period, so the row-major stores (CPR lanes per row) and the 16-row fragment
  // reads (16 lanes, one chunk column) both spread over all 64 banks.
  auto swz = [](int row) { return ((row * S::CPR) >> 4) % S::CPR; };
  auto sstore = [&](int st, const u32x4(&A)[S::LA], const u32x4(&B)[S::LB]) {
#pragma unroll
    for (int i = 0; i < S::LA; ++i) {
      const int row = (tid + i * S::NT) / S::CPR;
      *reinterpret_cast<u32x4*>(sA + (st * TP + row) * S::LDK + ((kc ^ swz(row)) * 8)) = A[i];
    }
#pragma unroll
    for (int i = 0; i < S::LB; ++i) {
      const int row = (tid + i * S::NT) / S::CPR;
      *reinterpret_cast<u32x4*>(sB + (st * TC + row) * S::LDK + ((kc ^ swz(row)) * 8)) = B[i];
    }
  };

  f32x4 acc[S::FP][S::FC];
#pragma unroll
  for (int i = 0; i < S::FP; ++i)
#pragma unroll
    for (int j = 0; j < S::FC; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // MFMA fragment of 16 rows: lane reads row (lane & 15), k-chunk kk*4 + (lane >> 4) of the 32-wide step kk.
  // Fragment row bases are multiples of 16, so the swizzle depends on (lane & 15) only.
  const int frag_row = lane & 15, frag_c = lane >> 4, frag_sw = swz(frag_row);
  auto rdfrag = [&](int st, int kk, u32x4(&af)[S::FP], u32x4(&bf)[S::FC]) {
    const int col = ((kk * 4 + frag_c) ^ frag_sw) * 8;
    const uint16_t* tA = sA + (st * TP + wp * S::WTP + frag_row) * S::LDK + col;
    const uint16_t* tB = sB + (st * TC + wc * S::WTC + frag_row) * S::LDK + col;
#pragma unroll
    for (int i = 0; i < S::FP; ++i) af[i] = *reinterpret_cast<const u32x4*>(tA + i * 16 * S::LDK);
#pragma unroll
    for (int j = 0; j < S::FC; ++j) bf[j] = *reinterpret_cast<const u32x4*>(tB + j * 16 * S::LDK);
  };
  auto mma = [&](const u32x4(&af)[S::FP], const u32x4(&bf)[S::FC]) {
#pragma unroll
    for (int i = 0; i < S::FP; ++i)
#pragma unroll
      for (int j = 0; j < S::FC; ++j) acc[i][j] = E::mfma(af[i], bf[j], acc[i][j]);
  };
  // One slice: refill register slot `st` with slice it + PF, multiply slice it from LDS stage it & 1 with the
  // fragments of step kk + 1 read while step kk multiplies, commit slice it + 1 (slot (st + 1) % PF) to the
  // other stage, meet at one barrier. No branch inside, so the compiler interleaves the LDS stores and the
  // buffer loads with the MFMAs.
  auto slice = [&](int it, u32x4(&rs_a)[S::LA], u32x4(&rs_b)[S::LB], const u32x4(&nx_a)[S::LA],
                   const u32x4(&nx_b)[S::LB]) {
    constexpr int KK = BK / 32;
    u32x4 af[2][S::FP], bf[2][S::FC];
    rdfrag(it & 1, 0, af[0], bf[0]);
    gload(rs_a, rs_b);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK) rdfrag(it & 1, kk + 1, af[(kk + 1) & 1], bf[(kk + 1) & 1]);
      mma(af[kk & 1], bf[kk & 1]);
    }
    sstore((it + 1) & 1, nx_a, nx_b);
    __syncthreads();
  };

  // Register slot it % PF holds slice it (PF slices in flight). The loop runs whole groups of PF slices, then
  // the remaining nk % PF slices one by one (uniform branches); loads past the last slice read zeros.
#pragma unroll
  for (int st = 0; st < PF; ++st) gload(ra[st], rb[st]);
  sstore(0, ra[0], rb[0]);
  __syncthreads();

  int base = 0;
  for (; base + PF <= nk; base += PF) {
#pragma unroll
    for (int st = 0; st < PF; ++st) slice(base + st, ra[st], rb[st], ra[(st + 1) % PF], rb[(st + 1) % PF]);
  }
#pragma unroll
  for (int st = 0; st + 1 < PF; ++st) {
    if (base + st < nk) slice(base + st, ra[st], rb[st], ra[(st + 1) % PF], rb[(st + 1) % PF]);
  }

  // Epilogue. Lane holds, for MFMA block (i, j), pixels nb..nb+3 of output channel o.
  float bv[S::FC];
#pragma unroll
  for (int j = 0; j < S::FC; ++j) {
    const int o = m0 + wc * S::WTC + j * 16 + (lane & 15);
    bv[j] = (split == 1 && bias != nullptr && o < g.O) ? E::to_f32(bias[o]) : 0.0f;
  }
  const long long total = static_cast<long long>(g.N) * g.O;
#pragma unroll
  for (int i = 0; i < S::FP; ++i) {
    const int nb = n0 + wp * S::WTP + i * 16 + (lane >> 4) * 4;
    if (nb >= g.N) continue;
    const int b = nb / g.HWo;
    const int p = nb - b * g.HWo;
    const bool whole = nb + 3 < g.N && p + 3 < g.HWo;  // 4 pixels, same image
#pragma unroll
    for (int j = 0; j < S::FC; ++j) {
      const int o = m0 + wc * S::WTC + j * 16 + (lane & 15);
      if (o >= g.O) continue;
      const f32x4 v = acc[i][j];
      const long long idx = (static_cast<long long>(b) * g.O + o) * g.HWo + p;
      if (split > 1) {
        float* pz = partial + blockIdx.z * total;
        if (whole && (reinterpret_cast<uintptr_t>(pz + idx) & 15u) == 0) {
          *reinterpret_cast<f32x4*>(pz + idx) = v;
        } else {
          for (int e = 0; e < 4; ++e) {
            const int n = nb + e;
            if (n >= g.N) break;
            const int be = n / g.HWo, pe = n - be * g.HWo;
            pz[(static_cast<long long>(be) * g.O + o) * g.HWo + pe] = v[e];
          }
        }
      } else {
        uint16_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float a = v[e] + bv[j];  // bias added to the FP32 accumulator, then ReLU, then one rounding
          if (g.relu) a = fmaxf(a, 0.0f);
          h[e] = E::from_f32(a);
        }
        uint16_t* dst = y + idx;
        if (whole && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
          *reinterpret_cast<u32x2*>(dst) = u32x2{uint32_t(h[0]) | (uint32_t(h[1]) << 16),
                                                 uint32_t(h[2]) | (uint32_t(h[3]) << 16)};
        } else {
          for (int e = 0; e < 4; ++e) {
            const int n = nb + e;
            if (n >= g.N) break;
            const int be = n / g.HWo, pe = n - be * g.HWo;
            y[(static_cast<long long>(be) * g.O + o) * g.HWo + pe] = h[e];
          }
        }
      }
    }
  }
}

// ---- registered configurations --------------------------------------------------------------------------------
typedef void (*KernelFn)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*, Geom, int);

struct Config {
  gie_igemm_config info;
  KernelFn fp16[2], bf16[2];  // [EXACT]: c_pad % tile_k == 0 takes the branch-free cursor
};

template <int TP, int TC, int BK, int WP, int WC, int PF>
Config make_config(int version) {
  using S = Shape<TP, TC, BK, WP, WC>;
  Config c;
  // reference naming: M = out channels (TC here), N = pixels (TP here)
  c.info.tile_m = TC;
  c.info.tile_n = TP;
  c.info.tile_k = BK;
  c.info.waves_m = WC;
  c.info.waves_n = WP;
  c.info.threads = S::NT;
  c.info.lds_bytes = S::kLds;
  c.info.stages = PF;
  c.info.version = version;
  c.fp16[0] = &igemm_kernel<Fp16, TP, TC, BK, WP, WC, PF, false>;
  c.fp16[1] = &igemm_kernel<Fp16, TP, TC, BK, WP, WC, PF, true>;
  c.bf16[0] = &igemm_kernel<Bf16, TP, TC, BK, WP, WC, PF, false>;
  c.bf16[1] = &igemm_kernel<Bf16, TP, TC, BK, WP, WC, PF, true>;
  return c;
}

const std::vector<Config>& configs() {
  static const std::vector<Config> table = [] {
    std::vector<Config> t;
    //            pixels x channels x k, waves (pixels x channels), register pipeline depth
    // four waves (one per SIMD)
    t.push_back(make_config<128, 128, 32, 2, 2, 4>(4));
    t.push_back(make_config<128, 128, 64, 2, 2, 3>(4));
    t.push_back(make_config<128, 64, 32, 2, 2, 4>(4));
    t.push_back(make_config<128, 64, 64, 2, 2, 3>(4));
    t.push_back(make_config<64, 128, 32, 2, 2, 4>(4));
    t.push_back(make_config<64, 128, 64, 2, 2, 3>(4));
    t.push_back(make_config<64, 64, 32, 2, 2, 4>(4));
    t.push_back(make_config<64, 64, 64, 2, 2, 4>(4));
    t.push_back(make_config<32, 64, 64, 1, 2, 4>(4));
    // eight waves (two per SIMD): twice the loads and LDS reads in flight per CU
    t.push_back(make_config<256, 128, 32, 4, 2, 3>(4));
    t.push_back(make_config<128, 256, 32, 2, 4, 3>(4));
    t.push_back(make_config<128, 64, 64, 4, 2, 4>(4));
    t.push_back(make_config<64, 128, 64, 2, 4, 3>(4));
    t.push_back(make_config<128, 128, 64, 2, 4, 3>(4));
    t.push_back(make_config<128, 128, 32, 4, 2, 4>(4));
    t.push_back(make_config<64, 64, 64, 2, 4, 4>(4));
    t.push_back(make_config<256, 64, 64, 4, 2, 2>(4));
    t.push_back(make_config<64, 128, 128, 2, 4, 2>(4));
    t.push_back(make_config<128, 64, 128, 4, 2, 2>(4));
    t.push_back(make_config<128, 128, 128, 2, 4, 2>(4));
    return t;
  }();
  return table;
}

int set_lds_limit(KernelFn fn, int bytes) {
  if (bytes <= 64 * 1024) return GIE_HIP_OK;
  return lds_opt_in(reinterpret_cast<const void*>(fn), bytes);
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_igemm_config_count(void) { return int(configs().size()); }

extern "C" int gie_hip_igemm_config_get(int index, gie_igemm_config* out) {
  if (index < 0 || index >= int(configs().size()) || !out) return GIE_HIP_EINVAL;
  *out = configs()[size_t(index)].info;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_igemm_occupancy(int index, int dtype, int* blocks_per_cu) {
  if (index < 0 || index >= int(configs().size()) || !blocks_per_cu) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  const Config& c = configs()[size_t(index)];
  KernelFn fn = dtype == GIE_HIP_FP16 ? c.fp16[1] : c.bf16[1];
  if (int rc = set_lds_limit(fn, c.info.lds_bytes)) return rc;
  int n = 0;
  const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn),
                                                                     c.info.threads, size_t(c.info.lds_bytes));
  if (e != hipSuccess) return int(e);
  *blocks_per_cu = n;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_conv_igemm(int config, int dtype, const gie_conv_geom* gg, const void* xn, const void* wk,
                                  const void* bias, void* y, float* partial, int split, void* stream) {
  if (config < 0 || config >= int(configs().size()) || !gg || !xn || !wk) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if (split < 1 || split > 64) return GIE_HIP_EINVAL;
  if (split == 1 && !y) return GIE_HIP_EINVAL;
  if (split > 1 && (!partial || (reinterpret_cast<uintptr_t>(partial) & 15u) != 0)) return GIE_HIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(xn) & 15u) != 0 || (reinterpret_cast<uintptr_t>(wk) & 15u) != 0)
    return GIE_HIP_EINVAL;
  const Config& c = configs()[size_t(config)];
  Geom g;
  g.B = gg->batch;
  g.C = gg->in_channels;
  g.H = gg->in_h;
  g.W = gg->in_w;
  g.O = gg->out_channels;
  g.KH = gg->kernel_h;
  g.KW = gg->kernel_w;
  g.SH = gg->stride_h;
  g.SW = gg->stride_w;
  g.PH = gg->pad_h;
  g.PW = gg->pad_w;
  g.OH = gg->out_h;
  g.OW = gg->out_w;
  g.Cp = gg->c_pad;
  g.relu = gg->relu ? 1 : 0;
  if (g.B <= 0 || g.C <= 0 || g.H <= 0 || g.W <= 0 || g.O <= 0 || g.KH <= 0 || g.KW <= 0 || g.SH <= 0 || g.SW <= 0 ||
      g.PH < 0 || g.PW < 0 || g.OH <= 0 || g.OW <= 0 || g.Cp < g.C || (g.Cp & 7) != 0)
    return GIE_HIP_EINVAL;
  // every offset the kernel forms in 32 bits must fit, and the buffer ranges stay below the out-of-range marker
  const long long hwo = static_cast<long long>(g.OH) * g.OW;
  const long long n = hwo * g.B;
  const long long kp = static_cast<long long>(g.KH) * g.KW * g.Cp;
  const long long img = static_cast<long long>(g.H) * g.W * g.Cp;
  const long long xbytes = img * g.B * 2, wbytes = kp * g.O * 2;
  if (n > 0x7fffffffLL || kp > 0x7fffffffLL || xbytes >= 0x7fffffffLL || wbytes >= 0x7fffffffLL)
    return GIE_HIP_EUNSUPPORTED;
  g.HWo = int(hwo);
  g.N = int(n);
  g.Kp = int(kp);
  g.img = int(img);
  g.xn_bytes = int(xbytes);
  g.wk_bytes = int(wbytes);
  const long long gx = (n + c.info.tile_n - 1) / c.info.tile_n;
  const long long gy = (g.O + c.info.tile_m - 1) / c.info.tile_m;
  if (gx > 0x7fffffffLL || gy > 65535) return GIE_HIP_EUNSUPPORTED;
  const int exact = (g.Cp % c.info.tile_k) == 0 ? 1 : 0;
  KernelFn fn = dtype == GIE_HIP_FP16 ? c.fp16[exact] : c.bf16[exact];
  if (int rc = set_lds_limit(fn, c.info.lds_bytes)) return rc;
  hipLaunchKernelGGL(fn, dim3(unsigned(gx), unsigned(gy), unsigned(split)), dim3(c.info.threads), c.info.lds_bytes,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(xn),
                     static_cast<const uint16_t*>(wk), static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y),
                     partial, g, split);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
