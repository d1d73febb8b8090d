// Halo-tiled implicit-GEMM convolution on gfx950 matrix cores (v_mfma_f32_32x32x16_{f16,bf16}, FP32
// accumulation) over the repacked activations xn [B][H][W][Cp] and weights wk [O][KH*KW][Cp]
// (Cp = in_channels rounded up to 8, zero padded; the fused repack dispatch of repack.hip writes both).
//
// GEMM view (reference naming): M = out_channels, N = batch*out_h*out_w output pixels, K = kh*kw*Cp. A workgroup
// owns TO output channels x TPX consecutive output pixels (a flat range that may span image rows and images)
// and walks the channels in slices of 32. Per slice it stages in LDS:
//   * the input "halo": every input row the tile's pixels touch, one LDS row ("slot") per (image, input row),
//     each pixel's 32 channels contiguous (64 bytes, padded to 80 so 16 consecutive pixels hit distinct banks);
//     columns and rows outside the image are zeros. Consecutive output rows of one image share slots (stride 1:
//     tap row r of output row j reads slot j + r), so each input pixel is loaded once per slice and read by all
//     KH*KW taps from LDS — the implicit GEMM never re-fetches activations per tap;
//   * the weights [TO][KH*KW][32 channels] (row pitch padded by 16 bytes for the same bank spread).
// Every global load is a 16-byte vector (8 channels) into registers, then a 16-byte LDS store; no VALU work
// besides addresses.
// Waves: (TPX/64 pixel halves) x (KH filter rows) x (2 channel halves) = 12 waves for 3x3 — three per SIMD, so
// one wave's loads, LDS reads and waits overlap the others' MFMAs. Each wave multiplies a 64-pixel x 64-channel
// tile (2 x 2 blocks of 32x32) for its filter row's KW taps and its 16 channels of the slice; the KH*2 partial
// tiles of each pixel half are summed through LDS after the last slice.
// Pipeline: global loads of slice i+1 go to registers while slice i multiplies from one LDS stage (fragments of
// tap t+2 in flight while tap t multiplies); then the registers go to the other stage and the workgroup meets at
// one barrier per slice. Loads past the data (image borders, padding rows/columns, channels past Cp, output
// channels past O, the slice after the last) use an out-of-range buffer offset, for which the hardware returns
// zeros, so the loop has no divergent branches.
// Epilogue: bias + ReLU on the FP32 sums, one RNE rounding; the 16-bit tile goes through LDS so waves store
// contiguous runs of output pixels (8-byte stores when 4 pixels share an image row and the address allows, else
// 2-byte stores). Or FP32 partials partial[z][NCHW] for split-K (reduced by splitk_reduce.hip).
// Split-K slices follow the reference's partition rule [floor(ns*z/S), floor(ns*(z+1)/S))
// (src/kernels/tensor_core_mma.cu:112-115) over channel slices, and its partial layout (:231-234).
#include <mutex>
#include <set>
#include <utility>
#include <vector>

#include "device_common.h"

namespace gie_hip {
namespace {

struct HaloGeom {
  int B, Cp, H, W, O, SH, SW, PH, PW, OH, OW;
  int HWo, N;
  int WPAD;     // LDS pixels per slot: (OW - 1) * SW + KW
  int E;        // slot gap at an image boundary: max(KH - SH, 0)
  int nslices;  // ceil(Cp / 32)
  int x_bytes, w_bytes;
  int relu;
  int act_stage;  // bytes of the activation part of one LDS stage
};

constexpr int kBufferWord3 = 0x00020000;
constexpr int kOut = 0x80000000;  // buffer offset past any range: loads return zeros
constexpr int kSlotTable = 256;   // bytes at the start of LDS: slot -> pixel offset of (b, ih, 0), or -1
constexpr int kMaxSlots = kSlotTable / 4;
constexpr int kMaxStagedPixels = 384;  // slots x WPAD of the largest tile (the host checks)
constexpr int kCS = 32;                // channels per slice
constexpr int kPXB = kCS * 2 + 16;     // LDS bytes per staged pixel

template <int KH, int KW, int TO, int TPX>
struct HShape {
  static constexpr int RS = KH * KW;
  static constexpr int WP = TPX / 64;   // pixel-half waves
  static constexpr int WK = KH * 2;     // K groups: filter row x channel half
  static constexpr int NT = WP * WK * 64;
  static constexpr int FO = TO / 32;    // 32-channel MFMA blocks per wave
  static constexpr int OPITCH = RS * kCS * 2 + 16;  // LDS bytes per output channel of the weight tile
  static constexpr int WST = TO * OPITCH;
  static constexpr int WIT = TO * RS * 4 / NT;         // 16-byte weight chunks per thread per slice
  static constexpr int AIT = (kMaxStagedPixels * 4 + NT - 1) / NT;  // activation chunks per thread (max)
  static constexpr int ACC = 2 * FO * 4 * 64 * 16;   // bytes of one wave's FP32 tile in LDS
  static constexpr int TROW = TPX * 2 + 8;            // 16-bit output tile row pitch
  static_assert(TPX % 64 == 0 && TO % 32 == 0, "tile must be whole waves");
  static_assert((TO * RS * 4) % NT == 0, "weight chunks must divide over threads");
  static_assert(WK == 2 || WK == 6, "reduction rounds are written for 1 or 3 filter rows");
};

__device__ __forceinline__ u32x4 ld128(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

template <typename E, int KH, int KW, int TO, int TPX>
__global__ __launch_bounds__(TPX / 64 * KH * 2 * 64) void halo_kernel(
    const uint16_t* __restrict__ xn, const uint16_t* __restrict__ wk, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ y, float* __restrict__ partial, HaloGeom g, int split) {
  using S = HShape<KH, KW, TO, TPX>;
  constexpr int RS = S::RS, NT = S::NT, FO = S::FO, OPITCH = S::OPITCH;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  int* slot_tab = reinterpret_cast<int*>(lds);
  const int stage_bytes = g.act_stage + S::WST;
  unsigned char* stage0 = lds + kSlotTable;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kg = wave % S::WK, wp = wave / S::WK;  // K group (filter row kg/2, channel half kg%2), pixel half
  const int wr = kg >> 1, wh = kg & 1;
  const int n_ot = (g.O + TO - 1) / TO;
  const int ot = int(blockIdx.x) % n_ot, pt = int(blockIdx.x) / n_ot;  // neighbours share pixels, XCDs share o
  const int o0 = ot * TO, P0 = pt * TPX;
  const int Pend = min(P0 + TPX, g.N);

  // ---- slot table: output row j of the tile, tap row r -> slot j*SH + r + E*(image - first image) ----------
  const int rf0 = P0 / g.OW, rfL = (Pend - 1) / g.OW;
  const int b0 = rf0 / g.OH, bL = rfL / g.OH;
  const int NS = (rfL - rf0) * g.SH + g.E * (bL - b0) + KH;
  for (int s = tid; s < kMaxSlots; s += NT) slot_tab[s] = -1;
  __syncthreads();
  for (int j = tid; j <= rfL - rf0; j += NT) {
    const int rf = rf0 + j, b = rf / g.OH, oh = rf - b * g.OH;
    const int base = j * g.SH + g.E * (b - b0);
#pragma unroll
    for (int r = 0; r < KH; ++r) {
      const int ih = oh * g.SH - g.PH + r;
      slot_tab[base + r] = (ih >= 0 && ih < g.H) ? (b * g.H + ih) * g.W : -1;
    }
  }
  __syncthreads();

  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(xn), 0, g.x_bytes,
                                                                      kBufferWord3);
  const __amdgpu_buffer_rsrc_t wr_ = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(wk), 0, g.w_bytes,
                                                                       kBufferWord3);

  // ---- activation chunks: (slot, column, 16-byte chunk), chunks fastest (64 contiguous bytes per pixel) -------
  const int ntask = NS * g.WPAD * 4;
  int a_goff[S::AIT], a_lds[S::AIT], a_ch[S::AIT];
#pragma unroll
  for (int i = 0; i < S::AIT; ++i) {
    const int t = tid + i * NT;
    const bool valid = t < ntask;
    const int tt = valid ? t : 0;
    const int chunk = tt & 3, pix = tt >> 2;
    const int slot = pix / g.WPAD, col = pix - slot * g.WPAD;
    const int so = slot_tab[slot], iw = col - g.PW;
    const bool in = valid && so >= 0 && iw >= 0 && iw < g.W;
    a_goff[i] = in ? ((so + iw) * g.Cp + chunk * 8) * 2 : kOut;
    a_lds[i] = valid ? pix * kPXB + chunk * 16 : g.act_stage - 16;  // spare chunk for idle lanes
    a_ch[i] = chunk * 8;
  }
  // ---- weight chunks: (output channel, tap, 16-byte chunk) ---------------------------------------------------------
  int w_goff[S::WIT], w_lds[S::WIT], w_ch[S::WIT];
#pragma unroll
  for (int i = 0; i < S::WIT; ++i) {
    const int t = tid + i * NT;
    const int chunk = t & 3, ot_ = t >> 2;
    const int tap = ot_ % RS, o = ot_ / RS;
    w_goff[i] = (o0 + o < g.O) ? (((o0 + o) * RS + tap) * g.Cp + chunk * 8) * 2 : kOut;
    w_lds[i] = o * OPITCH + tap * kCS * 2 + chunk * 16;
    w_ch[i] = chunk * 8;
  }

  u32x4 ra[S::AIT], rw[S::WIT];
  auto gload = [&](int sl, bool live) {
    const int c0 = sl * kCS;
    const int cbytes = c0 * 2;
    // a chunk past Cp (last slice of a channel count that is not a multiple of 32) reads zeros
#pragma unroll
    for (int i = 0; i < S::AIT; ++i)
      ra[i] = ld128(xr, (live & (c0 + a_ch[i] < g.Cp) & (a_goff[i] != kOut)) ? a_goff[i] + cbytes : kOut);
#pragma unroll
    for (int i = 0; i < S::WIT; ++i)
      rw[i] = ld128(wr_, (live & (c0 + w_ch[i] < g.Cp) & (w_goff[i] != kOut)) ? w_goff[i] + cbytes : kOut);
  };
  auto sstore = [&](unsigned char* st) {
#pragma unroll
    for (int i = 0; i < S::AIT; ++i) *reinterpret_cast<u32x4*>(st + a_lds[i]) = ra[i];
    unsigned char* wst = st + g.act_stage;
#pragma unroll
    for (int i = 0; i < S::WIT; ++i) *reinterpret_cast<u32x4*>(wst + w_lds[i]) = rw[i];
  };
  // ---- per-lane fragment addresses ------------------------------------------------------------------------------
  const int chunk = wh * 2 + (lane >> 5);  // which 8 channels of the slice this lane feeds
  int a_addr[2];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    const int px_raw = P0 + wp * 64 + pb * 32 + (lane & 31);
    const int px = px_raw < g.N ? px_raw : P0;  // rows past N multiply a valid pixel; never stored
    const int rf = px / g.OW, ow = px - rf * g.OW, b = rf / g.OH;
    const int slot0 = (rf - rf0) * g.SH + g.E * (b - b0) + wr;  // this wave's filter row
    a_addr[pb] = (slot0 * g.WPAD + ow * g.SW) * kPXB + chunk * 16;
  }
  int b_addr[FO];
#pragma unroll
  for (int ob = 0; ob < FO; ++ob)
    b_addr[ob] = g.act_stage + (ob * 32 + (lane & 31)) * OPITCH + wr * KW * kCS * 2 + chunk * 16;

  f32x16 acc[2][FO];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb)
#pragma unroll
    for (int ob = 0; ob < FO; ++ob) acc[pb][ob] = f32x16{};

  // tap s of this wave's filter row: the activation pixel moves by s columns, the weight by one tap
  auto rdfrag = [&](const unsigned char* st, int s, u32x4(&af)[2], u32x4(&bf)[FO]) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) af[pb] = *reinterpret_cast<const u32x4*>(st + a_addr[pb] + s * kPXB);
#pragma unroll
    for (int ob = 0; ob < FO; ++ob) bf[ob] = *reinterpret_cast<const u32x4*>(st + b_addr[ob] + s * kCS * 2);
  };
  // Fragments of tap s + 2 are read while tap s multiplies (three register sets); the scheduling groups pin
  // that order, which the compiler's own scheduler would otherwise collapse into read-wait-multiply.
  auto compute = [&](const unsigned char* st) {
    constexpr int NR = 2 + FO;  // LDS reads per tap
    u32x4 af[3][2], bf[3][FO];
    rdfrag(st, 0, af[0], bf[0]);
    if (KW > 1) rdfrag(st, 1, af[1], bf[1]);
#pragma unroll
    for (int s = 0; s < KW; ++s) {
      if (s + 2 < KW) rdfrag(st, s + 2, af[(s + 2) % 3], bf[(s + 2) % 3]);
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int ob = 0; ob < FO; ++ob) acc[pb][ob] = E::mfma32(af[s % 3][pb], bf[s % 3][ob], acc[pb][ob]);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, KW > 1 ? 2 * NR : NR, 0);
#pragma unroll
    for (int s = 0; s < KW; ++s) {
      if (s + 2 < KW) __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * FO, 0);
    }
  };

  // ---- main loop over this workgroup's channel slices ----------------------------------------------------------
  const int z = int(blockIdx.z);
  const int sl0 = int((static_cast<long long>(g.nslices) * z) / split);
  const int sl1 = int((static_cast<long long>(g.nslices) * (z + 1)) / split);
  gload(sl0, sl0 < sl1);
  sstore(stage0);
  __syncthreads();
  for (int sl = sl0; sl < sl1; ++sl) {
    unsigned char* cur = stage0 + ((sl - sl0) & 1) * stage_bytes;
    unsigned char* nxt = stage0 + (((sl - sl0) & 1) ^ 1) * stage_bytes;
    gload(sl + 1, sl + 1 < sl1);  // zeros after the last slice: no branch around the loads
    __builtin_amdgcn_sched_barrier(0);  // the loads leave before the multiplies start
    compute(cur);
    __builtin_amdgcn_sched_barrier(0);
    sstore(nxt);
    __syncthreads();
  }

  // ---- epilogue: sum the K groups of each pixel half through LDS -------------------------------------------------
  // slot q of pixel half wp holds one wave's 64x64 FP32 tile, lane-major so every access is a whole 1 KiB row
  f32x4* red = reinterpret_cast<f32x4*>(stage0);
  auto red_idx = [&](int q, int pb, int ob, int r4) {
    return ((((wp * 3 + q) * 2 + pb) * FO + ob) * 4 + r4) * 64 + lane;
  };
  auto put = [&](int q) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int ob = 0; ob < FO; ++ob)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          red[red_idx(q, pb, ob, r4)] = f32x4{acc[pb][ob][4 * r4], acc[pb][ob][4 * r4 + 1], acc[pb][ob][4 * r4 + 2],
                                              acc[pb][ob][4 * r4 + 3]};
  };
  auto add = [&](int q) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int ob = 0; ob < FO; ++ob)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 v = red[red_idx(q, pb, ob, r4)];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[pb][ob][4 * r4 + e] += v[e];
        }
  };
  if (S::WK == 6) {  // 6 -> 3 -> 1
    if (kg >= 3) put(kg - 3);
    __syncthreads();
    if (kg < 3) add(kg);
    __syncthreads();
    if (kg == 1 || kg == 2) put(kg - 1);
    __syncthreads();
    if (kg == 0) {
      add(0);
      add(1);
    }
  } else {  // 2 -> 1
    if (kg == 1) put(0);
    __syncthreads();
    if (kg == 0) add(0);
  }
  // 32x32 accumulator layout: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4 (pixel), column l%32 (channel)
  if (split > 1) {
    if (kg == 0) {
      float* pz = partial + static_cast<long long>(z) * g.N * g.O;
#pragma unroll
      for (int ob = 0; ob < FO; ++ob) {
        const int o = o0 + ob * 32 + (lane & 31);
        if (o >= g.O) continue;
#pragma unroll
        for (int pb = 0; pb < 2; ++pb)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int px = P0 + wp * 64 + pb * 32 + 8 * r4 + 4 * (lane >> 5);
            if (px >= g.N) continue;
            const int b = px / g.HWo, p = px - b * g.HWo;
            float* dst = pz + (static_cast<long long>(b) * g.O + o) * g.HWo + p;
            if (px + 3 < g.N && p + 3 < g.HWo && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
              *reinterpret_cast<f32x4*>(dst) = f32x4{acc[pb][ob][4 * r4], acc[pb][ob][4 * r4 + 1],
                                                     acc[pb][ob][4 * r4 + 2], acc[pb][ob][4 * r4 + 3]};
            } else {
              for (int e = 0; e < 4 && px + e < g.N; ++e) {
                const int be = (px + e) / g.HWo, pe = px + e - be * g.HWo;
                pz[(static_cast<long long>(be) * g.O + o) * g.HWo + pe] = acc[pb][ob][4 * r4 + e];
              }
            }
          }
      }
    }
    return;
  }
  // the 16-bit tile lives past the reduction slots still being read by the other pixel half
  unsigned char* tile = stage0 + S::WP * 2 * S::ACC;  // [TO][TPX] 16-bit, row pitch TROW
  if (kg == 0) {
#pragma unroll
    for (int ob = 0; ob < FO; ++ob) {
      const int ol = ob * 32 + (lane & 31);
      const int o = o0 + ol;
      const float bv = (bias != nullptr && o < g.O) ? E::to_f32(bias[o]) : 0.0f;
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          uint32_t hv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float a = acc[pb][ob][4 * r4 + e] + bv;  // bias on the FP32 sum, then ReLU, then one rounding
            if (g.relu) a = fmaxf(a, 0.0f);
            hv[e] = E::from_f32(a);
          }
          const int pl = wp * 64 + pb * 32 + 8 * r4 + 4 * (lane >> 5);
          *reinterpret_cast<u32x2*>(tile + ol * S::TROW + pl * 2) = u32x2{hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16)};
        }
    }
  }
  __syncthreads();
  constexpr int G4 = TPX / 4;
  for (int idx = tid; idx < TO * G4; idx += NT) {
    const int ol = idx / G4, q = idx - (idx / G4) * G4;
    const int o = o0 + ol, px = P0 + 4 * q;
    if (o >= g.O || px >= g.N) continue;
    const u32x2 v = *reinterpret_cast<const u32x2*>(tile + ol * S::TROW + q * 8);
    const int b = px / g.HWo, p = px - b * g.HWo;
    uint16_t* dst = y + (static_cast<long long>(b) * g.O + o) * g.HWo + p;
    if (px + 3 < g.N && p + 3 < g.HWo && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
      *reinterpret_cast<u32x2*>(dst) = v;
    } else {
      const uint16_t hv[4] = {uint16_t(v[0]), uint16_t(v[0] >> 16), uint16_t(v[1]), uint16_t(v[1] >> 16)};
      for (int e = 0; e < 4 && px + e < g.N; ++e) {
        const int be = (px + e) / g.HWo, pe = px + e - be * g.HWo;
        y[(static_cast<long long>(be) * g.O + o) * g.HWo + pe] = hv[e];
      }
    }
  }
}

// ---- registered configurations ----------------------------------------------------------------------------------
typedef void (*HaloFn)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*, HaloGeom, int);

struct HaloConfig {
  gie_halo_config info;
  int wst, acc, trow, ait;
  HaloFn fn[2];  // [fp16, bf16]
};

template <int KH, int KW, int TO, int TPX>
HaloConfig make_halo(int version) {
  using S = HShape<KH, KW, TO, TPX>;
  HaloConfig c;
  c.info.tile_m = TO;
  c.info.tile_n = TPX;
  c.info.tile_k = kCS;
  c.info.kernel_h = KH;
  c.info.kernel_w = KW;
  c.info.threads = S::NT;
  c.info.version = version;
  c.wst = S::WST;
  c.acc = S::ACC;
  c.trow = S::TROW;
  c.ait = S::AIT;
  c.fn[0] = &halo_kernel<Fp16, KH, KW, TO, TPX>;
  c.fn[1] = &halo_kernel<Bf16, KH, KW, TO, TPX>;
  return c;
}

const std::vector<HaloConfig>& halo_configs() {
  static const std::vector<HaloConfig> t = [] {
    std::vector<HaloConfig> v;
    //                KH KW  TO  TPX
    v.push_back(make_halo<3, 3, 64, 128>(2));
    v.push_back(make_halo<1, 1, 64, 128>(2));
    v.push_back(make_halo<1, 1, 128, 128>(2));
    return v;
  }();
  return t;
}

constexpr int kLdsLimit = 160 * 1024;

// Geometry checks shared by the capability query and the launch. Fills g and the LDS bytes on success.
int halo_prepare(const HaloConfig& c, const gie_conv_geom* gg, HaloGeom* g, int* lds_bytes) {
  if (!gg) return GIE_HIP_EINVAL;
  if (gg->kernel_h != c.info.kernel_h || gg->kernel_w != c.info.kernel_w) return GIE_HIP_EUNSUPPORTED;
  g->B = gg->batch;
  g->Cp = gg->c_pad;
  g->H = gg->in_h;
  g->W = gg->in_w;
  g->O = gg->out_channels;
  g->SH = gg->stride_h;
  g->SW = gg->stride_w;
  g->PH = gg->pad_h;
  g->PW = gg->pad_w;
  g->OH = gg->out_h;
  g->OW = gg->out_w;
  g->relu = gg->relu ? 1 : 0;
  if (g->B <= 0 || gg->in_channels <= 0 || g->Cp < gg->in_channels || (g->Cp & 7) != 0 || g->H <= 0 || g->W <= 0 ||
      g->O <= 0 || g->SH <= 0 || g->SW <= 0 || g->PH < 0 || g->PW < 0 || g->OH <= 0 || g->OW <= 0)
    return GIE_HIP_EINVAL;
  const int KH = c.info.kernel_h, KW = c.info.kernel_w, TPX = c.info.tile_n;
  const long long hwo = static_cast<long long>(g->OH) * g->OW;
  const long long n = hwo * g->B;
  const long long xb = static_cast<long long>(g->H) * g->W * g->Cp * g->B * 2;
  const long long wb = static_cast<long long>(g->O) * KH * KW * g->Cp * 2;
  if (n > 0x7fffffffLL || xb >= 0x7fffffffLL || wb >= 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  g->HWo = int(hwo);
  g->N = int(n);
  g->x_bytes = int(xb);
  g->w_bytes = int(wb);
  g->WPAD = (g->OW - 1) * g->SW + KW;
  g->E = KH > g->SH ? KH - g->SH : 0;
  g->nslices = (g->Cp + kCS - 1) / kCS;
  // slots of the largest tile: rows it spans, taps per row, image boundaries it crosses
  const long long rows = std::min<long long>(static_cast<long long>(g->OH) * g->B, (TPX - 1) / g->OW + 2);
  const long long bounds = std::min<long long>(g->B - 1, (TPX - 1) / hwo + 1);
  const long long ns = (rows - 1) * g->SH + KH + g->E * bounds;
  if (ns > kMaxSlots) return GIE_HIP_EUNSUPPORTED;
  const long long pixels = ns * g->WPAD;
  if (pixels > kMaxStagedPixels || pixels * 4 > static_cast<long long>(c.ait) * c.info.threads)
    return GIE_HIP_EUNSUPPORTED;
  g->act_stage = int((pixels + 1) * kPXB);  // + one spare pixel written by idle lanes
  const long long stage = g->act_stage + static_cast<long long>(c.wst);
  const int wp = c.info.tile_n / 64;
  const long long red = static_cast<long long>(wp) * (c.info.kernel_h == 3 ? 3 : 1) * c.acc;
  const long long epi = std::max(red, static_cast<long long>(wp) * 2 * c.acc + c.info.tile_m * c.trow);
  const long long lds = kSlotTable + std::max(2 * stage, epi);
  if (lds > kLdsLimit) return GIE_HIP_EUNSUPPORTED;
  *lds_bytes = int(lds);
  return GIE_HIP_OK;
}

int set_lds_limit(HaloFn fn, int bytes) {
  if (bytes <= 64 * 1024) return GIE_HIP_OK;
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return int(hipErrorInvalidDevice);
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({reinterpret_cast<const void*>(fn), dev})) return GIE_HIP_OK;
  // the largest amount any geometry may use, so one attribute call covers them all
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
  if (e != hipSuccess) return int(e);
  done.insert({reinterpret_cast<const void*>(fn), dev});
  return GIE_HIP_OK;
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_halo_config_count(void) { return int(halo_configs().size()); }

extern "C" int gie_hip_halo_config_get(int index, gie_halo_config* out) {
  if (index < 0 || index >= int(halo_configs().size()) || !out) return GIE_HIP_EINVAL;
  *out = halo_configs()[size_t(index)].info;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_halo_check(int config, const gie_conv_geom* g, int* lds_bytes) {
  if (config < 0 || config >= int(halo_configs().size()) || !g) return GIE_HIP_EINVAL;
  HaloGeom hg;
  int lds = 0;
  const int rc = halo_prepare(halo_configs()[size_t(config)], g, &hg, &lds);
  if (rc == GIE_HIP_OK && lds_bytes) *lds_bytes = lds;
  return rc;
}

extern "C" int gie_hip_conv_halo(int config, int dtype, const gie_conv_geom* gg, const void* xn, const void* wk,
                                 const void* bias, void* y, float* partial, int split, void* stream) {
  if (config < 0 || config >= int(halo_configs().size()) || !gg || !xn || !wk) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if (split < 1 || split > 64) return GIE_HIP_EINVAL;
  if (split == 1 && !y) return GIE_HIP_EINVAL;
  if (split > 1 && (!partial || (reinterpret_cast<uintptr_t>(partial) & 15u) != 0)) return GIE_HIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(xn) & 15u) || (reinterpret_cast<uintptr_t>(wk) & 15u)) return GIE_HIP_EINVAL;
  const HaloConfig& c = halo_configs()[size_t(config)];
  HaloGeom g;
  int lds = 0;
  if (int rc = halo_prepare(c, gg, &g, &lds)) return rc;
  if (split > g.nslices) return GIE_HIP_EUNSUPPORTED;
  const long long n_ot = (g.O + c.info.tile_m - 1) / c.info.tile_m;
  const long long n_pt = (static_cast<long long>(g.N) + c.info.tile_n - 1) / c.info.tile_n;
  if (n_ot * n_pt > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  HaloFn fn = c.fn[dtype == GIE_HIP_BF16 ? 1 : 0];
  if (int rc = set_lds_limit(fn, lds)) return rc;
  hipLaunchKernelGGL(fn, dim3(unsigned(n_ot * n_pt), 1, unsigned(split)), dim3(c.info.threads), lds,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(xn),
                     static_cast<const uint16_t*>(wk), static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y),
                     partial, g, split);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
