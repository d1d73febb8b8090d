// Slab convolution: 3x3 filter, stride 1, padding 1, straight from NCHW x and OIHW w on gfx950 matrix cores
// (v_mfma_f32_16x16x32_{f16,bf16}, FP32 accumulation). One launch; no repack and no workspace (split 1).
//
// A workgroup owns 32 output channels x one slab of RB output rows of one image. In LDS the slab's input rows
// (one halo row above and below) form a flat array of positions, P per row (P >= in_w + 1): input (ih, iw) sits at
// position q = (ih - oh0 + 1) * P + iw; positions in_w .. P-1 of every row are padding (the right padding of the row
// and, seen from the next row, its left padding). Output pixel (oh, ow) has the flat index o = (oh - oh0) * P + ow,
// and tap (r, s) of it reads position o + r * P + s - 1. A 16 x 16 MFMA block is 16 consecutive flat outputs, so
// the pixel operand of tap row r is one 16-position read at o + r * P for all three tap columns, and the tap column
// enters through three accumulator sets:
//     acc_s[o] = sum_r W[r][s] . X[o + r*P],     y[o] = acc_0[o - 1] + acc_1[o] + acc_2[o + 1],
// the shifts being DPP lane moves applied once in the epilogue (flat outputs at columns >= in_w are dropped). The
// inner loop is LDS reads, 36 v_perm per slice and MFMAs.
//
// Waves: 4 = (filter half fh: 16 filters) x (row half wr: RW = 16 * NBW / P rows = NBW blocks), one per SIMD.
//
// Both operands travel by direct-to-LDS loads, NST stages, one 32-channel slice per stage:
//   * weights: each filter's OIHW run of the slice (CS x 9 contiguous halves) by 16-byte loads into a staging row
//     of CS*18 + 16 bytes (the extra 16 bytes spread the rows over the banks). A wave reads its lanes' 144-byte runs
//     (8 channels x 9 taps of one filter) with 9 ds_read_b128 and transposes them in registers (v_perm) into the 9
//     tap fragments (8 channels of one tap per lane) — there is no weight repack anywhere;
//   * activations: [channel][32-byte segments of 16 positions], segment slot = segment ^ swizzle(channel) so the
//     transposing fragment reads of 8 channels hit 8 distinct bank groups; out-of-image rows load as zeros. The
//     full and lean forms load 4-byte position pairs, padding columns included (as zeros); the pipelined form loads
//     16-byte chunks of 8 positions, whose tails run into the padding positions, and its epilogue never reads
//     those. The pixel fragments come out with ds_read_b64_tr_b16 (4 channels of 16 positions per 16-lane group,
//     each lane receiving the 4 channels of its position). Rows of odd width (or x not 4-byte aligned) take 2-byte
//     register loads and 2-byte LDS writes instead (full form; padding cleared once).
// Epilogue (slab_store): the DPP shift-add of the three accumulator sets, then bias + ReLU + one RNE rounding (the
// reference's apply_epilogue order, src/kernels/fused_epilogue.cuh:11-16) and stores straight from the registers:
// 4-byte pixel pairs (lane pairs exchange halves by DPP) or 2-byte values; the split form (loader waves) stages the
// pixel pairs of a whole-image unit in LDS instead and writes its 32 planes as one run of 16-byte device-scope stores
// (split_stage_rows, split_copy_out). split > 1: FP32 partials
// partial[z][NCHW] over the z-th range of channel slices [floor(S*z/split), floor(S*(z+1)/split)), the partition of
// src/kernels/tensor_core_mma.cu:112-115, reduced by splitk_reduce.hip.
// Grid: units (split range, image, slab, 32-filter block); XCD x (slot mod 8) takes a contiguous range of units, with
// the filter block fastest when that fetches fewer bytes per XCD (config 2: each XCD holds 4 images and every weight)
// or the image fastest (weight-heavy layers such as config 5: each XCD holds a few filter blocks and every image).
#include <algorithm>
#include <cmath>
#include <atomic>
#include <mutex>

#include "slab_common.h"

namespace gie_hip {
namespace {

constexpr int kSlTO = 32;  // output channels per workgroup

struct SlabGeom {
  int B, C, H, W, O, HW;
  int S;                       // channel slices
  int n_bands, n_ob, n_units;  // slabs per image, 32-filter blocks, workgroup units
  int per_xcd;                 // units per XCD
  int x_bytes, w_bytes;
  int relu, split;
  int y_vec;                   // outputs leave as 4-byte pixel pairs
  int y_stage;                 // split form: the unit's output run is staged in LDS and leaves as 16-byte stores
  long long total;             // |Y| elements (partial stride)
  float inv_hw, inv_w;         // 1 / HW, 1 / W for fdiv
  // unit = ((z * rad[2] + d2) * rad[1] + d1) * rad[0] + d0 with d1 = slab; order 0: d0 = filter block, d2 = image
  // (each XCD's range of units shares images), order 1: d0 = image, d2 = filter block (shares weights)
  int order;
  int rad[3];
  unsigned mg[3];  // n / rad[k] = (umulhi(n, mg[k]) + n) >> sh[k] for n < 2^30
  int sh[3];
};

struct SlabUnit {
  int b, z, ob, band;
};

// Every kernel argument the set-up and the epilogue read, requested before the first branch: the compiler otherwise
// issues the argument loads per basic block (the unit count for the early exit, then the geometry, then the
// pointers), three round trips to the argument segment of several hundred cycles each instead of one.
__device__ __forceinline__ void args_in_sgprs(const void* x, const void* w, const void* bias, const void* y,
                                              const void* partial, const SlabGeom& g) {
  asm volatile("" ::"s"(x), "s"(w), "s"(bias), "s"(y), "s"(partial));
  asm volatile("" ::"s"(g.n_units), "s"(g.per_xcd), "s"(g.order), "s"(g.rad[0]), "s"(g.rad[1]), "s"(g.rad[2]),
               "s"(g.mg[0]), "s"(g.mg[1]), "s"(g.mg[2]), "s"(g.sh[0]), "s"(g.sh[1]), "s"(g.sh[2]));
  asm volatile("" ::"s"(g.S), "s"(g.split), "s"(g.C), "s"(g.H), "s"(g.W), "s"(g.HW), "s"(g.O), "s"(g.x_bytes),
               "s"(g.w_bytes), "s"(g.relu), "s"(g.y_vec), "s"(g.y_stage), "s"(g.total));
}
__device__ __forceinline__ SlabUnit decode_unit(int unit, const SlabGeom& g) {
  const int q0 = magic_div(unit, g.mg[0], g.sh[0]), d0 = unit - q0 * g.rad[0];
  const int q1 = magic_div(q0, g.mg[1], g.sh[1]), d1 = q0 - q1 * g.rad[1];
  const int z = magic_div(q1, g.mg[2], g.sh[2]), d2 = q1 - z * g.rad[2];
  SlabUnit u;
  u.z = z;
  u.band = d1;
  u.ob = g.order == 0 ? d0 : d2;
  u.b = g.order == 0 ? d2 : d0;
  return u;
}

template <int P, int NBW, int NST>
struct SlabShape {
  static constexpr int G = P >= 16 ? 16 : P;            // spacing of the pixel-fragment reads (positions)
  static constexpr int RW = 16 * NBW / P;               // output rows per wave
  static constexpr int RB = 2 * RW;                     // output rows per slab
  static constexpr int NR = RB + 2;                     // LDS rows per channel (halo row above and below)
  static constexpr int NBR = (16 * (NBW - 1) + 2 * P) / G + 1;  // pixel-fragment reads per slice
  static constexpr int CS = 32;                         // channels per slice (one MFMA k-step)
  static constexpr int NW = 4, NT = 256;                // waves: (filter half) x (row half), one per SIMD
  // weights: per filter the slice's OIHW run (CS * 9 halves) in 16-byte chunks + one pad chunk
  static constexpr int WCH = CS * 18 / 16;
  static constexpr int CPF = WCH + 1;
  static constexpr int WPITCH = CPF * 16;
  static constexpr int WBLK = (kSlTO * CPF + 63) / 64;  // 1 KiB load blocks holding data per slice
  static constexpr int KBW = (WBLK + NW - 1) / NW;      // weight blocks per wave: every wave issues the same
  static constexpr int WST = KBW * NW * 1024;           // count, the blocks past WBLK load zeros
  // activations: per channel NS segments of 16 positions (32 bytes)
  static constexpr int NS = ((NR * P + 15) / 16 + 7) / 8 * 8;
  static constexpr int CHP = NS * 32;
  static constexpr int ACT = CS * CHP;
  static constexpr int R = CHP / 256;                   // 4-byte load instructions per channel
  static constexpr int KA = ACT / 256 / NW;             // 4-byte load instructions per wave per slice
  static constexpr int KR = (CS * NR * (P - 1) + NT - 1) / NT;  // 2-byte form: elements per thread per slice
  static constexpr int LDS = NST * (ACT + WST);         // [activation stages][weight stages]
  static constexpr int U = NST % 2 == 0 ? NST : 2 * NST;  // loop unroll: stage and register set are constants
  static_assert((16 * NBW) % P == 0, "a wave's rows are whole 16-position blocks");
  static_assert(KA == 8 * R, "each wave's load instructions cover 8 whole channels");
  static_assert(CHP % 256 == 0, "channel regions start on the same bank");
  static_assert((NST - 1) * ACT < 65536 && (NST - 1) * WST + 256 < 65536, "stage offsets fit the LDS offset field");
  static_assert(LDS <= kLdsLimit, "LDS budget");
};

// Activation load forms of the full and lean kernels: kDma4 = 4-byte direct-to-LDS loads of every padded position;
// kReg2 = 2-byte register loads (odd rows, or x only 2-byte aligned).
constexpr int kDma4 = 1, kReg2 = 2;

// Epilogue of one unit, shared by the slab kernels: tap-column shifts (DPP), then split 1: bias + ReLU + one rounding
// and pixel-pair (or 2-byte) stores straight from the accumulators; split > 1: FP32 partials. One loop per store
// form; positions outside the image and filters past O store to kOut (dropped), so no lane is masked by branches.
// PADS_LOADED: the padding columns of the LDS rows hold whatever the row loads brought in (16-byte loads run past
// the row end into them); the left neighbour of column 0 and the right neighbour of column W - 1 are padding, so those
// two shifted terms are selected out instead of read as zeros.
// Block j of a unit's output: the three tap-column accumulator sets shifted into place and added.
template <int P, int NBW, bool PADS_LOADED>
__device__ __forceinline__ f32x4 slab_column(const f32x4 (&acc)[3][NBW], int j, int lane, int wr, int W) {
  constexpr int RW = 16 * NBW / P;
  if constexpr (PADS_LOADED && P == 16) {
    // a 16-position block is one row: the cross-block terms reach only column 0 (its left neighbour is padding)
    // and column 15 (never stored), and the row shift already gives column 0 nothing; only the right neighbour of
    // column W - 1, position W, has to be zeroed before the shift
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const f32x4 a2 = (lane & 15) == W ? zero : acc[2][j];
    return acc[1][j] + dpp4<kShr1>(acc[0][j]) + dpp4<kShl1>(a2);
  } else if constexpr (PADS_LOADED) {
    f32x4 t0 = dpp4<kShr1>(acc[0][j]), t2 = dpp4<kShl1>(acc[2][j]);
    if (j > 0) t0 += dpp4<kShl15>(acc[0][j - 1]);
    if (j + 1 < NBW) t2 += dpp4<kShr15>(acc[2][j + 1]);
    const int c = (wr * RW * P + 16 * j + (lane & 15)) % P;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    return acc[1][j] + (c != 0 ? t0 : zero) + (c != W - 1 ? t2 : zero);
  } else {
    f32x4 out = acc[1][j] + dpp4<kShr1>(acc[0][j]) + dpp4<kShl1>(acc[2][j]);
    if (j > 0) out += dpp4<kShl15>(acc[0][j - 1]);
    if (j + 1 < NBW) out += dpp4<kShr15>(acc[2][j + 1]);
    return out;
  }
}

// Bias + ReLU + one rounding of a lane's four filters at one position, then the pixel-pair exchange between lane
// pairs: the even lane (column c) ends with filters 0 and 1 at columns (c, c + 1), the odd lane with filters 2 and 3
// at columns (c - 1, c), each as one 4-byte word (low half = the left column).
template <typename E>
__device__ __forceinline__ void round_pairs(const f32x4& out, const float (&bv)[4], int relu, uint32_t oddm,
                                            uint32_t* wa, uint32_t* wb) {
  uint32_t h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = out[i] + bv[i];
    h[i] = E::from_f32(relu ? fmaxf(v, 0.0f) : v);
  }
  const uint32_t lo01 = h[0] | (h[1] << 16), lo23 = h[2] | (h[3] << 16);
  const uint32_t send = (lo01 & oddm) | (lo23 & ~oddm);
  const uint32_t recv = uint32_t(__builtin_amdgcn_mov_dpp(int(send), 0xB1, 0xf, 0xf, false));  // swap lane pairs
  // even: (h0, recv.lo) and (h1, recv.hi); odd: (recv.lo, h2) and (recv.hi, h3)
  const uint32_t wa_e = (h[0] & 0xffffu) | (recv << 16), wb_e = (h[1] & 0xffffu) | (recv & 0xffff0000u);
  const uint32_t wa_o = (recv & 0xffffu) | (h[2] << 16), wb_o = (recv >> 16) | (h[3] << 16);
  *wa = (wa_o & oddm) | (wa_e & ~oddm);
  *wb = (wb_o & oddm) | (wb_e & ~oddm);
}

// The pixel-pair words of one 16-position output row (one row per block, P == 16): bias + ReLU + one rounding of the
// lane's four filters with two packed conversions, then two selects, one lane-pair swap and two byte permutes. Word a
// holds filter fp's values at columns (c, c + 1), word b filter fp + 1's (even lane: fp = 0 and c its column; odd
// lane: fp = 2 and c its column - 1).
struct PairSel {
  uint32_t odd, sel_a, sel_b;
  __device__ __forceinline__ explicit PairSel(int lane)
      : odd(uint32_t(lane & 1)), sel_a(odd ? 0x01000504u : 0x05040100u), sel_b(odd ? 0x03020706u : 0x07060302u) {}
};
template <typename E, bool RELU>
__device__ __forceinline__ void row_pairs(const f32x4& out, const float (&bv)[4], const PairSel& ps, uint32_t* wa,
                                          uint32_t* wb) {
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float t = out[i] + bv[i];
    v[i] = RELU ? fmaxf(t, 0.0f) : t;
  }
  const uint32_t h01 = E::pack2(v[0], v[1]), h23 = E::pack2(v[2], v[3]);
  const uint32_t send = ps.odd ? h01 : h23, mine = ps.odd ? h23 : h01;
  const uint32_t recv = uint32_t(__builtin_amdgcn_mov_dpp(int(send), 0xB1, 0xf, 0xf, false));  // swap lane pairs
  *wa = __builtin_amdgcn_perm(recv, mine, ps.sel_a);
  *wb = __builtin_amdgcn_perm(recv, mine, ps.sel_b);
}

template <typename E, int P, int NBW, bool PADS_LOADED = false>
__device__ __forceinline__ void slab_store(const f32x4 (&acc)[3][NBW], const uint32_t (&bbits)[4], int lane, int wr,
                                           int oh0, int nrows, int b, int z, int o0, int f0,
                                           uint16_t* __restrict__ y, float* __restrict__ partial, const SlabGeom& g) {
  constexpr int RW = 16 * NBW / P;
  (void)o0;
  auto column = [&](int j) __attribute__((always_inline)) {
    return slab_column<P, NBW, PADS_LOADED>(acc, j, lane, wr, g.W);
  };
  const int nf = g.O - f0;                         // filters of the lane's four that exist (>= 4: all)
  const int fbase = (b * g.O + f0) * g.HW;         // element index of (b, f0, 0)
  if (g.split > 1) {
    const v4i pr = make_vsharp(partial + static_cast<long long>(z) * g.total, int(g.total * 4));
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const f32x4 out = column(j);
      const int p = wr * RW * P + 16 * j + (lane & 15), row = p / P, col = p % P;
      const bool valid = col < g.W && row < nrows;
      const int e = fbase + (oh0 + row) * g.W + col;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store4(pr, valid && i < nf ? (e + i * g.HW) * 4 : kOut, __float_as_uint(out[i]));
    }
    return;
  }
  float bv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bv[i] = E::to_f32(uint16_t(bbits[i]));
  const v4i yr = make_vsharp(y, int(g.total * 2));
  auto finish = [&](const f32x4& out, uint32_t (&h)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = out[i] + bv[i];
      h[i] = E::from_f32(g.relu ? fmaxf(v, 0.0f) : v);
    }
  };
  if constexpr (PADS_LOADED && P == 16) {
    if (g.y_vec) {
      // one 16-position block per output row: block j is row wr * RW + j, the lane's column is lane % 16. Pixel
      // pairs by row_pairs; the store offsets are a per-lane base (kOut for a column or filter outside the output)
      // plus a wave-uniform row displacement, and rows past the slab's end are skipped by a uniform branch.
      const PairSel ps(lane);
      const int fp = int(ps.odd) * 2, col = (lane & 15) - int(ps.odd);
      const int row0 = oh0 + wr * RW;
      const bool lane_ok = col < g.W && fp < nf;
      const int base = lane_ok ? (fbase + fp * g.HW + row0 * g.W + col) * 2 : kOut;
      const v4i yr = make_vsharp(y, int(g.total * 2));
      auto rows = [&](auto relu_c) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NBW; ++j) {
          if (wr * RW + j >= nrows) break;
          uint32_t wa, wb;
          row_pairs<E, decltype(relu_c)::value>(column(j), bv, ps, &wa, &wb);
          store4s(yr, base, 2 * j * g.W, wa);
          store4s(yr, base, 2 * (j * g.W + g.HW), wb);
        }
      };
      if (g.relu) rows(std::true_type{});
      else rows(std::false_type{});
      return;
    }
  }
  if (g.y_vec) {
    // pixel pairs: even lane (column c) stores filters 0, 1 at (c, c+1), odd lane filters 2, 3 at (c-1, c)
    const uint32_t oddm = 0u - uint32_t(lane & 1);  // all ones on odd lanes
    const int fp = int(oddm & 2u);                   // first filter of the lane's pair stores
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int p = wr * RW * P + 16 * j + (lane & 15), row = p / P, col = p % P;
      uint32_t wa, wb;
      round_pairs<E>(column(j), bv, g.relu, oddm, &wa, &wb);
      // the odd lane's pair starts at column c - 1, which is valid when its own column is
      const bool pv = col - int(oddm & 1u) < g.W && row < nrows;
      const int e = fbase + fp * g.HW + (oh0 + row) * g.W + col - int(oddm & 1u);
      store4(yr, pv && fp < nf ? e * 2 : kOut, wa);
      store4(yr, pv && fp + 1 < nf ? (e + g.HW) * 2 : kOut, wb);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    uint32_t h[4];
    finish(column(j), h);
    const int p = wr * RW * P + 16 * j + (lane & 15), row = p / P, col = p % P;
    const bool valid = col < g.W && row < nrows;
    const int e = fbase + (oh0 + row) * g.W + col;
#pragma unroll
    for (int i = 0; i < 4; ++i) store2(yr, valid && i < nf ? (e + i * g.HW) * 2 : kOut, h[i]);
  }
}

template <typename E, int P, int NBW, int NST, int MODE>
__global__ __launch_bounds__(256, 1) void slab_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                     const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                     float* __restrict__ partial, SlabGeom g) {
  using Sh = SlabShape<P, NBW, NST>;
  constexpr int CS = Sh::CS, NW = Sh::NW, NT = Sh::NT, RW = Sh::RW, RB = Sh::RB, NR = Sh::NR, G = Sh::G;
  constexpr int NBR = Sh::NBR, CPF = Sh::CPF, WCH = Sh::WCH, WPITCH = Sh::WPITCH, KBW = Sh::KBW;
  constexpr int WST = Sh::WST, CHP = Sh::CHP, ACT = Sh::ACT, KA = Sh::KA, R = Sh::R, U = Sh::U;
  constexpr int KR = Sh::KR;
  constexpr bool REG = MODE == kReg2;                   // activations through registers
  constexpr int NL = REG ? KR : 0;                      // register loads per thread per slice
  constexpr int NI = KBW + (MODE == kDma4 ? KA : NL);   // loads per wave per slice
  constexpr int WOFF = NST * ACT;                       // LDS: [activation stages][weight stages]
  static_assert(NST * NI < 64, "loads in flight fit the vmcnt counter");
  static_assert(!REG || NST >= 3, "register forms write a slice one step after loading it");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fh = wave & 1, wr = wave >> 1;

  // ---- unit: XCD (slot mod 8) takes units [xcd * per_xcd, ...), filter block fastest ----
  const int slot = int(blockIdx.x);
  const int unit = (slot >> 3) + (slot & 7) * g.per_xcd;
  if (unit >= g.n_units) return;  // workgroup-uniform
  const SlabUnit un = decode_unit(unit, g);
  const int b = un.b, z = un.z;
  const int o0 = un.ob * kSlTO, oh0 = un.band * RB;
  const int s_beg = (g.S * z) / g.split, ns = (g.S * (z + 1)) / g.split - s_beg;
  const int nrows = min(RB, g.H - oh0);

  const v4i xr = make_vsharp(x, g.x_bytes);
  const v4i wrs = make_vsharp(w, g.w_bytes);
  const unsigned lds0 = lds_addr(lds);

  // bias bits of the lane's four filters, fetched now, used in the epilogue
  const int f0 = o0 + fh * 16 + 4 * (lane >> 4);  // the lane's first filter
  uint32_t bbits[4] = {0u, 0u, 0u, 0u};
  if (g.split == 1 && bias != nullptr) {
#pragma unroll
    for (int i = 0; i < 4; ++i) bbits[i] = bias[min(f0 + i, g.O - 1)];
  }

  // ---- weight loads: block wave + NW * kb; lane slot u = (filter u / CPF, chunk u % CPF); per slice += CS * 18
  int w_voff[KBW];
#pragma unroll
  for (int kb = 0; kb < KBW; ++kb) {
    const int u = (wave + NW * kb) * 64 + lane, f = u / CPF, k = u - f * CPF;
    w_voff[kb] = (f < kSlTO && k < WCH && o0 + f < g.O) ? (o0 + f) * g.C * 18 + 16 * k : kOut;
  }
  int w_soff = s_beg * CS * 18;  // scalar offset of the next slice to load
  int w_rem = g.C - s_beg * CS;  // its channels still inside C
  int a_c0 = s_beg * CS;         // first channel of the next slice to load (activations)

  // ---- activations, direct form: instruction i of this wave covers 256 bytes of channel 8 * wave + i / R;
  // the per-lane offsets depend on (i % R, the channel's swizzle) only ----
  constexpr int NV = MODE == kDma4 ? 4 * R : 1;
  int a_voff[NV];
  const int a_soff0 = (b * g.C + 8 * wave) * g.HW * 2;  // + (slice channel + i / R) * HW * 2
  if constexpr (MODE == kDma4) {
    const int swz_hi = (wave & 1) << 2;  // channel bit 3 = wave & 1 for all of this wave's channels
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int seg = (v % R) * 8 + (lane >> 3);
      const int pos = ((seg ^ ((v / R) | swz_hi)) << 4) + 2 * (lane & 7);
      const int row = pos / P, col = pos % P, ih = oh0 - 1 + row;
      a_voff[v] = (row < NR && ih >= 0 && ih < g.H && col < g.W) ? (ih * g.W + col) * 2 : kOut;
    }
  }
  // ---- activations, register form: element e = k * NT + tid of (channel, input row of the slab, column), the
  // thread's elements fixed across slices ----
  int r_voff[NL > 0 ? NL : 1];
  unsigned r_dst[NL > 0 ? NL : 1];
  int r_lim[NL > 0 ? NL : 1];  // the element's channel, compared against the slice's channels
  uint32_t r_v2[NL > 0 ? NL : 1];
  if constexpr (REG) {
    const int ih_lo = max(oh0 - 1, 0), ih_hi = min(oh0 + RB + 1, g.H);
    const int per_ch = (ih_hi - ih_lo) * g.W;
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const int e = k * NT + tid, ch = e / per_ch, rem = e - ch * per_ch, rr = rem / g.W, col = rem - rr * g.W;
      const int pos = (ih_lo - oh0 + 1 + rr) * P + col;
      r_voff[k] = ch < CS ? (ch * g.HW + (ih_lo + rr) * g.W + col) * 2 : kOut;
      r_lim[k] = ch < CS ? ch : (1 << 24);
      r_dst[k] = lds0 + unsigned(ch * CHP + (((pos >> 4) ^ seg_swz(ch)) << 5) + (pos & 15) * 2);
    }
  }

  // the next slice in order: activations (register form: into registers v2, written one step later)...
  auto issue_act = [&](int st, uint32_t (&v2)[NL > 0 ? NL : 1]) __attribute__((always_inline)) {
    if constexpr (MODE == kDma4) {
      const unsigned ab = lds0 + unsigned(st * ACT + wave * KA * 256);
#pragma unroll
      for (int i = 0; i < KA; ++i) {
        const int soff = a_soff0 + (a_c0 + i / R) * g.HW * 2;
        dma4s(xr, ab + unsigned(i * 256), a_c0 + 8 * wave + i / R < g.C ? a_voff[(i % R) + R * ((i / R) & 3)] : kOut,
              soff);
      }
    } else {
      const int soff = (b * g.C + a_c0) * g.HW * 2;
#pragma unroll
      for (int k = 0; k < NL; ++k) v2[k] = load2s(xr, a_c0 + r_lim[k] < g.C ? r_voff[k] : kOut, soff);
    }
    a_c0 += CS;
  };
  // ...then its weights
  auto issue_w = [&](int st) __attribute__((always_inline)) {
    const unsigned wb = lds0 + unsigned(WOFF + st * WST);
    if (w_rem >= CS) {
#pragma unroll
      for (int kb = 0; kb < KBW; ++kb) dma16s(wrs, wb + unsigned((wave + NW * kb) * 1024), w_voff[kb], w_soff);
    } else {  // the slice runs past C: chunks holding channels >= C load zeros
#pragma unroll
      for (int kb = 0; kb < KBW; ++kb) {
        const int u = (wave + NW * kb) * 64 + lane, k = u - (u / CPF) * CPF;
        dma16s(wrs, wb + unsigned((wave + NW * kb) * 1024), 8 * k < 9 * w_rem ? w_voff[kb] : kOut, w_soff);
      }
    }
    w_soff += CS * 18;
    w_rem -= CS;
  };
  // register form: activations loaded into registers by an earlier issue, for the slice with channel base c0, written
  // into stage st (the caller has waited for them); elements of channels past the slice are not written
  auto write_regs = [&](int st, const uint32_t (&v2)[NL > 0 ? NL : 1]) __attribute__((always_inline)) {
    if constexpr (REG) {
#pragma unroll
      for (int k = 0; k < NL; ++k)
        if (r_lim[k] < CS) *reinterpret_cast<lds_h*>(size_t(r_dst[k] + unsigned(st * ACT))) = uint16_t(v2[k]);
    }
  };
  auto touch_regs = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NL; ++k) touch_v(r_v2[k]);
  };

  // ---- fragment addresses (stage 0; the stage offset is the instruction's immediate offset) ----
  // A: lane (filter fh*16 + lane%16, channels 8*(lane/16) .. +7): 144 contiguous bytes of the staging row
  const unsigned a_rd = lds0 + unsigned(WOFF + (fh * 16 + (lane & 15)) * WPITCH + 8 * (lane >> 4) * 18);
  // B: block u (16 positions from wr*RW*P + u*G), channel quads h = 0, 1 of the lane's k-group; each lane reads the
  // 4 positions 4*(lane%4) .. +3 of channel row (lane%16)/4 of the quad
  unsigned b_rd[NBR][2];
#pragma unroll
  for (int u = 0; u < NBR; ++u) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ch = 8 * (lane >> 4) + 4 * h + ((lane & 15) >> 2);
      const int pos = wr * RW * P + u * G + 4 * (lane & 3);
      b_rd[u][h] = lds0 + unsigned(ch * CHP + (((pos >> 4) ^ seg_swz(ch)) << 5) + (pos & 15) * 2);
    }
  }

  f32x4 acc[3][NBW];
#pragma unroll
  for (int s = 0; s < 3; ++s) {
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[s][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // two fragment sets: slice i multiplies from set i & 1 while slice i + 1 is read into the other
  u32x4 fw[2][9], fb[2][NBR];
  uint32_t d[36];
  auto read_b = [&](int st, int set, int u0, int u1) __attribute__((always_inline)) {  // blocks u0 .. u1-1
#pragma unroll
    for (int u = u0; u < u1; ++u) {
      const u32x2 lo = rd_tr(b_rd[u][0] + unsigned(st * ACT)), hi = rd_tr(b_rd[u][1] + unsigned(st * ACT));
      fb[set][u] = u32x4{lo.x, lo.y, hi.x, hi.y};
    }
  };
  auto read_a = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      const u32x4 v = rd16(a_rd + unsigned(st * WST + 16 * t));
      d[4 * t] = v.x, d[4 * t + 1] = v.y, d[4 * t + 2] = v.z, d[4 * t + 3] = v.w;
    }
  };
  auto transpose_a = [&](int set, int t0, int t1) __attribute__((always_inline)) {  // taps t0 .. t1-1
#pragma unroll
    for (int t = t0; t < t1; ++t)
      fw[set][t] = u32x4{pick2(d, t, 9 + t), pick2(d, 18 + t, 27 + t), pick2(d, 36 + t, 45 + t), pick2(d, 54 + t, 63 + t)};
  };
  auto mfma_tap = [&](int set, int t) __attribute__((always_inline)) {  // the NBW MFMAs of tap t = (r, s)
    const int r = t / 3, sc = t % 3;
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[sc][j] = E::mfma(fw[set][t], fb[set][(16 * j + r * P) / G], acc[sc][j]);
  };

  // ---- prologue: slices 0 .. NST-1 loading (one per stage); register forms write slices 0 .. NST-2 now, from
  // loads all issued before the first wait ----
  if constexpr (REG) {
    // padding positions are never written, so every activation stage starts zeroed
    for (int i = tid * 16; i < NST * ACT; i += NT * 16) *reinterpret_cast<u32x4*>(lds + i) = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
  }
  {
    uint32_t p2[NST - 1][NL > 0 ? NL : 1];
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      if (st < ns) {
        if (st + 1 < NST) issue_act(st, p2[st]);
        else issue_act(st, r_v2);  // written in step 0
        issue_w(st);
      }
    }
    if constexpr (REG) {
      // slice st's activations are followed by its weights and everything of the slices after it
#pragma unroll
      for (int st = 0; st + 1 < NST; ++st) {
        if (st < ns) {
          // issued after slice st's activations: its weights and the slices st+1 .. min(NST, ns)-1
          wait_vm_upto<KBW + (NST - 1) * NI>(KBW + (min(NST, ns) - 1 - st) * NI);
#pragma unroll
          for (int k = 0; k < NL; ++k) touch_v(p2[st][k]);
          write_regs(st, p2[st]);
        }
      }
    }
  }
  // slice 0 has landed (register forms: written); slices 1 .. NST-1 may still be in flight
  if (NST <= ns) wait_vmcnt<(NST - 1) * NI>();
  else wait_vmcnt<0>();
  stage_barrier();
  if (ns > 0) {
    read_b(0, 0, 0, NBR);
    read_a(0);
    transpose_a(0, 0, 9);
  }

  // ---- step i: slice i multiplies (9 tap groups of NBW MFMAs) while, between the groups, slice i + NST - 1's
  // activations (register forms, loaded in step i - 1) are written, slice i + NST starts loading into slice i's
  // stage (its fragments were read in step i - 1, which every wave finished before this step's barrier), and
  // slice i + 1's fragments are read and transposed ----
  auto step = [&](int i, auto u_c) __attribute__((always_inline)) {
    constexpr int uu = decltype(u_c)::value;
    constexpr int cur = uu & 1, nxt = cur ^ 1;
    constexpr int st_next = (uu + 1) % NST;         // stage holding slice i + 1
    constexpr int st_load = uu % NST;               // stage of slice i, reloaded with slice i + NST
    constexpr int st_write = (uu + NST - 1) % NST;  // stage of slice i + NST - 1 (register forms)
    const bool more = i + 1 < ns;
    const bool wr_now = REG && i + NST - 1 < ns && more;
    const bool ld_now = i + NST < ns;
    if (more) {
      // slice i + 1 has landed for every wave (this wave's loads counted: slices i+2 .. i+NST-1 may be in flight;
      // the barrier covers the other waves)
      if constexpr (NST > 2) {
        if (i + NST - 1 < ns) wait_vmcnt<(NST - 2) * NI>();
        else wait_vmcnt<0>();
      } else {
        wait_vmcnt<0>();
      }
      stage_barrier();
    }
    // register forms: slice i + NST - 1's activations (issued last step, before its weights) have landed
    if (wr_now) {
      wait_vm<KBW>();
      touch_regs();
    }
    __builtin_amdgcn_sched_barrier(0);
    // The LDS counter waits in issue order (and counts at most 15), so the weight fragments of slice i + 1 are
    // requested first and transposed before any other LDS access is issued; the activation writes and the pixel
    // fragments follow (the latter are consumed only in the next step).
    mfma_tap(cur, 0);
    if (more) read_a(st_next);
    __builtin_amdgcn_sched_barrier(0);
    mfma_tap(cur, 1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_tap(cur, 2);
    if (more) transpose_a(nxt, 0, 3);
    __builtin_amdgcn_sched_barrier(0);
    mfma_tap(cur, 3);
    if (more) transpose_a(nxt, 3, 6);
    __builtin_amdgcn_sched_barrier(0);
    mfma_tap(cur, 4);
    if (more) transpose_a(nxt, 6, 9);
    __builtin_amdgcn_sched_barrier(0);
    mfma_tap(cur, 5);
    if (wr_now) write_regs(st_write, r_v2);
    __builtin_amdgcn_sched_barrier(0);
    mfma_tap(cur, 6);
    if (ld_now) {
      issue_act(st_load, r_v2);
      issue_w(st_load);
    }
    __builtin_amdgcn_sched_barrier(0);
    mfma_tap(cur, 7);
    if (more) read_b(st_next, nxt, 0, (NBR + 1) / 2);
    __builtin_amdgcn_sched_barrier(0);
    mfma_tap(cur, 8);
    if (more) read_b(st_next, nxt, (NBR + 1) / 2, NBR);
    __builtin_amdgcn_sched_barrier(0);
  };
  for (int i = 0; i < ns; i += U) {
    step(i, std::integral_constant<int, 0>{});
    if (i + 1 < ns) step(i + 1, std::integral_constant<int, 1 % U>{});
    if constexpr (U > 2) {
      if (i + 2 < ns) step(i + 2, std::integral_constant<int, 2 % U>{});
      if (i + 3 < ns) step(i + 3, std::integral_constant<int, 3 % U>{});
    }
    if constexpr (U > 4) {
      if (i + 4 < ns) step(i + 4, std::integral_constant<int, 4 % U>{});
      if (i + 5 < ns) step(i + 5, std::integral_constant<int, 5 % U>{});
    }
  }

  // ---- epilogue: tap-column shifts, bias + ReLU + one rounding, stores straight from the registers ----
  slab_store<E, P, NBW>(acc, bbits, lane, wr, oh0, nrows, b, z, o0, f0, y, partial, g);
}

// ---- lean form: two workgroups per CU ----
// The same units, LDS layout and direct-to-LDS loads as slab_kernel with two load stages (kDma4 form only), held in at
// most 256 VGPR+AGPR per lane so that two workgroups share each CU and cover each other's waits and barriers:
//   * one set of weight fragments, rebuilt at the start of each slice from the staged OIHW rows;
//   * pixel fragments read one tap row at a time: row r reads only the blocks no earlier row needed;
//   * slice i + 1 loads into the other stage right after the barrier that starts slice i (every wave has finished
//     slice i - 1 there by then), so each slice's loads overlap one slice of MFMAs.
template <int P, int NBW>
struct LeanRows {
  static constexpr int G = P >= 16 ? 16 : P;
  static constexpr int first_row(int u) {  // first tap row whose MFMAs read pixel block u
    for (int r = 0; r < 3; ++r)
      for (int j = 0; j < NBW; ++j)
        if ((16 * j + r * P) / G == u) return r;
    return 3;
  }
};

template <typename E, int P, int NBW, int NST>
__global__ __launch_bounds__(256, 2) void slab_lean_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                          float* __restrict__ partial, SlabGeom g) {
  using Sh = SlabShape<P, NBW, NST>;
  using Rows = LeanRows<P, NBW>;
  constexpr int CS = Sh::CS, NW = Sh::NW, RW = Sh::RW, RB = Sh::RB, NR = Sh::NR, G = Sh::G, NBR = Sh::NBR;
  constexpr int CPF = Sh::CPF, WCH = Sh::WCH, WPITCH = Sh::WPITCH, KBW = Sh::KBW, WST = Sh::WST, CHP = Sh::CHP;
  constexpr int ACT = Sh::ACT, KA = Sh::KA, R = Sh::R;
  constexpr int WOFF = NST * ACT;  // LDS: [NST activation stages][NST weight stages]
  constexpr int NI = KBW + KA;     // loads per wave per slice
  static_assert(NST > 2 || Sh::LDS <= 80 * 1024, "two stages: two workgroups per CU");
  static_assert((NST - 1) * NI < 64, "loads in flight fit the vmcnt counter");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fh = wave & 1, wr = wave >> 1;

  // ---- unit (all wave-uniform): divisions by host-computed magic numbers ----
  const int slot = int(blockIdx.x);
  const int unit = (slot >> 3) + (slot & 7) * g.per_xcd;
  if (unit >= g.n_units) return;
  const SlabUnit un = decode_unit(unit, g);
  const int b = un.b, z = un.z;
  const int o0 = un.ob * kSlTO, oh0 = un.band * RB;
  int s_beg = 0, ns = g.S;
  if (g.split > 1) {
    s_beg = (g.S * z) / g.split;
    ns = (g.S * (z + 1)) / g.split - s_beg;
  }
  const int nrows = min(RB, g.H - oh0);

  const v4i xr = make_vsharp(x, g.x_bytes);
  const v4i wrs = make_vsharp(w, g.w_bytes);
  const unsigned lds0 = lds_addr(lds);

  // bias of the lane's four filters by counted loads: issued first, so the first slice's wait covers them
  const int f0 = o0 + fh * 16 + 4 * (lane >> 4);
  uint32_t bbits[4];
  {
    const v4i br = make_vsharp(bias, g.split == 1 && bias != nullptr ? 2 * g.O : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) bbits[i] = load2s(br, 2 * min(f0 + i, g.O - 1), 0);
  }

  // ---- direct-load offsets: per lane fixed across slices; per slice only the scalar offsets move ----
  int w_voff[KBW];
#pragma unroll
  for (int kb = 0; kb < KBW; ++kb) {
    const int u = (wave + NW * kb) * 64 + lane, f = u / CPF, k = u - f * CPF;
    w_voff[kb] = (f < kSlTO && k < WCH && o0 + f < g.O) ? (o0 + f) * g.C * 18 + 16 * k : kOut;
  }
  constexpr int NV = 4 * R;
  int a_voff[NV];
  {
    const int swz_hi = (wave & 1) << 2;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int seg = (v % R) * 8 + (lane >> 3);
      const int pos = ((seg ^ ((v / R) | swz_hi)) << 4) + 2 * (lane & 7);
      const int row = pos / P, col = pos % P, ih = oh0 - 1 + row;
      a_voff[v] = (row < NR && ih >= 0 && ih < g.H && col < g.W) ? (ih * g.W + col) * 2 : kOut;
    }
  }
  const int hw2 = g.HW * 2;
  int c_next = s_beg * CS;  // first channel of the next slice to load (wave-uniform)
  // the next slice into stage st: this wave's 8 channels' padded planes (KA 4-byte loads) and its share of the
  // 32 filters' OIHW runs (KBW 16-byte loads); channels past C load zeros
  auto issue = [&](int st) __attribute__((always_inline)) {
    const unsigned ab = lds0 + unsigned(st * ACT + wave * KA * 256);
    const unsigned wb = lds0 + unsigned(WOFF + st * WST);
    const int a_soff = (b * g.C + c_next + 8 * wave) * hw2;
    const int w_soff = c_next * 18;
    if (c_next + CS <= g.C) {
#pragma unroll
      for (int i = 0; i < KA; ++i)
        dma4s(xr, ab + unsigned(i * 256), a_voff[(i % R) + R * ((i / R) & 3)], a_soff + (i / R) * hw2);
#pragma unroll
      for (int kb = 0; kb < KBW; ++kb) dma16s(wrs, wb + unsigned((wave + NW * kb) * 1024), w_voff[kb], w_soff);
    } else {
      const int w_rem = g.C - c_next;
#pragma unroll
      for (int i = 0; i < KA; ++i)
        dma4s(xr, ab + unsigned(i * 256), c_next + 8 * wave + i / R < g.C ? a_voff[(i % R) + R * ((i / R) & 3)] : kOut,
              a_soff + (i / R) * hw2);
#pragma unroll
      for (int kb = 0; kb < KBW; ++kb) {
        const int u = (wave + NW * kb) * 64 + lane, k = u - (u / CPF) * CPF;
        dma16s(wrs, wb + unsigned((wave + NW * kb) * 1024), 8 * k < 9 * w_rem ? w_voff[kb] : kOut, w_soff);
      }
    }
    c_next += CS;
  };
#pragma unroll
  for (int st = 0; st + 1 < NST; ++st)
    if (st < ns) issue(st);

  const unsigned a_rd = lds0 + unsigned(WOFF + (fh * 16 + (lane & 15)) * WPITCH + 8 * (lane >> 4) * 18);
  unsigned b_rd[NBR][2];
#pragma unroll
  for (int u = 0; u < NBR; ++u) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ch = 8 * (lane >> 4) + 4 * h + ((lane & 15) >> 2);
      const int pos = wr * RW * P + u * G + 4 * (lane & 3);
      b_rd[u][h] = lds0 + unsigned(ch * CHP + (((pos >> 4) ^ seg_swz(ch)) << 5) + (pos & 15) * 2);
    }
  }

  f32x4 acc[3][NBW];
#pragma unroll
  for (int s2 = 0; s2 < 3; ++s2) {
#pragma unroll
    for (int j2 = 0; j2 < NBW; ++j2) acc[s2][j2] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  u32x4 fw[9], fb[NBR];
  uint32_t d[36];

  // slice i from stage st = i % NST: all of its LDS reads are requested right after the barrier; slice i + NST - 1's
  // loads go out (into the stage slice i - 1 used) once the first tap row's MFMAs are issued
  auto slice = [&](int i, auto st_c) __attribute__((always_inline)) {
    constexpr int st = decltype(st_c)::value;
    // this wave's loads of slice i have landed (slices i + 1 .. i + NST - 2 may still be in flight)
    if constexpr (NST == 2) {
      wait_vmcnt<0>();
    } else {
      if (i + NST - 2 < ns) wait_vmcnt<(NST - 2) * NI>();
      else wait_vm_upto<(NST - 2) * NI>((ns - 1 - i) * NI);
    }
    stage_barrier();  // every wave's loads of slice i have landed and every wave has finished slice i - 1
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      const u32x4 v = rd16(a_rd + unsigned(st * WST + 16 * t));
      d[4 * t] = v.x, d[4 * t + 1] = v.y, d[4 * t + 2] = v.z, d[4 * t + 3] = v.w;
    }
#pragma unroll
    for (int r = 0; r < 3; ++r) {
#pragma unroll
      for (int u = 0; u < NBR; ++u) {
        if (Rows::first_row(u) == r) {
          const u32x2 lo = rd_tr(b_rd[u][0] + unsigned(st * ACT)), hi = rd_tr(b_rd[u][1] + unsigned(st * ACT));
          fb[u] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
      }
      if (r == 0) {
#pragma unroll
        for (int t = 0; t < 9; ++t)
          fw[t] = u32x4{pick2(d, t, 9 + t), pick2(d, 18 + t, 27 + t), pick2(d, 36 + t, 45 + t), pick2(d, 54 + t, 63 + t)};
      }
#pragma unroll
      for (int sc = 0; sc < 3; ++sc) {
        const int t = 3 * r + sc;
#pragma unroll
        for (int j = 0; j < NBW; ++j) acc[sc][j] = E::mfma(fw[t], fb[(16 * j + r * P) / G], acc[sc][j]);
      }
      if (r == 0) {
        __builtin_amdgcn_sched_barrier(0);
        if (i + NST - 1 < ns) issue((st + NST - 1) % NST);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  for (int i = 0; i < ns; i += NST) {
    slice(i, std::integral_constant<int, 0>{});
    if (i + 1 < ns) slice(i + 1, std::integral_constant<int, 1 % NST>{});
    if constexpr (NST > 2) {
      if (i + 2 < ns) slice(i + 2, std::integral_constant<int, 2 % NST>{});
    }
    if constexpr (NST > 3) {
      if (i + 3 < ns) slice(i + 3, std::integral_constant<int, 3 % NST>{});
    }
  }
  wait_vmcnt<0>();  // the bias loads (already covered by the first slice's wait; stated for the epilogue)
#pragma unroll
  for (int i = 0; i < 4; ++i) touch_v(bbits[i]);
  slab_store<E, P, NBW>(acc, bbits, lane, wr, oh0, nrows, b, z, o0, f0, y, partial, g);
}

// ---- pipelined form: one workgroup per CU, every slot of the MFMA stream carrying the side work ----
// With one wave per SIMD a wave issues one instruction per 4-cycle slot, and a 16 x 16 x 32 MFMA occupies the
// matrix core for 4 slots: the 3 slots behind each MFMA are the only room for everything else. Left to itself the
// compiler emits each tap's MFMAs back to back and the side work (fragment transposes, the next slice's loads) as one
// clump after them, during which the matrix core idles. This form fixes the order: step j multiplies slice j from
// registers while slice j + 1 is read from LDS and transposed into the other fragment set and slice j + NST loads
// into the stage slice j occupied, one MFMA per slot followed by at most a few of those instructions. The step's
// only wait is at its start (slice j + 1 landed for this wave, then the barrier for all waves), so each slice's loads
// have NST - 1 steps to land. Loads for slices past the last one go through zero-length buffer resources: they
// write zeros into a stage no later step multiplies, and every step counts the same number of loads.
// Activations load 16 bytes (8 positions) per lane, a quarter of the load instructions of 4-byte loads: the address
// work per load instruction, not the bytes, bounds how fast a CU issues them. A chunk may run past its row's end into
// the padding positions, so the epilogue selects out the two shifted terms that would read them.
// Whole 32-channel slices only (C % 32 == 0), even rows and a 4-byte aligned x (4-byte aligned 16-byte chunks).
template <int P, int NBW>
struct PipeSched {
  static constexpr int G = P >= 16 ? 16 : P;
  static constexpr int NBR = (16 * (NBW - 1) + 2 * P) / G + 1;
  static constexpr int NM = 9 * NBW;                         // MFMAs per slice: tap-major, NBW blocks per tap
  static constexpr int NRD = 9 + 2 * NBR;                    // LDS reads per slice: 9 weight runs, then pixel halves
  static constexpr int NRS = NRD < NM ? NRD : NM;            // slots carrying reads
  static constexpr int PB = NRD < NM - 1 ? NRD : NM - 1;     // first slot carrying a transpose (after every read)
  static constexpr int rd_slot(int q) { return q * NRS / NRD; }
  static constexpr int perm_slot(int p) { return PB + p * (NM - PB) / 36; }
  static constexpr int load_slot(int q, int ni) { return q * NM / ni; }
};

template <typename E, int P, int NBW, int NST>
__global__ __launch_bounds__(256, 1) void slab_pipe_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                          float* __restrict__ partial, SlabGeom g) {
  using Sh = SlabShape<P, NBW, NST>;
  using Sc = PipeSched<P, NBW>;
  constexpr int CS = Sh::CS, NW = Sh::NW, RW = Sh::RW, RB = Sh::RB, NR = Sh::NR, G = Sh::G, NBR = Sh::NBR;
  constexpr int CPF = Sh::CPF, WCH = Sh::WCH, WPITCH = Sh::WPITCH, KBW = Sh::KBW, WST = Sh::WST, CHP = Sh::CHP;
  constexpr int ACT = Sh::ACT;
  constexpr int WOFF = NST * ACT;      // LDS: [NST activation stages][NST weight stages]
  constexpr int KA = ACT / 1024 / NW;  // 16-byte activation loads per wave per slice, two channel regions each
  static_assert(CHP == 512 && KA * 2 == 8, "a wave's 8 channels take KA loads of two 512-byte channel regions");
  constexpr int NI = KBW + KA;         // loads per wave per slice
  constexpr int NM = Sc::NM, NRD = Sc::NRD;
  constexpr int U = NST % 2 == 0 ? NST : 2 * NST;  // steps per loop turn: fragment set and stages are constants
  static_assert(NST >= 3, "a slice loads NST - 1 steps ahead of its use");
  static_assert((NST - 1) * NI + 4 < 64, "loads in flight (and the bias loads) fit the vmcnt counter");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  args_in_sgprs(x, w, bias, y, partial, g);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fh = wave & 1, wr = wave >> 1;

  const int slot = int(blockIdx.x);
  const int unit = (slot >> 3) + (slot & 7) * g.per_xcd;
  if (unit >= g.n_units) return;
  const SlabUnit un = decode_unit(unit, g);
  const int b = un.b, z = un.z;
  const int o0 = un.ob * kSlTO, oh0 = un.band * RB;
  int s_beg = 0, ns = g.S;
  if (g.split > 1) {
    s_beg = (g.S * z) / g.split;
    ns = (g.S * (z + 1)) / g.split - s_beg;
  }
  const int nrows = min(RB, g.H - oh0);

  const v4i xr = make_vsharp(x, g.x_bytes), wrs = make_vsharp(w, g.w_bytes);
  const v4i x0 = make_vsharp(x, 0), w0 = make_vsharp(w, 0);  // every offset out of range: loads give zeros
  const unsigned lds0 = lds_addr(lds);

  const int f0 = o0 + fh * 16 + 4 * (lane >> 4);
  uint32_t bbits[4];
  {
    const v4i br = make_vsharp(bias, g.split == 1 && bias != nullptr ? 2 * g.O : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) bbits[i] = load2s(br, 2 * min(f0 + i, g.O - 1), 0);
  }

  // per-lane load offsets, worked out branch-free (value, then a select) so the first loads go out early
  int w_voff[KBW];
  const int wrow = g.C * 18;  // bytes of one filter's OIHW weights
#pragma unroll
  for (int kb = 0; kb < KBW; ++kb) {
    const int u = (wave + NW * kb) * 64 + lane, f = u / CPF, k = u - f * CPF;
    const int val = (o0 + f) * wrow + 16 * k;
    const bool ok = (f < kSlTO) & (k < WCH) & (o0 + f < g.O);
    w_voff[kb] = ok ? val : kOut;
  }
  // activations: 16 bytes (8 positions) per lane; lane = (channel cl of the load's pair, segment slot, half). A chunk
  // that starts inside a row may run past its end into the padding positions (the epilogue never reads them there);
  // rows outside the image load zeros. Load q covers channels 8 * wave + 2q + cl, whose swizzle depends on q % 2 only.
  int a_voff[2];
  {
    const int cl = lane >> 5, sslot = (lane >> 1) & 15, half = lane & 1;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int pos = ((sslot ^ seg_swz(8 * wave + 2 * e + cl)) << 4) + 8 * half;
      const int row = pos / P, col = pos % P, ih = oh0 - 1 + row;
      const int val = (cl * g.HW + ih * g.W + col) * 2;
      const bool ok = (row < NR) & (unsigned(ih) < unsigned(g.H)) & (col < g.W);
      a_voff[e] = ok ? val : kOut;
    }
  }
  const int hw2 = g.HW * 2;
  const int a_soff0 = (b * g.C + s_beg * CS + 8 * wave) * hw2;  // + slice * CS * hw2 + (q / R) * hw2
  const int w_soff0 = s_beg * CS * 18;                           // + slice * CS * 18

  // load q of slice s (relative to s_beg) into stage ST: q < KA this wave's activation rows, then its weight blocks
  struct SliceArgs {
    v4i xs, ws;
    int a_soff, w_soff;
  };
  auto slice_args = [&](int s) __attribute__((always_inline)) {
    const bool real = s < ns;
    return SliceArgs{real ? xr : x0, real ? wrs : w0, real ? a_soff0 + s * CS * hw2 : 0, real ? w_soff0 + s * CS * 18 : 0};
  };
  auto load_one = [&](auto qc, auto st_c, const SliceArgs& sa) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value, ST = decltype(st_c)::value;
    if constexpr (q < KA) {
      dma16s(sa.xs, lds0 + unsigned(ST * ACT + (wave * KA + q) * 1024), a_voff[q & 1], sa.a_soff + 2 * q * hw2);
    } else {
      constexpr int kb = q - KA;
      dma16s(sa.ws, lds0 + unsigned(WOFF + ST * WST + (wave + NW * kb) * 1024), w_voff[kb], sa.w_soff);
    }
  };
  auto load_slice = [&](int s, auto st_c) __attribute__((always_inline)) {
    const SliceArgs sa = slice_args(s);
    for_seq([&](auto qc) __attribute__((always_inline)) { load_one(qc, st_c, sa); },
            std::make_integer_sequence<int, NI>{});
  };

  // ---- prologue: slices 0 .. NST-2 start loading before any fragment address is worked out ----
  for_seq([&](auto sc) __attribute__((always_inline)) { load_slice(decltype(sc)::value, sc); },
          std::make_integer_sequence<int, NST - 1>{});
  __builtin_amdgcn_sched_barrier(0);

  const unsigned a_rd = lds0 + unsigned(WOFF + (fh * 16 + (lane & 15)) * WPITCH + 8 * (lane >> 4) * 18);
  unsigned b_rd[NBR][2];
#pragma unroll
  for (int u = 0; u < NBR; ++u) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ch = 8 * (lane >> 4) + 4 * h + ((lane & 15) >> 2);
      const int pos = wr * RW * P + u * G + 4 * (lane & 3);
      b_rd[u][h] = lds0 + unsigned(ch * CHP + (((pos >> 4) ^ seg_swz(ch)) << 5) + (pos & 15) * 2);
    }
  }

  f32x4 acc[3][NBW];
#pragma unroll
  for (int s2 = 0; s2 < 3; ++s2) {
#pragma unroll
    for (int j2 = 0; j2 < NBW; ++j2) acc[s2][j2] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  u32x4 fw[2][9], fb[2][NBR];
  uint32_t d[36];
  // read q of the slice in stage ST into fragment set S: q < 9 the lane's 16-byte piece t = q of its weight run,
  // then pixel block (q - 9) / 2, channel quad (q - 9) % 2
  auto read_one = [&](auto qc, auto st_c, auto set_c) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value, ST = decltype(st_c)::value, S = decltype(set_c)::value;
    if constexpr (q < 9) {
      const u32x4 v = rd16(a_rd + unsigned(ST * WST + 16 * q));
      d[4 * q] = v.x, d[4 * q + 1] = v.y, d[4 * q + 2] = v.z, d[4 * q + 3] = v.w;
    } else {
      constexpr int u = (q - 9) / 2, h = (q - 9) % 2;
      const u32x2 v = rd_tr(b_rd[u][h] + unsigned(ST * ACT));
      fb[S][u][2 * h] = v.x;
      fb[S][u][2 * h + 1] = v.y;
    }
  };
  // transpose p: dword p % 4 of tap p / 4's weight fragment (8 channels of one tap per lane)
  auto perm_one = [&](auto pc, auto set_c) __attribute__((always_inline)) {
    constexpr int p = decltype(pc)::value, S = decltype(set_c)::value, t = p / 4, c = p % 4;
    fw[S][t][c] = pick2(d, 18 * c + t, 18 * c + 9 + t);
  };
  auto mfma_one = [&](auto kc, auto set_c) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value, S = decltype(set_c)::value;
    constexpr int t = k / NBW, j = k % NBW, r = t / 3, sc = t % 3;
    acc[sc][j] = E::mfma(fw[S][t], fb[S][(16 * j + r * P) / G], acc[sc][j]);
  };

  // ---- the last stage loads once the bias and slice 0 have landed (loads in flight stay within the counter); slice 0
  // is read into set 0 ----
  wait_vmcnt<(NST - 2) * NI>();
  load_slice(NST - 1, std::integral_constant<int, NST - 1>{});
  stage_barrier();  // slice 0 has landed for every wave
  for_seq([&](auto qc) __attribute__((always_inline)) {
    read_one(qc, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
  }, std::make_integer_sequence<int, NRD>{});
  for_seq([&](auto pc) __attribute__((always_inline)) { perm_one(pc, std::integral_constant<int, 0>{}); },
          std::make_integer_sequence<int, 36>{});

  // ---- step j (u = j mod U): slice j multiplies from set u % 2 ----
  auto step = [&](int j, auto u_c) __attribute__((always_inline)) {
    constexpr int uu = decltype(u_c)::value;
    constexpr int cur = uu & 1, nxt = cur ^ 1, st_rd = (uu + 1) % NST, st_ld = uu % NST;
    wait_vmcnt<(NST - 2) * NI>();  // this wave's loads of slice j + 1 have landed (slices j+2 .. j+NST-1 in flight)
    stage_barrier();               // ... every wave's, and every wave has read slice j out of stage st_ld
    const SliceArgs sa = slice_args(j + NST);
    __builtin_amdgcn_sched_barrier(0);
    for_seq([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      mfma_one(kc, std::integral_constant<int, cur>{});
      for_seq([&](auto qc) __attribute__((always_inline)) {
        if constexpr (Sc::rd_slot(decltype(qc)::value) == k)
          read_one(qc, std::integral_constant<int, st_rd>{}, std::integral_constant<int, nxt>{});
      }, std::make_integer_sequence<int, NRD>{});
      for_seq([&](auto qc) __attribute__((always_inline)) {
        if constexpr (Sc::load_slot(decltype(qc)::value, NI) == k)
          load_one(qc, std::integral_constant<int, st_ld>{}, sa);
      }, std::make_integer_sequence<int, NI>{});
      for_seq([&](auto pc) __attribute__((always_inline)) {
        if constexpr (Sc::perm_slot(decltype(pc)::value) == k) perm_one(pc, std::integral_constant<int, nxt>{});
      }, std::make_integer_sequence<int, 36>{});
      __builtin_amdgcn_sched_barrier(0);
    }, std::make_integer_sequence<int, NM>{});
  };
  for (int j = 0; j < ns; j += U) {
    for_seq([&](auto uc) __attribute__((always_inline)) {
      if (j + decltype(uc)::value < ns) step(j + decltype(uc)::value, uc);
    }, std::make_integer_sequence<int, U>{});
  }
  wait_vmcnt<0>();  // the zero loads past the last slice (and the bias loads, long landed)
#pragma unroll
  for (int i = 0; i < 4; ++i) touch_v(bbits[i]);
  slab_store<E, P, NBW, true>(acc, bbits, lane, wr, oh0, nrows, b, z, o0, f0, y, partial, g);
}

// ---- split form: loader waves beside the multiplying waves ----
// The pipelined form's waves issue their own direct-to-LDS loads between MFMAs. Those loads are cheap in bandwidth
// (the L2 serves the 36 KB a slice needs in a fraction of a step) but each one can hold its wave at issue while the
// texture-address FIFO is full, and with one wave per SIMD the MFMA stream behind it waits too. This form gives
// every SIMD a second wave that only loads: waves 0-3 multiply (their slot schedule has LDS reads, transposes and
// MFMAs, no vector-memory instruction), waves 4-7 issue the same loads the pipelined form's waves 0-3 issue, wait for
// them and meet the multiplying waves at the one barrier per step. The same LDS stages, load blocks and fragment
// reads as the pipelined form.
// Registers: two waves per SIMD leave each at most 256. The multiplying waves keep one set of weight fragments:
// slice j's taps 5-8 are transposed at the start of step j (their last use in slice j - 1 was in step j - 1, their
// first use in slice j comes after slot 35), then slice j + 1's weight runs are read over the same registers, and its
// taps 0-4 are transposed at the end of step j, after their last use in slice j (slot 34).
template <int P, int NBW>
struct SplitSched {
  static constexpr int G = P >= 16 ? 16 : P;
  static constexpr int NBR = (16 * (NBW - 1) + 2 * P) / G + 1;
  static constexpr int NM = 9 * NBW;
  static constexpr int TL = 5;                   // taps 0 .. TL-1 transposed late, TL .. 8 early
  static constexpr int NE = 4 * (9 - TL);        // early transposes (taps TL .. 8 of this step's slice)
  static constexpr int NLATE = 4 * TL;           // late transposes (taps 0 .. TL-1 of the next slice)
  static constexpr int NB = 2 * NBR;             // pixel-fragment reads of the next slice
  static constexpr int E_END = NM * 2 / 7;       // early transposes within slots [0, E_END)
  static constexpr int W_BEG = E_END;            // weight-run reads: slots W_BEG .. W_BEG + 8
  static constexpr int B_BEG = W_BEG + 9;        // pixel reads after them
  static constexpr int L_BEG = NM - (NLATE + 1) / 2 - 1;  // late transposes, two per slot, ending at the last slot
  static constexpr int early_slot(int p) { return p * E_END / NE; }
  static constexpr int wread_slot(int q) { return W_BEG + q; }
  static constexpr int bread_slot(int q) { return B_BEG + q * (L_BEG - B_BEG) / NB; }
  static constexpr int late_slot(int p) { return L_BEG + p / 2; }
  static_assert(early_slot(NE - 1) < NBW * TL, "early transposes end before tap TL's first use (slot NBW * TL)");
  static_assert(L_BEG >= NBW * TL, "late transposes start after the last use of tap TL - 1 (slot NBW * TL - 1)");
  static_assert(B_BEG < L_BEG && late_slot(NLATE - 1) < NM, "slot plan");
};

// The direct-to-LDS loads of loader share lw (0..3) of a slice: KA activation blocks (8 channels' rows, two channel
// regions per 16-byte load) and KBW weight blocks, as the pipelined form's wave lw issues them; slices past the unit's
// last load through zero-length resources (every step counts the same loads).
template <int P, int NBW, int NST>
struct SplitShare {
  using Sh = SlabShape<P, NBW, NST>;
  static constexpr int CS = Sh::CS, NW = Sh::NW, NR = Sh::NR, CPF = Sh::CPF, WCH = Sh::WCH, KBW = Sh::KBW;
  static constexpr int ACT = Sh::ACT, WST = Sh::WST, WOFF = NST * ACT, KA = ACT / 1024 / NW;
  v4i xr, wrs, x0, w0;
  int w_voff[KBW], a_voff[2];
  int hw2, a_soff0, w_soff0, lw, ns;
  unsigned lds0;
  __device__ __forceinline__ SplitShare(const uint16_t* x, const uint16_t* w, const SlabGeom& g, int lw_, int lane, int b,
                                        int o0, int oh0, int s_beg, int ns_, unsigned lds0_)
      : lw(lw_), ns(ns_), lds0(lds0_) {
    xr = make_vsharp(x, g.x_bytes), wrs = make_vsharp(w, g.w_bytes);
    x0 = make_vsharp(x, 0), w0 = make_vsharp(w, 0);  // every offset out of range: loads give zeros
    const int wrow = g.C * 18;  // bytes of one filter's OIHW weights
#pragma unroll
    for (int kb = 0; kb < KBW; ++kb) {
      const int u = (lw + NW * kb) * 64 + lane, f = u / CPF, k = u - f * CPF;
      const int val = (o0 + f) * wrow + 16 * k;
      const bool ok = (f < kSlTO) & (k < WCH) & (o0 + f < g.O);
      w_voff[kb] = ok ? val : kOut;
    }
    const int cl = lane >> 5, sslot = (lane >> 1) & 15, half = lane & 1;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int pos = ((sslot ^ seg_swz(8 * lw + 2 * e + cl)) << 4) + 8 * half;
      const int row = pos / P, col = pos % P, ih = oh0 - 1 + row;
      const int val = (cl * g.HW + ih * g.W + col) * 2;
      const bool ok = (row < NR) & (unsigned(ih) < unsigned(g.H)) & (col < g.W);
      a_voff[e] = ok ? val : kOut;
    }
    hw2 = g.HW * 2;
    a_soff0 = (b * g.C + s_beg * CS + 8 * lw) * hw2;
    w_soff0 = s_beg * CS * 18;
  }
  // load q of slice s into stage st: q < KA the share's activation rows, then its weight blocks
  __device__ __forceinline__ void issue(int s, int st) const {
    const bool real = s < ns;
    const v4i xs = real ? xr : x0, ws = real ? wrs : w0;
    const int a_soff = real ? a_soff0 + s * CS * hw2 : 0, w_soff = real ? w_soff0 + s * CS * 18 : 0;
#pragma unroll
    for (int q = 0; q < KA; ++q)
      dma16s(xs, lds0 + unsigned(st * ACT + (lw * KA + q) * 1024), a_voff[q & 1], a_soff + 2 * q * hw2);
#pragma unroll
    for (int kb = 0; kb < KBW; ++kb)
      dma16s(ws, lds0 + unsigned(WOFF + st * WST + (lw + NW * kb) * 1024), w_voff[kb], w_soff);
  }
};

// Staged epilogue of the split form (g.y_stage: whole images per unit, O % 32 == 0, 16-byte aligned y, P == 16). The
// unit's 32 output planes are one contiguous run of 64 * HW bytes; the multiplying waves write their pixel pairs at
// their places in that run into an LDS activation stage that no load targets any more, and after one barrier all eight
// waves write the run with 16-byte device-scope stores (store16_wt), each store instruction one contiguous kilobyte of
// y, so whole lines are written through the L2 and none is left dirty for the end of the launch (the direct
// pixel-pair stores spread every instruction over eight filter planes in 28-byte pieces).
// Lanes past the last column write their pairs to a dummy area after the run (inside the stage), so no lane is masked.
template <typename E, int NBW>
__device__ __forceinline__ void split_stage_rows(const f32x4 (&acc)[3][NBW], const uint32_t (&bbits)[4], int lane,
                                                 int wr, int fl, int nrows, unsigned stg, const SlabGeom& g) {
  constexpr int RW = NBW;  // P == 16: one output row per 16-position block
  float bv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bv[i] = E::to_f32(uint16_t(bbits[i]));
  const PairSel ps(lane);
  const int fp = int(ps.odd) * 2, col = (lane & 15) - int(ps.odd);
  const unsigned plane = unsigned(2 * g.HW);
  const unsigned base = stg + (col < g.W ? unsigned(((fl + fp) * g.HW + wr * RW * g.W + col) * 2) : 32u * plane);
  typedef __attribute__((address_space(3))) uint32_t lds_u32;
  auto rows = [&](auto relu_c) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      if (wr * RW + j >= nrows) break;
      uint32_t wa, wb;
      row_pairs<E, decltype(relu_c)::value>(slab_column<16, NBW, true>(acc, j, lane, wr, g.W), bv, ps, &wa, &wb);
      const unsigned a = base + unsigned(2 * j * g.W);
      *reinterpret_cast<lds_u32*>(size_t(a)) = wa;
      *reinterpret_cast<lds_u32*>(size_t(a + plane)) = wb;
    }
  };
  if (g.relu) rows(std::true_type{});
  else rows(std::false_type{});
}

// The staged run of 64 * HW bytes (4 * HW 16-byte chunks) from LDS to y, by the workgroup's 512 threads.
__device__ __forceinline__ void split_copy_out(unsigned stg, uint16_t* __restrict__ y, int b, int o0, int tid,
                                               const SlabGeom& g) {
  const int n16 = 4 * g.HW;
  const v4i yr = make_vsharp(y + static_cast<long long>(b * g.O + o0) * g.HW, 16 * n16);
  for (int c = tid; c < n16; c += 512) store16_wt(yr, 16 * c, rd16(stg + unsigned(16 * c)));
}

template <typename E, int P, int NBW, int NST>
__global__ __launch_bounds__(512, 1) void slab_split_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w,
                                                           const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                           float* __restrict__ partial, SlabGeom g) {
  using Sh = SlabShape<P, NBW, NST>;
  using Sc = SplitSched<P, NBW>;
  constexpr int NW = Sh::NW, RW = Sh::RW, RB = Sh::RB, G = Sh::G, NBR = Sh::NBR;
  constexpr int WPITCH = Sh::WPITCH, KBW = Sh::KBW, WST = Sh::WST, CHP = Sh::CHP;
  constexpr int ACT = Sh::ACT;
  constexpr int WOFF = NST * ACT;      // LDS: [NST activation stages][NST weight stages]
  constexpr int KA = ACT / 1024 / NW;  // 16-byte activation loads per loader per slice, two channel regions each
  static_assert(CHP == 512 && KA * 2 == 8, "a loader's 8 channels take KA loads of two 512-byte channel regions");
  constexpr int NI = KBW + KA;         // loads per loader per slice
  constexpr int NM = Sc::NM, NB = Sc::NB, TL = Sc::TL;
  constexpr int U = NST % 2 == 0 ? NST : 2 * NST;  // steps per loop turn: fragment set and stages are constants
  static_assert(NST >= 3, "a slice loads NST - 1 steps ahead of its use");
  static_assert((NST - 1) * NI < 64, "loads in flight fit the vmcnt counter");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  args_in_sgprs(x, w, bias, y, partial, g);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slot = int(blockIdx.x);
  const int unit = (slot >> 3) + (slot & 7) * g.per_xcd;
  if (unit >= g.n_units) return;
  const SlabUnit un = decode_unit(unit, g);
  const int b = un.b, z = un.z;
  const int o0 = un.ob * kSlTO, oh0 = un.band * RB;
  int s_beg = 0, ns = g.S;
  if (g.split > 1) {
    s_beg = (g.S * z) / g.split;
    ns = (g.S * (z + 1)) / g.split - s_beg;
  }
  const unsigned lds0 = lds_addr(lds);

  if (wave >= NW) {
    // ================= loader wave lw = wave - NW: the loads the pipelined form's wave lw issues =================
    const SplitShare<P, NBW, NST> ld(x, w, g, wave - NW, lane, b, o0, oh0, s_beg, ns, lds0);
    // slice 0 first (slice 1 is the multiplying waves': each issues its partner loader's share at its start, so
    // eight waves load the cold start's two slices); slice 2 goes out once slice 0 has landed
    static_assert(NST == 3, "the start-up sequence below issues slices 0 and then 2 (slice 1: the multiplying waves)");
    ld.issue(0, 0);
    wait_vmcnt<0>();  // slice 0
    stage_barrier();  // B0: slice 0 is in LDS
    ld.issue(2, 2);
    stage_barrier();  // start of step 0 (slice 1: the multiplying waves waited for their loads)
    for (int j = 0; j + 1 < ns; ++j) {
      // step j: slice j was read in step j - 1, so its stage takes slice j + NST; slice j + 2 must land before the
      // barrier that starts step j + 1
      ld.issue(j + NST, j % NST);
      wait_vmcnt<(NST - 2) * NI>();
      stage_barrier();
    }
    wait_vmcnt<0>();  // the zero loads past the last slice land before this wave ends
    if constexpr (P == 16) {
      if (g.y_stage) {
        stage_barrier();  // the multiplying waves' rows are in LDS
        split_copy_out(lds0 + unsigned(((ns - 1) % NST) * ACT), y, b, o0, tid, g);
      }
    }
    return;
  }

  // ================= multiplying wave: (filter half fh, row half wr) =================
  {  // first, slice 1's share `wave` (its partner loader issues slice 0 and the later slices)
    const SplitShare<P, NBW, NST> ld(x, w, g, wave, lane, b, o0, oh0, s_beg, ns, lds0);
    ld.issue(1, 1);
  }
  const int fh = wave & 1, wr = wave >> 1;
  const int nrows = min(RB, g.H - oh0);
  const int f0 = o0 + fh * 16 + 4 * (lane >> 4);
  uint32_t bbits[4];
  {
    const v4i br = make_vsharp(bias, g.split == 1 && bias != nullptr ? 2 * g.O : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) bbits[i] = load2s(br, 2 * min(f0 + i, g.O - 1), 0);
  }
  const unsigned a_rd = lds0 + unsigned(WOFF + (fh * 16 + (lane & 15)) * WPITCH + 8 * (lane >> 4) * 18);
  unsigned b_rd[NBR][2];
#pragma unroll
  for (int u = 0; u < NBR; ++u) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ch = 8 * (lane >> 4) + 4 * h + ((lane & 15) >> 2);
      const int pos = wr * RW * P + u * G + 4 * (lane & 3);
      b_rd[u][h] = lds0 + unsigned(ch * CHP + (((pos >> 4) ^ seg_swz(ch)) << 5) + (pos & 15) * 2);
    }
  }
  f32x4 acc[3][NBW];
#pragma unroll
  for (int s2 = 0; s2 < 3; ++s2) {
#pragma unroll
    for (int j2 = 0; j2 < NBW; ++j2) acc[s2][j2] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  u32x4 fw[9], fb[2][NBR];
  uint32_t d[36];
  auto read_w = [&](auto qc, auto st_c) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value, ST = decltype(st_c)::value;
    const u32x4 v = rd16(a_rd + unsigned(ST * WST + 16 * q));
    d[4 * q] = v.x, d[4 * q + 1] = v.y, d[4 * q + 2] = v.z, d[4 * q + 3] = v.w;
  };
  auto read_b = [&](auto qc, auto st_c, auto set_c) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value, ST = decltype(st_c)::value, S = decltype(set_c)::value;
    constexpr int u = q / 2, h = q % 2;
    const u32x2 v = rd_tr(b_rd[u][h] + unsigned(ST * ACT));
    fb[S][u][2 * h] = v.x;
    fb[S][u][2 * h + 1] = v.y;
  };
  // transpose p of tap t = p / 4: dword p % 4 of the tap's weight fragment (8 channels of one tap per lane)
  auto perm_tap = [&](auto pc) __attribute__((always_inline)) {
    constexpr int p = decltype(pc)::value, t = p / 4, c = p % 4;
    fw[t][c] = pick2(d, 18 * c + t, 18 * c + 9 + t);
  };
  auto mfma_one = [&](auto kc, auto set_c) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value, S = decltype(set_c)::value;
    constexpr int t = k / NBW, j = k % NBW, r = t / 3, sc = t % 3;
    acc[sc][j] = E::mfma(fw[t], fb[S][(16 * j + r * P) / G], acc[sc][j]);
  };

  stage_barrier();  // B0: slice 0 is in LDS
  // slice 0 into registers: its weight runs, its pixel fragments (set 0) and the transposes of taps 0 .. TL-1 (the
  // others are done at the start of step 0, as in every step)
  for_seq([&](auto qc) __attribute__((always_inline)) { read_w(qc, std::integral_constant<int, 0>{}); },
          std::make_integer_sequence<int, 9>{});
  for_seq([&](auto qc) __attribute__((always_inline)) {
    read_b(qc, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
  }, std::make_integer_sequence<int, NB>{});
  for_seq([&](auto pc) __attribute__((always_inline)) { perm_tap(pc); }, std::make_integer_sequence<int, 4 * TL>{});

  // ---- step j (u = j mod U): slice j multiplies from pixel set u % 2 ----
  auto step = [&](auto u_c) __attribute__((always_inline)) {
    constexpr int uu = decltype(u_c)::value;
    constexpr int cur = uu & 1, nxt = cur ^ 1, st_rd = (uu + 1) % NST;
    stage_barrier();  // slice j + 1 has landed (the loaders waited), every wave is done with step j - 1
    __builtin_amdgcn_sched_barrier(0);
    for_seq([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      mfma_one(kc, std::integral_constant<int, cur>{});
      for_seq([&](auto pc) __attribute__((always_inline)) {
        constexpr int p = decltype(pc)::value;
        if constexpr (Sc::early_slot(p) == k) perm_tap(std::integral_constant<int, 4 * TL + p>{});
      }, std::make_integer_sequence<int, Sc::NE>{});
      for_seq([&](auto qc) __attribute__((always_inline)) {
        if constexpr (Sc::wread_slot(decltype(qc)::value) == k) read_w(qc, std::integral_constant<int, st_rd>{});
      }, std::make_integer_sequence<int, 9>{});
      for_seq([&](auto qc) __attribute__((always_inline)) {
        if constexpr (Sc::bread_slot(decltype(qc)::value) == k)
          read_b(qc, std::integral_constant<int, st_rd>{}, std::integral_constant<int, nxt>{});
      }, std::make_integer_sequence<int, NB>{});
      for_seq([&](auto pc) __attribute__((always_inline)) {
        if constexpr (Sc::late_slot(decltype(pc)::value) == k) perm_tap(pc);
      }, std::make_integer_sequence<int, Sc::NLATE>{});
      __builtin_amdgcn_sched_barrier(0);
    }, std::make_integer_sequence<int, NM>{});
  };
  wait_vmcnt<4>();  // this wave's share of slice 1 (the 4 bias loads after it may be in flight)
  for (int j = 0; j < ns; j += U) {
    for_seq([&](auto uc) __attribute__((always_inline)) {
      if (j + decltype(uc)::value < ns) step(uc);
    }, std::make_integer_sequence<int, U>{});
  }
  wait_vmcnt<0>();  // the bias loads
#pragma unroll
  for (int i = 0; i < 4; ++i) touch_v(bbits[i]);
  if constexpr (P == 16) {
    if (g.y_stage) {
      // slice ns - 1's stage: its last load landed before step ns - 2, its last reads were in step ns - 2, and the
      // loads past the last slice (slices ns, ns + 1) target the other two stages
      const unsigned stg = lds0 + unsigned(((ns - 1) % NST) * ACT);
      split_stage_rows<E, NBW>(acc, bbits, lane, wr, f0 - o0, nrows, stg, g);
      stage_barrier();  // every wave's rows are in LDS
      split_copy_out(stg, y, b, o0, tid, g);
      return;
    }
  }
  slab_store<E, P, NBW, true>(acc, bbits, lane, wr, oh0, nrows, b, z, o0, f0, y, partial, g);
}

// kernel forms: slab_kernel (double-buffered fragments), slab_lean_kernel (single fragment set, at most 256
// VGPR+AGPR), slab_pipe_kernel (double-buffered fragments, fixed slot schedule, whole slices)
constexpr int kFull = 0, kLean = 1, kPipe = 2, kSplit = 3;
struct SlabCfg {
  int P, NBW, NST;
  int form;
};
// (row pitch, 16-position blocks per wave, load stages, form)
constexpr SlabCfg kSlabCfgs[] = {{16, 7, 3, kFull}, {16, 7, 2, kFull}, {16, 4, 3, kFull}, {8, 2, 3, kFull},
                                 {8, 4, 3, kFull},  {32, 4, 3, kFull}, {16, 7, 2, kLean}, {16, 4, 2, kLean},
                                 {8, 2, 2, kLean},  {8, 4, 2, kLean},  {32, 4, 2, kLean}, {16, 7, 3, kLean},
                                 {16, 7, 3, kPipe}, {16, 7, 3, kSplit}};
constexpr int kSlabN = int(sizeof(kSlabCfgs) / sizeof(kSlabCfgs[0]));

template <int I>
struct CfgT {
  static constexpr int P = kSlabCfgs[I].P, NBW = kSlabCfgs[I].NBW, NST = kSlabCfgs[I].NST;
  static constexpr int FORM = kSlabCfgs[I].form;
  using Sh = SlabShape<P, NBW, NST>;
  static constexpr int LDS = Sh::LDS;
};

typedef void (*SlabFn)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*, SlabGeom);

// the 2-byte register form exists where it needs at most 16 loads per thread and slice
// (the register forms write a slice one step after loading it, so they need three stages or more)
template <int I>
SlabFn pick_fn(bool bf, int mode) {
  using C = CfgT<I>;
  if constexpr (C::FORM == kLean) {
    if (mode == kDma4)
      return bf ? &slab_lean_kernel<Bf16, C::P, C::NBW, C::NST> : &slab_lean_kernel<Fp16, C::P, C::NBW, C::NST>;
    return nullptr;
  } else if constexpr (C::FORM == kPipe) {
    if (mode == kDma4)
      return bf ? &slab_pipe_kernel<Bf16, C::P, C::NBW, C::NST> : &slab_pipe_kernel<Fp16, C::P, C::NBW, C::NST>;
    return nullptr;
  } else if constexpr (C::FORM == kSplit) {
    if (mode == kDma4)
      return bf ? &slab_split_kernel<Bf16, C::P, C::NBW, C::NST> : &slab_split_kernel<Fp16, C::P, C::NBW, C::NST>;
    return nullptr;
  } else {
    if (mode == kDma4)
      return bf ? &slab_kernel<Bf16, C::P, C::NBW, C::NST, kDma4> : &slab_kernel<Fp16, C::P, C::NBW, C::NST, kDma4>;
    if constexpr (C::NST >= 3) {
      if constexpr (C::Sh::KR <= 16)
        return bf ? &slab_kernel<Bf16, C::P, C::NBW, C::NST, kReg2> : &slab_kernel<Fp16, C::P, C::NBW, C::NST, kReg2>;
    }
    return nullptr;
  }
}

struct SlabShapeInfo {
  int P, RB, CS, NT, LDS, ACT, FORM;
};

template <int I>
SlabShapeInfo shape_of() {
  using Sh = typename CfgT<I>::Sh;
  // the split form adds one loader wave per SIMD
  return SlabShapeInfo{CfgT<I>::P,   Sh::RB, Sh::CS, CfgT<I>::FORM == kSplit ? 2 * Sh::NT : Sh::NT, CfgT<I>::LDS,
                       Sh::ACT, CfgT<I>::FORM};
}

template <int... Is>
bool dispatch(int cfg, bool bf, int mode, SlabFn* fn, SlabShapeInfo* si, std::integer_sequence<int, Is...>) {
  bool hit = false;
  ((cfg == Is ? (*si = shape_of<Is>(), *fn = pick_fn<Is>(bf, mode), hit = true) : false), ...);
  return hit;
}

struct SlabPlan {
  SlabGeom g;
  SlabFn fn;
  int nt, lds;
};

// Geometry checks and launch parameters of configuration cfg; the activation load form and the output store width
// are decided from the pointers.
int slab_prepare(int cfg, const gie_conv_geom* gg, int dtype, const void* x, const void* y, const float* partial,
                 int split, SlabPlan* sp) {
  if (cfg < 0 || cfg >= kSlabN || !gg) return GIE_HIP_EINVAL;
  if (gg->kernel_h != 3 || gg->kernel_w != 3 || gg->stride_h != 1 || gg->stride_w != 1 || gg->pad_h != 1 ||
      gg->pad_w != 1)
    return GIE_HIP_EUNSUPPORTED;
  if (gg->batch <= 0 || gg->in_channels <= 0 || gg->out_channels <= 0 || gg->in_h <= 0 || gg->in_w <= 0)
    return GIE_HIP_EINVAL;
  if (gg->in_channels % 8 != 0) return GIE_HIP_EUNSUPPORTED;  // 16-byte chunks of the weight runs
  if ((kSlabCfgs[cfg].form == kPipe || kSlabCfgs[cfg].form == kSplit) && gg->in_channels % 32 != 0)
    return GIE_HIP_EUNSUPPORTED;  // whole slices
  const long long hw = 1LL * gg->in_h * gg->in_w;
  const bool bf = dtype == GIE_HIP_BF16;
  SlabShapeInfo si{};
  SlabFn fn = nullptr;
  if (!dispatch(cfg, bf, kDma4, &fn, &si, std::make_integer_sequence<int, kSlabN>{})) return GIE_HIP_EINVAL;
  if (gg->in_w + 1 > si.P) return GIE_HIP_EUNSUPPORTED;
  const int bands = (gg->in_h + si.RB - 1) / si.RB;
  // activation load form: even rows of a 4-byte aligned x take direct loads; odd rows or a 2-byte aligned x take
  // 2-byte register loads (full form only)
  const bool even = gg->in_w % 2 == 0 && !(reinterpret_cast<uintptr_t>(x) & 3u);
  SlabFn alt = nullptr;
  if (!even) {
    dispatch(cfg, bf, kReg2, &alt, &si, std::make_integer_sequence<int, kSlabN>{});
    fn = alt;
  }
  if (fn == nullptr) return GIE_HIP_EUNSUPPORTED;
  const long long xb = 2LL * gg->batch * gg->in_channels * hw;
  const long long wb = 18LL * gg->out_channels * gg->in_channels;
  const long long total = 1LL * gg->batch * gg->out_channels * hw;
  // 32-bit buffer offsets with kOut (2^31) past every range: y bytes and FP32 partial bytes below 2^31
  if (xb >= (1LL << 30) || wb >= (1LL << 30) || total >= (1LL << 29)) return GIE_HIP_EUNSUPPORTED;
  const int S = (gg->in_channels + si.CS - 1) / si.CS;
  if (split < 1 || split > S) return GIE_HIP_EINVAL;
  SlabGeom& g = sp->g;
  g.B = gg->batch, g.C = gg->in_channels, g.H = gg->in_h, g.W = gg->in_w, g.O = gg->out_channels, g.HW = int(hw);
  g.S = S;
  g.n_bands = bands;
  g.n_ob = (g.O + kSlTO - 1) / kSlTO;
  const long long units = 1LL * split * g.B * bands * g.n_ob;
  if (units > (1LL << 30)) return GIE_HIP_EUNSUPPORTED;
  g.n_units = int(units);
  g.per_xcd = (g.n_units + 7) / 8;
  // n / d for n < 2^30: l = ceil(log2 d), mg = floor(2^32 (2^l - d) / d) + 1, q = (umulhi(n, mg) + n) >> l
  const auto magic = [](int d, unsigned* mg, int* sh) {
    int l = 0;
    while ((1LL << l) < d) ++l;
    *sh = l;
    *mg = unsigned((((1ULL << l) - unsigned(d)) << 32) / unsigned(d) + 1);
  };
  // unit order: the one whose XCD ranges (per_xcd consecutive units) fetch fewer bytes into their L2 — filter block
  // fastest shares images (few images x every weight), image fastest shares weights (few filter blocks x every image)
  const double wz = 32.0 * gg->in_channels * 18.0 / split;           // one filter block's weights per channel range
  const double xz = 2.0 * gg->in_channels * double(hw) / split / bands;  // one slab's planes per channel range
  const double per = double(g.per_xcd);
  const double by_ob = std::min(double(g.n_ob), per) * wz + std::ceil(per / g.n_ob) * xz;
  const double by_b = std::min(double(g.B) * bands, per) * xz + std::ceil(per / (double(g.B) * bands)) * wz;
  g.order = by_b < by_ob ? 1 : 0;
  g.rad[0] = g.order == 0 ? g.n_ob : g.B;
  g.rad[1] = g.n_bands;
  g.rad[2] = g.order == 0 ? g.B : g.n_ob;
  for (int k = 0; k < 3; ++k) magic(g.rad[k], &g.mg[k], &g.sh[k]);
  g.x_bytes = int(xb), g.w_bytes = int(wb);
  g.relu = gg->relu;
  g.split = split;
  g.total = total;
  g.inv_hw = 1.0f / float(hw);
  g.inv_w = 1.0f / float(gg->in_w);
  // 4-byte stores of pixel pairs: even rows, so every pair starts on an even element of a 4-byte aligned y
  g.y_vec = split == 1 && gg->in_w % 2 == 0 && !(reinterpret_cast<uintptr_t>(y) & 3u);
  // staged output (split form): whole images per unit and whole 32-filter blocks, so a unit's 32 output planes are one
  // run of 64 * HW bytes, 16-byte aligned when y is; the run, plus the dummy words of the lanes past the last column,
  // fits one activation stage
  g.y_stage = si.FORM == kSplit && g.y_vec && bands == 1 && g.O % kSlTO == 0 &&
              !(reinterpret_cast<uintptr_t>(y) & 15u) && 64 * hw + 2 * (1LL * si.RB * gg->in_w + hw) + 4 <= si.ACT;
  sp->fn = fn;
  sp->nt = si.NT;
  sp->lds = si.LDS;
  return GIE_HIP_OK;
}

int launch_slab(const SlabPlan& sp, const void* x, const void* w, const void* bias, void* y, float* partial,
                void* stream) {
  hipLaunchKernelGGL(sp.fn, dim3(unsigned(8 * sp.g.per_xcd)), dim3(unsigned(sp.nt)), sp.lds,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x),
                     static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y),
                     partial, sp.g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}

// Pointer checks shared by the entry points: x, y, bias 2-byte aligned, partials 4-byte aligned; w must be 16-byte
// aligned for the 16-byte weight chunks (GIE_HIP_EUNSUPPORTED otherwise, so a caller can fall back).
int check_pointers(int dtype, const void* x, const void* w, const void* bias, const void* y, const float* partial) {
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if ((bias && (reinterpret_cast<uintptr_t>(bias) & 1u)) || (y && (reinterpret_cast<uintptr_t>(y) & 1u)) ||
      (reinterpret_cast<uintptr_t>(x) & 1u) || (partial && (reinterpret_cast<uintptr_t>(partial) & 3u)))
    return GIE_HIP_EINVAL;
  if (reinterpret_cast<uintptr_t>(w) & 15u) return GIE_HIP_EUNSUPPORTED;
  return GIE_HIP_OK;
}

// ---- allocation-free variant ---------------------------------------------------------------------------------------
// gie_hip_conv_slab_noalloc keeps its FP32 split-K partials in `scratch`, a file-scope device array: every GPU the
// library runs on holds its own copy (kSlabScratchFloats floats = 32 MiB) from module load until the process ends.
// Host code never passes `scratch` itself (on the host that name is a stand-in, not a device address): the first
// call on a device looks up that device's address with hipGetSymbolAddress and every later call uses the kept one.
constexpr long long kSlabScratchFloats = 8LL << 20;
static __device__ __align__(256) float scratch[kSlabScratchFloats];

constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

int raise_lds_limits() {
  for (int cfg = 0; cfg < kSlabN; ++cfg)
    for (int bf = 0; bf < 2; ++bf)
      for (int mode : {kDma4, kReg2}) {
        SlabFn fn = nullptr;
        SlabShapeInfo si{};
        if (!dispatch(cfg, bf != 0, mode, &fn, &si, std::make_integer_sequence<int, kSlabN>{}) || fn == nullptr ||
            si.LDS <= 64 * 1024)
          continue;
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, si.LDS);
        if (e != hipSuccess) return int(e);
      }
  return GIE_HIP_OK;
}

// Device address of the current device's `scratch`. Set-up, once per device with that device current: the symbol
// lookup and the LDS opt-in of every slab kernel (so no later call allocates host bookkeeping either).
int scratch_of_current_device(float** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return int(hipErrorInvalidDevice);
  if (dev < 0 || dev >= kMaxDevices) return GIE_HIP_EUNSUPPORTED;
  float* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return int(e);
      if (addr == nullptr) return int(hipErrorInvalidSymbol);
      if (int rc = raise_lds_limits()) return rc;
      p = static_cast<float*>(addr);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return GIE_HIP_OK;
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_slab_config_count(void) { return kSlabN; }

extern "C" int gie_hip_slab_config_get(int index, gie_slab_config* out) {
  if (index < 0 || index >= kSlabN || !out) return GIE_HIP_EINVAL;
  gie_conv_geom g{};
  g.batch = 1, g.in_channels = 64, g.in_h = 2, g.in_w = 2, g.out_channels = 1;  // even rows: either load form
  g.kernel_h = g.kernel_w = 3, g.stride_h = g.stride_w = 1, g.pad_h = g.pad_w = 1;
  SlabPlan sp;
  if (int rc = slab_prepare(index, &g, GIE_HIP_FP16, nullptr, nullptr, nullptr, 1, &sp)) return rc;
  const SlabCfg& c = kSlabCfgs[index];
  out->tile_m = kSlTO;
  out->rows = 2 * (16 * c.NBW / c.P);
  out->pitch = c.P;
  out->tile_k = 32;
  out->stages = c.NST;
  out->workgroups_per_cu = c.form == kLean && sp.lds <= 80 * 1024 ? 2 : 1;
  out->form = c.form;
  out->threads = sp.nt;
  out->lds_bytes = sp.lds;
  out->version = 5;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_slab_check(int config, const gie_conv_geom* g, int* lds_bytes) {
  SlabPlan sp;
  if (int rc = slab_prepare(config, g, GIE_HIP_FP16, nullptr, nullptr, nullptr, 1, &sp)) return rc;
  if (lds_bytes) *lds_bytes = sp.lds;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_conv_slab(int config, int dtype, const gie_conv_geom* gg, const void* x, const void* w,
                                 const void* bias, void* y, float* partial, int split, void* stream) {
  if (!gg || !x || !w) return GIE_HIP_EINVAL;
  if (split > 1 ? partial == nullptr : y == nullptr) return GIE_HIP_EINVAL;
  if (int rc = check_pointers(dtype, x, w, bias, y, partial)) return rc;
  SlabPlan sp;
  if (int rc = slab_prepare(config, gg, dtype, x, y, partial, split, &sp)) return rc;
  if (int rc = set_lds_limit(reinterpret_cast<const void*>(sp.fn), sp.lds)) return rc;
  return launch_slab(sp, x, w, bias, y, partial, stream);
}

extern "C" int gie_hip_conv_slab_noalloc(int config, int dtype, const gie_conv_geom* gg, const void* x, const void* w,
                                         const void* bias, void* y, int split, void* stream) {
  if (!gg || !x || !w || !y) return GIE_HIP_EINVAL;
  if (int rc = check_pointers(dtype, x, w, bias, y, nullptr)) return rc;
  float* part = nullptr;
  if (int rc = scratch_of_current_device(&part)) return rc;
  SlabPlan sp;
  if (int rc = slab_prepare(config, gg, dtype, x, y, split > 1 ? part : nullptr, split, &sp)) return rc;
  if (split > 1 && 1LL * split * sp.g.total > kSlabScratchFloats) return GIE_HIP_ESCRATCH;
  // every unit of range z writes its whole share of partial[z], so the scratch needs no clearing between calls
  if (int rc = launch_slab(sp, x, w, bias, y, split > 1 ? part : nullptr, stream)) return rc;
  if (split == 1) return GIE_HIP_OK;
  return gie_hip_splitk_reduce(dtype, part, bias, y, sp.g.total, split, sp.g.O, sp.g.HW, sp.g.relu, stream);
}

extern "C" long long gie_hip_slab_scratch_floats(void) { return kSlabScratchFloats; }
