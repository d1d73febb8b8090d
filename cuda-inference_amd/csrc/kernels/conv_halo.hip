// Halo-tiled implicit-GEMM convolution on gfx950 matrix cores (v_mfma_f32_32x32x16_{f16,bf16}, FP32
// accumulation) over the channel-blocked activations xb [B][S][H*W][32] and weights wb [O][S][KH*KW][32]
// (S = ceil(C / 32) slices of 32 channels, zero padded; repack_blocked.hip writes both in one dispatch).
//
// GEMM view (reference naming): M = out_channels, N = batch*out_h*out_w output pixels, K = kh*kw*32*S. A workgroup
// owns TO output channels x TPX consecutive output pixels (a flat range that may span image rows and images)
// and walks the channels in slices of 32. Per slice an LDS stage holds:
//   * the input "halo": every input row the tile's pixels touch, one LDS row ("slot") per (image, input row),
//     each pixel's 32 channels as four 16-byte chunks; columns and rows outside the image are zeros.
//     Consecutive output rows of one image share slots (stride 1: tap row r of output row j reads slot j + r),
//     so each input pixel is loaded once per slice and read by all KH*KW taps from LDS;
//   * the weights [TO][KH*KW][4 chunks].
// Both are filled by direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds): 64 lanes write 1 KiB of
// consecutive LDS per instruction, with no registers, no LDS store instructions and no VALU on the way; each lane
// fetches the global chunk that belongs at its LDS position. Chunks are XOR-swizzled, and each slot starts at a
// bank offset, so the 16-lane groups of every fragment read (16 consecutive output pixels, or 16 consecutive
// output channels) hit 16 distinct bank groups without padding bytes.
// Waves: (TPX/64 pixel halves) x (KH filter rows) x (2 channel halves) = 12 waves for 3x3, three per SIMD. Each
// wave multiplies a 64-pixel x 64-channel tile (2 x 2 blocks of 32x32) for its filter row's KW taps and its 16
// channels of the slice; the KH*2 partial tiles of each pixel half are summed through LDS after the last slice.
// Pipeline: NST LDS stages; the loads of slice i + NST - 1 are in flight while slice i multiplies (fragments of
// tap t + 2 read while tap t multiplies); one counted wait and one barrier per slice. Loads past the data
// (image borders, padding rows/columns, output channels past O, slices after the last) use
// an out-of-range buffer offset, for which the hardware writes zeros.
// Epilogue: bias + ReLU on the FP32 sums, one RNE rounding; the 16-bit tile goes through LDS so waves store
// contiguous runs of output pixels (8-byte stores when 4 pixels share an image row and the address allows, else
// 2-byte stores). Or FP32 partials partial[z][NCHW] for split-K (reduced by splitk_reduce.hip).
// Split-K slices follow the reference's partition rule [floor(ns*z/S), floor(ns*(z+1)/S))
// (src/kernels/tensor_core_mma.cu:112-115) over channel slices, and its partial layout (:231-234).
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <set>
#include <utility>
#include <vector>

#include "lds_pipe.h"

namespace gie_hip {
namespace {

struct HaloGeom {
  int B, S, H, W, O, SH, SW, PH, PW, OH, OW;
  int HWo, N;
  int WPAD;      // staged pixels per slot: (OW - 1) * SW + KW
  int E;         // slot gap at an image boundary: max(KH - SH, 0)
  int x_bytes, w_bytes;
  int xslice, wslice;  // bytes from one channel slice to the next in xb / wb
  int xoff, woff;      // byte offsets of xb and wb from the lower of the two (one buffer resource spans both)
  int span;            // bytes the buffer resource covers
  int relu;
  int P, lgP;   // 16-byte units per slot: 4 * WPAD rounded up to a power of two (>= 16), and its log2
  int AU;        // activation units per stage (largest tile's slots x P, whole 1 KiB blocks)
  int SU;        // units per stage: weights (TO * KH*KW * 4) then activations
  int NBA;       // 1 KiB activation blocks per stage
  float inv_ow, inv_oh, inv_hwo;  // reciprocals for the exact fast divisions below (operands < 2^22)
};

constexpr int kSlotTable = 256;   // bytes at the start of LDS: slot -> pixel offset of (b, ih, 0), or -1
constexpr int kMaxSlots = kSlotTable / 4;
constexpr int kBiasBytes = 512;   // next: the workgroup's bias values as FP32 (tile_m <= 128)
constexpr int kHead = kSlotTable + kBiasBytes;
constexpr int kCS = 32;           // channels per slice

template <int KH, int KW, int TO, int TPX, int NST>
struct HShape {
  static constexpr int RS = KH * KW;
  static constexpr int WP = TPX / 64;   // pixel-half waves
  static constexpr int WK = KH * 2;     // K groups: filter row x channel half
  static constexpr int NW = WP * WK;    // waves
  static constexpr int NT = NW * 64;
  static constexpr int FO = TO / 32;    // 32-channel MFMA blocks per wave
  static constexpr int WU = TO * RS * 4;  // weight units per stage
  static constexpr int NBW = WU / 64;      // weight blocks (1 KiB) per stage
  static constexpr int KBW = (NBW + NW - 1) / NW;  // weight loads per wave per slice
  static constexpr int ACC = 2 * FO * 4 * 64 * 16;  // bytes of one wave's FP32 tile in LDS
  static constexpr int TROW = TPX * 2 + 8;           // 16-bit output tile row pitch
  static_assert(TPX % 64 == 0 && TO % 32 == 0 && TO <= 128, "tile must be whole waves");
  static_assert(NST == 2 || NST == 3, "two or three LDS stages");
  static_assert(WU % 64 == 0, "weight region must be whole 1 KiB blocks");
};

template <typename E, int KH, int KW, int TO, int TPX, int NST, int KBA>
__global__ __launch_bounds__(TPX / 64 * KH * 2 * 64) void halo_kernel(
    const uint16_t* __restrict__ xn, const uint16_t* __restrict__ wk, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ y, float* __restrict__ partial, HaloGeom g, int split) {
  using S = HShape<KH, KW, TO, TPX, NST>;
  constexpr int RS = S::RS, NT = S::NT, NW = S::NW, FO = S::FO;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  int* slot_tab = reinterpret_cast<int*>(lds);
  float* bias_s = reinterpret_cast<float*>(lds + kSlotTable);
  unsigned char* stage0 = lds + kHead;
  const int stage_bytes = g.SU * 16;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: block choice and M0 stay scalar
  const int kg = wave % S::WK, wp = wave / S::WK;  // K group (filter row kg/2, channel half kg%2), pixel half
  const int wr = kg >> 1, wh = kg & 1;
  const int n_ot = (g.O + TO - 1) / TO;
  const int ot = int(blockIdx.x) % n_ot, pt = int(blockIdx.x) / n_ot;  // neighbours share pixels, XCDs share o
  const int o0 = ot * TO, P0 = pt * TPX;
  const int Pend = min(P0 + TPX, g.N);
  const int z = int(blockIdx.z);
  const int sl0 = int((static_cast<long long>(g.S) * z) / split);
  const int sl1 = int((static_cast<long long>(g.S) * (z + 1)) / split);
  // bias now, consumed in the epilogue: its latency hides under the main loop
  const float bias_r = (bias != nullptr && tid < TO && o0 + tid < g.O) ? E::to_f32(bias[o0 + tid]) : 0.0f;

  // one resource over both repacked tensors: xb at g.xoff, wb at g.woff from the lower address
  const v4i rsrc = make_vsharp(reinterpret_cast<const unsigned char*>(xn) - g.xoff, g.span);
  const unsigned lds_stage0 = lds_addr(stage0);
  // Stage layout: weights [0, WU) units, then activations [WU, WU + AU). A load instruction fills one 1 KiB block;
  // block j of a region is loaded by wave j % NW, surplus instructions repeat the region's last block (same
  // bytes to the same place). Each lane inverts the layout to find the global chunk of its unit, once; slices
  // then add a fixed stride. Padding lanes carry kOut, which any slice advance keeps past the resource (a slice
  // after the last sets the top bit of every offset), so the issue loop has no per-lane selects.
  auto issue = [&](const int(&off)[S::KBW > KBA ? S::KBW : KBA], const unsigned(&dst)[S::KBW > KBA ? S::KBW : KBA],
                   auto nc, int step, int sl, bool live, unsigned st) {
    const int dead = live ? 0 : kOut;
#pragma unroll
    for (int k = 0; k < decltype(nc)::value; ++k) dma16(rsrc, st + dst[k], (off[k] + sl * step) | dead);
  };
  constexpr int KM = S::KBW > KBA ? S::KBW : KBA;
  using NW_ = std::integral_constant<int, S::KBW>;
  using NA_ = std::integral_constant<int, KBA>;

  // Weight unit of (output channel o, tap t, chunk k): chunk k of row o at k ^ ((o >> 2) & 3), so the 16 lanes
  // of a fragment read (16 consecutive o, one t and k) hit distinct bank groups (rows are 4*RS units apart).
  auto w_unit = [&](int o, int t, int k) { return (o * RS + t) * 4 + (k ^ ((o >> 2) & 3)); };
  int w_off[KM], w_dst[KM];
  unsigned w_dstu[KM];
#pragma unroll
  for (int k = 0; k < S::KBW; ++k) {
    const int blk = min(wave + k * NW, S::NBW - 1);
    const int wu = blk * 64 + lane;
    const int o = wu / (RS * 4), t = (wu >> 2) - o * RS, kp = wu & 3;
    const int k8 = (kp ^ ((o >> 2) & 3)) * 8;
    w_off[k] = (o0 + o < g.O) ? g.woff + (((o0 + o) * g.S * RS + t) * 32 + k8) * 2 : kOut;
    w_dst[k] = blk * 1024;
    w_dstu[k] = unsigned(w_dst[k]);
  }
  // weights of the first slices go out before the slot table is even built
#pragma unroll
  for (int p = 0; p < NST - 1; ++p)
    issue(w_off, w_dstu, NW_{}, g.wslice, sl0 + p, sl0 + p < sl1, lds_stage0 + p * stage_bytes);

  // ---- slot table: output row j of the tile, tap row r -> slot j*SH + r + E*(image - first image) ----------
  // (every slot in [0, NS) is some (j, r) when SH <= KH; otherwise the gaps are cleared first)
  const int rf0 = fdiv(P0, g.OW, g.inv_ow), rfL = fdiv(Pend - 1, g.OW, g.inv_ow);
  const int b0 = fdiv(rf0, g.OH, g.inv_oh);
  if (g.SH > KH) {
    for (int s = tid; s < kMaxSlots; s += NT) slot_tab[s] = -1;
    __syncthreads();
  }
  for (int j = tid; j <= rfL - rf0; j += NT) {
    const int rf = rf0 + j, b = fdiv(rf, g.OH, g.inv_oh), oh = rf - b * g.OH;
    const int base = j * g.SH + g.E * (b - b0);
#pragma unroll
    for (int r = 0; r < KH; ++r) {
      const int ih = oh * g.SH - g.PH + r;
      slot_tab[base + r] = (ih >= 0 && ih < g.H) ? (b * g.S * g.H + ih) * g.W * 32 : -1;  // xb element, slice 0
    }
  }
  __syncthreads();

  // Slot j occupies activation units [j*P, (j+1)*P); pixel column c's four chunks start at (4c + d(j)) mod P
  // with d(j) = 4*j*OW mod 16, and logical chunk k of the pixel sits at k ^ ((v >> 2) & 3), v = j*OW + c. Then
  // the bank group of (j, c, k) is (4v + (k ^ ((v >> 2) & 3))) mod 16: distinct for 16 consecutive v, i.e. for
  // 16 consecutive output pixels of one tap even where they wrap from one image row to the next.
  auto act_unit = [&](int slot, int col, int k) {
    const int v = slot * g.OW + col;
    const int pos = (4 * col + ((4 * slot * g.OW) & 15)) & (g.P - 1);
    return S::WU + (slot << g.lgP) + pos + (k ^ ((v >> 2) & 3));
  };
  int a_off[KM];
  unsigned a_dstu[KM];
#pragma unroll
  for (int k = 0; k < KBA; ++k) {
    const int blk = min(wave + k * NW, g.NBA - 1);
    const int u = blk * 64 + lane;
    const int slot = u >> g.lgP, pos = (u - ((4 * slot * g.OW) & 15)) & (g.P - 1);
    const int col = pos >> 2, kp = pos & 3;
    int off = kOut;
    if (col < g.WPAD) {
      const int v = slot * g.OW + col;
      const int k8 = (kp ^ ((v >> 2) & 3)) * 8;
      const int so = slot_tab[slot], iw = col - g.PW;
      if (so >= 0 && iw >= 0 && iw < g.W) off = g.xoff + (so + iw * 32 + k8) * 2;
    }
    a_off[k] = off;
    a_dstu[k] = unsigned(S::WU * 16 + blk * 1024);
  }
#pragma unroll
  for (int p = 0; p < NST - 1; ++p)
    issue(a_off, a_dstu, NA_{}, g.xslice, sl0 + p, sl0 + p < sl1, lds_stage0 + p * stage_bytes);

  // ---- per-lane fragment addresses (bytes within a stage), fixed for the whole loop ---------------------------
  const int chunk = wh * 2 + (lane >> 5);  // which 8 channels of the slice this lane feeds
  int a_addr[KW][2];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    const int px_raw = P0 + wp * 64 + pb * 32 + (lane & 31);
    const int px = px_raw < g.N ? px_raw : P0;  // rows past N multiply a valid pixel; never stored
    const int rf = fdiv(px, g.OW, g.inv_ow), ow = px - rf * g.OW, b = fdiv(rf, g.OH, g.inv_oh);
    const int slot = (rf - rf0) * g.SH + g.E * (b - b0) + wr;  // this wave's filter row
#pragma unroll
    for (int s = 0; s < KW; ++s) a_addr[s][pb] = act_unit(slot, ow * g.SW + s, chunk) * 16;
  }
  int b_addr[KW][FO];
#pragma unroll
  for (int ob = 0; ob < FO; ++ob)
#pragma unroll
    for (int s = 0; s < KW; ++s) b_addr[s][ob] = w_unit(ob * 32 + (lane & 31), wr * KW + s, chunk) * 16;

  f32x16 acc[2][FO];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb)
#pragma unroll
    for (int ob = 0; ob < FO; ++ob) acc[pb][ob] = f32x16{};

  auto rdfrag = [&](const unsigned char* st, int s, u32x4(&af)[2], u32x4(&bf)[FO]) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) af[pb] = *reinterpret_cast<const u32x4*>(st + a_addr[s][pb]);
#pragma unroll
    for (int ob = 0; ob < FO; ++ob) bf[ob] = *reinterpret_cast<const u32x4*>(st + b_addr[s][ob]);
  };
  // One slice: every fragment of the wave's KW taps is read from LDS first (KW x (2 + FO) registers of 16 bytes),
  // then this thread's loads for a later slice are issued (they land while the multiplies run), then the
  // multiplies. With three waves per SIMD the read latency of one wave is covered by another's multiplies.
  auto slice = [&](const unsigned char* st, int sl_next, bool live_next, unsigned st_next) {
    u32x4 af[KW][2], bf[KW][FO];
#pragma unroll
    for (int s = 0; s < KW; ++s) rdfrag(st, s, af[s], bf[s]);
    __builtin_amdgcn_sched_barrier(0);  // the compiler would otherwise trade the read-ahead for registers
    issue(w_off, w_dstu, NW_{}, g.wslice, sl_next, live_next, st_next);
    issue(a_off, a_dstu, NA_{}, g.xslice, sl_next, live_next, st_next);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < KW; ++s)
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int ob = 0; ob < FO; ++ob) acc[pb][ob] = E::mfma32(af[s][pb], bf[s][ob], acc[pb][ob]);
  };

  // ---- main loop over this workgroup's channel slices ----------------------------------------------------------
  // prologue order W(s0) [W(s1)] A(s0) [A(s1)]: slice s0 has landed once at most A(s1) is outstanding
  wait_vmcnt<KBA * (NST - 2)>();  // this thread's part of the first slice has landed
  stage_barrier();               // ... and everyone's
  int cur = 0;
  for (int sl = sl0; sl < sl1; ++sl) {
    const int nxt = cur == 0 ? NST - 1 : cur - 1;  // (cur + NST - 1) % NST: the stage read one slice ago
    // loads of slice sl + NST - 1 (zeros past the last slice) while slice sl multiplies
    slice(stage0 + cur * stage_bytes, sl + NST - 1, sl + NST - 1 < sl1, lds_stage0 + nxt * stage_bytes);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<(S::KBW + KBA) * (NST - 2)>();  // the next slice's loads (issued one iteration ago) have landed
    stage_barrier();
    cur = cur + 1 == NST ? 0 : cur + 1;
  }
  wait_vmcnt<0>();  // the zero loads past the last slice still write into the stages the epilogue reuses
  __syncthreads();

  // ---- epilogue: sum the K groups of each pixel half through LDS -------------------------------------------------
  // Slot q of pixel half wp holds one wave's 64x64 FP32 tile, lane-major so every access is a whole 1 KiB row.
  // K groups NQ..2NQ-1 store, groups 0..NQ-1 add them and store the pair sums back; then every thread takes a
  // share of the tile, sums the NQ pair sums in a fixed order and applies bias + ReLU + one rounding. Reads are
  // issued as a batch before their sums so their latencies overlap.
  f32x4* red = reinterpret_cast<f32x4*>(stage0);
  constexpr int NQ = S::WK / 2;         // pair sums per pixel half (3 for 3x3, 1 for 1x1)
  constexpr int PER = 2 * FO * 4 * 64;  // f32x4 items of one wave's tile
  constexpr int ITEMS = S::WP * PER;
  constexpr int IPT = (ITEMS + NT - 1) / NT;  // items per thread in the final pass
  auto slot_idx = [&](int q, int item) {  // item = (((wp*2 + pb)*FO + ob)*4 + r4)*64 + lane
    const int wpi = item / PER;
    return (wpi * NQ + q) * PER + (item - wpi * PER);
  };
  auto my_item = [&](int pb, int ob, int r4) { return (((wp * 2 + pb) * FO + ob) * 4 + r4) * 64 + lane; };
  const int pair = kg % NQ;  // K groups kg and kg + NQ form one pair
  if (kg >= NQ) {
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int ob = 0; ob < FO; ++ob)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          red[slot_idx(pair, my_item(pb, ob, r4))] = f32x4{acc[pb][ob][4 * r4], acc[pb][ob][4 * r4 + 1],
                                                           acc[pb][ob][4 * r4 + 2], acc[pb][ob][4 * r4 + 3]};
  }
  if (tid < TO) bias_s[tid] = bias_r;
  __syncthreads();
  if (kg < NQ) {
    f32x4 v[2][FO][4];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int ob = 0; ob < FO; ++ob)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) v[pb][ob][r4] = red[slot_idx(pair, my_item(pb, ob, r4))];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int ob = 0; ob < FO; ++ob)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          red[slot_idx(pair, my_item(pb, ob, r4))] =
              f32x4{acc[pb][ob][4 * r4] + v[pb][ob][r4][0], acc[pb][ob][4 * r4 + 1] + v[pb][ob][r4][1],
                    acc[pb][ob][4 * r4 + 2] + v[pb][ob][r4][2], acc[pb][ob][4 * r4 + 3] + v[pb][ob][r4][3]};
  }
  __syncthreads();
  // item -> output: 32x32 accumulator layout, register r of lane l is row 8*(r/4) + 4*(l/32) + r%4 (pixel),
  // column l%32 (channel); an f32x4 item is 4 consecutive pixels of one output channel
  auto item_o = [&](int item) { return ((item / (4 * 64)) % FO) * 32 + (item & 31); };
  auto item_px = [&](int item) {
    const int l = item & 63, r4 = (item / 64) & 3, pbw = item / (4 * 64 * FO);  // wp*2 + pb
    return pbw * 32 + 8 * r4 + 4 * (l >> 5);
  };
  f32x4 sums[IPT];
  {
    f32x4 parts[IPT][NQ];
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      const int item = min(tid + i * NT, ITEMS - 1);
#pragma unroll
      for (int q = 0; q < NQ; ++q) parts[i][q] = red[slot_idx(q, item)];
    }
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      sums[i] = parts[i][0];
#pragma unroll
      for (int q = 1; q < NQ; ++q) sums[i] += parts[i][q];
    }
  }
  if (split > 1) {
    float* pz = partial + static_cast<long long>(z) * g.N * g.O;
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      const int item = tid + i * NT;
      if (item >= ITEMS) break;
      const f32x4 v = sums[i];
      const int o = o0 + item_o(item), px = P0 + item_px(item);
      if (o >= g.O || px >= g.N) continue;
      const int b = fdiv(px, g.HWo, g.inv_hwo), p = px - b * g.HWo;
      float* dst = pz + (static_cast<long long>(b) * g.O + o) * g.HWo + p;
      if (px + 3 < g.N && p + 3 < g.HWo && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
        *reinterpret_cast<f32x4*>(dst) = v;
      } else {
        for (int e = 0; e < 4 && px + e < g.N; ++e) {
          const int be = fdiv(px + e, g.HWo, g.inv_hwo), pe = px + e - be * g.HWo;
          pz[(static_cast<long long>(be) * g.O + o) * g.HWo + pe] = v[e];
        }
      }
    }
    return;
  }
  // 16-bit tile [TO][TPX] (row pitch TROW) past every pair-sum slot, then coalesced NCHW stores
  unsigned char* tile = stage0 + S::WP * NQ * S::ACC;
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int item = tid + i * NT;
    if (item >= ITEMS) break;
    const int ol = item_o(item);
    const float bv = bias_s[ol];
    uint32_t hv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a = sums[i][e] + bv;  // bias on the FP32 sum, then ReLU, then one rounding
      if (g.relu) a = fmaxf(a, 0.0f);
      hv[e] = E::from_f32(a);
    }
    *reinterpret_cast<u32x2*>(tile + ol * S::TROW + item_px(item) * 2) = u32x2{hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16)};
  }
  __syncthreads();
  // each storing thread keeps one 4-pixel group, so the pixel -> (image, position) division happens once
  constexpr int G4 = TPX / 4;
  constexpr int SROWS = NT / G4;                   // output channels stored per pass
  constexpr int SPT = (TO + SROWS - 1) / SROWS;    // passes
  const int q4 = tid % G4;
  const int px = P0 + 4 * q4;
  const int pb_ = px < g.N ? fdiv(px, g.HWo, g.inv_hwo) : 0, pp = px - pb_ * g.HWo;
  const bool whole = px + 3 < g.N && pp + 3 < g.HWo;
  u32x2 sv[SPT];
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const int ol = min(tid / G4 + i * SROWS, TO - 1);
    sv[i] = *reinterpret_cast<const u32x2*>(tile + ol * S::TROW + q4 * 8);
  }
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const int ol = tid / G4 + i * SROWS;
    const int o = o0 + ol;
    if (ol >= TO || o >= g.O || px >= g.N) continue;
    const u32x2 v = sv[i];
    uint16_t* dst = y + (static_cast<long long>(pb_) * g.O + o) * g.HWo + pp;
    if (whole && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
      *reinterpret_cast<u32x2*>(dst) = v;
    } else {
      const uint16_t hv[4] = {uint16_t(v[0]), uint16_t(v[0] >> 16), uint16_t(v[1]), uint16_t(v[1] >> 16)};
      for (int e = 0; e < 4 && px + e < g.N; ++e) {
        const int be = fdiv(px + e, g.HWo, g.inv_hwo), pe = px + e - be * g.HWo;
        y[(static_cast<long long>(be) * g.O + o) * g.HWo + pe] = hv[e];
      }
    }
  }
}

// ---- registered configurations ----------------------------------------------------------------------------------
typedef void (*HaloFn)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*, HaloGeom, int);

constexpr int kKbMax = 8;  // load instructions per wave per slice

struct HaloConfig {
  gie_halo_config info;
  int nst;  // LDS stages
  int acc, trow, wu, nw;
  HaloFn fn[2][kKbMax + 1];  // [fp16, bf16][load instructions per wave per slice]
};

template <typename E, int KH, int KW, int TO, int TPX, int NST, int... KBs>
void fill_fns(HaloFn* out, std::integer_sequence<int, KBs...>) {
  ((out[KBs + 1] = &halo_kernel<E, KH, KW, TO, TPX, NST, KBs + 1>), ...);
}

template <int KH, int KW, int TO, int TPX, int NST>
HaloConfig make_halo(int version) {
  using S = HShape<KH, KW, TO, TPX, NST>;
  HaloConfig c;
  c.info.tile_m = TO;
  c.info.tile_n = TPX;
  c.info.tile_k = kCS;
  c.info.kernel_h = KH;
  c.info.kernel_w = KW;
  c.info.threads = S::NT;
  c.info.stages = NST;
  c.info.version = version;
  c.nst = NST;
  c.acc = S::ACC;
  c.trow = S::TROW;
  c.wu = S::WU;
  c.nw = S::NW;
  c.fn[0][0] = c.fn[1][0] = nullptr;
  fill_fns<Fp16, KH, KW, TO, TPX, NST>(c.fn[0], std::make_integer_sequence<int, kKbMax>{});
  fill_fns<Bf16, KH, KW, TO, TPX, NST>(c.fn[1], std::make_integer_sequence<int, kKbMax>{});
  return c;
}

const std::vector<HaloConfig>& halo_configs() {
  static const std::vector<HaloConfig> t = [] {
    std::vector<HaloConfig> v;
    //                KH KW  TO  TPX NST
    v.push_back(make_halo<3, 3, 64, 128, 3>(3));
    v.push_back(make_halo<3, 3, 64, 128, 2>(3));
    v.push_back(make_halo<1, 1, 64, 128, 3>(3));
    v.push_back(make_halo<1, 1, 128, 128, 3>(3));
    return v;
  }();
  return t;
}

// Geometry checks shared by the capability query and the launch. Fills g, the LDS bytes and the number of
// load instructions per wave per slice on success.
int halo_prepare(const HaloConfig& c, const gie_conv_geom* gg, HaloGeom* g, int* lds_bytes, int* kb) {
  if (!gg) return GIE_HIP_EINVAL;
  if (gg->kernel_h != c.info.kernel_h || gg->kernel_w != c.info.kernel_w) return GIE_HIP_EUNSUPPORTED;
  g->B = gg->batch;
  g->S = (gg->in_channels + kCS - 1) / kCS;
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
  if (g->B <= 0 || gg->in_channels <= 0 || g->H <= 0 || g->W <= 0 || g->O <= 0 || g->SH <= 0 || g->SW <= 0 ||
      g->PH < 0 || g->PW < 0 || g->OH <= 0 || g->OW <= 0)
    return GIE_HIP_EINVAL;
  const int KH = c.info.kernel_h, KW = c.info.kernel_w, TPX = c.info.tile_n;
  const long long hwo = static_cast<long long>(g->OH) * g->OW;
  const long long n = hwo * g->B;
  const long long xs = static_cast<long long>(g->H) * g->W * 64, ws = static_cast<long long>(KH) * KW * 64;
  const long long xb = xs * g->S * g->B, wb = ws * g->S * g->O;
  if (n > 0x7fffffffLL || xb >= 0x7fffffffLL || wb >= 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  g->HWo = int(hwo);
  g->N = int(n);
  g->x_bytes = int(xb);
  g->w_bytes = int(wb);
  g->xslice = int(xs);
  g->wslice = int(ws);
  g->WPAD = (g->OW - 1) * g->SW + KW;
  g->E = KH > g->SH ? KH - g->SH : 0;
  // slots of the largest tile: rows it spans, taps per row, image boundaries it crosses
  const long long rows = std::min<long long>(static_cast<long long>(g->OH) * g->B, (TPX - 1) / g->OW + 2);
  const long long bounds = std::min<long long>(g->B - 1, (TPX - 1) / hwo + 1);
  const long long ns = (rows - 1) * g->SH + KH + g->E * bounds;
  if (ns > kMaxSlots) return GIE_HIP_EUNSUPPORTED;
  int lgp = 4;
  while ((1LL << lgp) < 4LL * g->WPAD) ++lgp;
  const long long p = 1LL << lgp;
  const long long au = (ns * p + 63) / 64 * 64;  // whole 1 KiB blocks
  const long long su = au + c.wu;
  if (su * 16 * c.nst > kLdsLimit) return GIE_HIP_EUNSUPPORTED;
  g->P = int(p);
  g->lgP = lgp;
  g->AU = int(au);
  g->SU = int(su);
  g->NBA = int(au / 64);
  const int k = (g->NBA + c.nw - 1) / c.nw;
  if (k > kKbMax) return GIE_HIP_EUNSUPPORTED;
  if (g->N >= (1 << 22)) return GIE_HIP_EUNSUPPORTED;  // exact fast divisions need pixel indices below 2^22
  g->inv_ow = 1.0f / float(g->OW);
  g->inv_oh = 1.0f / float(g->OH);
  g->inv_hwo = 1.0f / float(g->HWo);
  const int wp = c.info.tile_n / 64;
  const long long epi = static_cast<long long>(wp) * c.info.kernel_h * c.acc + c.info.tile_m * c.trow;
  const long long lds = kHead + std::max(c.nst * su * 16, epi);
  if (lds > kLdsLimit) return GIE_HIP_EUNSUPPORTED;
  *lds_bytes = int(lds);
  *kb = k;
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
  int lds = 0, kb = 0;
  const int rc = halo_prepare(halo_configs()[size_t(config)], g, &hg, &lds, &kb);
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
  int lds = 0, kb = 0;
  if (int rc = halo_prepare(c, gg, &g, &lds, &kb)) return rc;
  if (split > g.S) return GIE_HIP_EUNSUPPORTED;
  const long long n_ot = (g.O + c.info.tile_m - 1) / c.info.tile_m;
  const long long n_pt = (static_cast<long long>(g.N) + c.info.tile_n - 1) / c.info.tile_n;
  if (n_ot * n_pt > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  // one buffer resource spans both tensors: offsets from the lower address, all below 2^31
  const uintptr_t xa = reinterpret_cast<uintptr_t>(xn), wa = reinterpret_cast<uintptr_t>(wk);
  const uintptr_t lo = xa < wa ? xa : wa;
  const unsigned long long span = std::max<unsigned long long>(xa - lo + g.x_bytes, wa - lo + g.w_bytes);
  if (span >= 0x7fffffffULL) return GIE_HIP_EUNSUPPORTED;
  g.xoff = int(xa - lo);
  g.woff = int(wa - lo);
  g.span = int(span);
  HaloFn fn = c.fn[dtype == GIE_HIP_BF16 ? 1 : 0][kb];
  if (!fn) return GIE_HIP_EUNSUPPORTED;
  if (int rc = set_lds_limit(reinterpret_cast<const void*>(fn), lds)) return rc;
  hipLaunchKernelGGL(fn, dim3(unsigned(n_ot * n_pt), 1, unsigned(split)), dim3(c.info.threads), lds,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(xn),
                     static_cast<const uint16_t*>(wk), static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y),
                     partial, g, split);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
