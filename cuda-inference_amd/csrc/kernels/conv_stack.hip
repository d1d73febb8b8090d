// Stacked-image convolution: 3x3 filter, stride 1, padding 1, for layers whose images are small and whose reduction
// is long (in_w + 1 <= 8, in_channels % 32 == 0; the 8 x 512 x 7 x 7 layer of the benchmark set), straight from NCHW x
// and OIHW w on gfx950 matrix cores (v_mfma_f32_16x16x32_{f16,bf16}, FP32 accumulation). One launch, plus the split-K
// reduce when split > 1; no repack of either operand.
//
// A workgroup (a "unit") owns 32 output channels x a group of NI images x one range of 32-channel slices. In LDS the
// NI images are stacked into one tall plane per channel: P positions per row (columns >= in_w are zero padding), a
// zero row above the first image and one zero row after every image (the bottom padding of that image and the top
// padding of the next). Stack row t (LDS row t + 1) is image t / (H+1), row t % (H+1); rows with t % (H+1) == H are
// the zero separators. A 3x3 convolution of the whole stack is then every image's own convolution, and output stack
// rows k with k % (H+1) == H are computed and dropped. So a long-reduction layer over small images becomes a few tall
// units with every weight of a (filter block, channel range) read by a handful of workgroups, instead of one
// workgroup per image re-reading all the weights.
//
// Operands and MFMA core follow the slab kernel (conv_slab.hip): the pixel operand of tap row r is one 16-position
// read at o + r*P for all three tap columns (ds_read_b64_tr_b16 from the [channel][position] plane), the tap column
// enters through three accumulator sets shifted by DPP lane moves in the epilogue,
//     acc_s[o] = sum_r W[r][s] . X[o + r*P],     y[o] = acc_0[o - 1] + acc_1[o] + acc_2[o + 1],
// and each lane's weights are its filter's 144-byte OIHW run (8 channels x 9 taps), transposed in registers (v_perm).
//
// Loads per slice: the weights by 16-byte direct-to-LDS loads (each filter's 576-byte run of the slice, the order
// OIHW stores it); the activations by 16-byte register loads, one per (channel, image row): an image row of in_w <= 7
// halves starts at any 2-byte boundary, so the load starts at the 4-byte boundary at or below it, and one v_perm per
// dword both shifts the row into place and zeroes the padding columns before a 16-byte LDS write.
//
// Waves: 4 = (filter half fh: 16 filters) x (row half wr: RW = 16 * NBW / P stack rows = NBW position blocks), one per
// SIMD. Two LDS stages; step j multiplies slice j while slice j + 1's fragments are read and transposed into the other
// register set, slice j + 2's activations (loaded during step j - 1) are written into the stage slice j left, slice
// j + 3's activations load into registers and slice j + 2's weights load into LDS: one MFMA per issue slot with the
// side work between them (the slab kernel's pipelined schedule), one wait and one barrier per step.
//
// Epilogue: the DPP shift-add of the three accumulator sets, then split 1: bias + ReLU + one RNE rounding (the
// reference's apply_epilogue order, src/kernels/fused_epilogue.cuh:11-16) and 2-byte stores; split > 1: FP32 partials
// partial[z][NCHW] over the z-th range of channel slices [floor(S*z/split), floor(S*(z+1)/split)), the partition of
// src/kernels/tensor_core_mma.cu:112-115, reduced by splitk_reduce.hip.
// Grid: unit = (z * n_ob + ob) * n_ig + ig; XCD x (slot mod 8) takes a contiguous range of units, so an XCD's L2 holds
// one or two channel ranges: their weights for every filter block and their activations for every image group.
#include <algorithm>
#include <cmath>

#include "slab_common.h"

namespace gie_hip {
namespace {

constexpr int kStTO = 32;  // output channels per workgroup

struct StackGeom {
  int B, C, H, W, O, HW;
  int S;                  // 32-channel slices
  int NI;                 // images per unit
  int n_ig, n_ob, n_units, per_xcd;
  int x_bytes, w_bytes;
  int relu, split;
  int total;              // |Y| elements (partial stride)
  int items;              // (channel, image row) pairs of one slice of a unit: 32 * NI * H
  int nz;                 // LDS rows per channel no item writes (zero rows): NR - NI * H
  unsigned mg_ig, mg_ob, mg_nih, mg_h, mg_nz;  // n / d = (umulhi(n, mg) + n) >> sh for n < 2^30
  int sh_ig, sh_ob, sh_nih, sh_h, sh_nz;       // divisors: n_ig, n_ob, NI * H, H, nz
  uint32_t keep[4];       // per dword of a row: the halves of columns < W
};

__device__ __forceinline__ void args_in_sgprs(const void* x, const void* w, const void* bias, const void* y,
                                              const void* partial, const StackGeom& g) {
  asm volatile("" ::"s"(x), "s"(w), "s"(bias), "s"(y), "s"(partial));
  asm volatile("" ::"s"(g.n_units), "s"(g.per_xcd), "s"(g.n_ig), "s"(g.n_ob), "s"(g.mg_ig), "s"(g.mg_ob),
               "s"(g.sh_ig), "s"(g.sh_ob), "s"(g.S), "s"(g.split), "s"(g.NI), "s"(g.items), "s"(g.nz));
  asm volatile("" ::"s"(g.C), "s"(g.H), "s"(g.W), "s"(g.HW), "s"(g.O), "s"(g.B), "s"(g.x_bytes), "s"(g.w_bytes),
               "s"(g.relu), "s"(g.total), "s"(g.mg_nih), "s"(g.sh_nih), "s"(g.mg_h), "s"(g.sh_h), "s"(g.mg_nz),
               "s"(g.sh_nz));
}



template <int P, int NBW, int KH>
struct StackShape {
  static constexpr int RW = 16 * NBW / P;               // stack rows per wave
  static constexpr int RB = 2 * RW;                     // stack rows per unit
  static constexpr int NR = RB + 2;                     // LDS rows per channel
  static constexpr int NBR = (16 * (NBW - 1) + 2 * P) / P + 1;  // pixel-fragment reads per slice (P apart)
  static constexpr int CS = 32;                         // channels per slice (one MFMA k-step)
  static constexpr int NW = 4, NT = 256;
  static constexpr int WCH = CS * 18 / 16;              // 16-byte chunks of one filter's slice run
  static constexpr int CPF = WCH + 1;                   // + one pad chunk (bank spread)
  static constexpr int WPITCH = CPF * 16;
  static constexpr int WBLK = (kStTO * CPF + 63) / 64;  // 1 KiB load blocks holding data per slice
  static constexpr int KBW = (WBLK + NW - 1) / NW;      // weight blocks per wave (the blocks past WBLK load zeros)
  static constexpr int WST = KBW * NW * 1024;
  // channel ch's plane starts at ch * CHP + 32 * swz(ch): the 8 channels one half-wave reads start in 8 distinct
  // 32-byte bank groups, and a position's address is linear in the position
  static constexpr int CHP = (NR * P * 2 + 224 + 255) / 256 * 256;
  static constexpr int ACT = CS * CHP;
  static constexpr int KR = (CS * RB + NT - 1) / NT;    // activation rows (items) per thread per slice
  static constexpr int LDSH = 2 * (ACT + WST);          // one channel half: [2 activation stages][2 weight stages]
  static constexpr int LDS = KH * LDSH;
  static_assert(KH == 1 || KH == 2, "one or two channel halves");
  static_assert(KH == 1 || 4 * 64 * 3 * NBW * 16 <= LDSH, "a half's accumulators fit its LDS for the combine");
  static_assert(P == 8, "rows of one 16-byte chunk (in_w <= 7), 16-position blocks of whole rows");
  static_assert((16 * NBW) % P == 0, "a wave's rows are whole 16-position blocks");
  static_assert(ACT + 16 * NBR < 65536 && WST + 256 < 65536, "stage offsets fit the LDS offset field");
  static_assert(LDS <= kLdsLimit, "LDS budget");
};

__device__ __forceinline__ unsigned plane_of(int ch, int chp) { return unsigned(ch * chp + 32 * seg_swz(ch)); }

// compile-time placement of one step's side work behind its 9 * NBW MFMAs: fragment reads first (the weight runs,
// then the pixel halves), transposes after the weight runs, activation writes in the first half and the next
// register loads (into the same registers) after them, weight loads spread over the step
template <int P, int NBW>
struct StackSched {
  using Sh = StackShape<P, NBW, 1>;
  static constexpr int NM = 9 * NBW;
  static constexpr int NRD = 9 + 2 * Sh::NBR;
  static constexpr int NRS = NRD < NM ? NRD : NM;
  static constexpr int PB = 9 < NM - 1 ? 9 : NM - 1;
  static constexpr int NA = Sh::KR;
  static constexpr int rd_slot(int q) { return q * NRS / NRD; }
  static constexpr int perm_slot(int p) { return PB + p * (NM - PB) / 36; }
  static constexpr int awr_slot(int a) { return a * (NM / 2) / NA; }
  static constexpr int ald_slot(int a) { return NM / 2 + a * (NM - NM / 2) / NA; }
  static constexpr int wld_slot(int q) { return q * NM / Sh::KBW; }
};

template <typename E, int P, int NBW, int KH>
__global__ __launch_bounds__(256 * KH, 1) void stack_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                      const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                      float* __restrict__ partial, StackGeom g) {
  using Sh = StackShape<P, NBW, KH>;
  using Sc = StackSched<P, NBW>;
  constexpr int CS = Sh::CS, NW = Sh::NW, NT = Sh::NT, RW = Sh::RW, NBR = Sh::NBR;
  constexpr int CPF = Sh::CPF, WCH = Sh::WCH, WPITCH = Sh::WPITCH, KBW = Sh::KBW, WST = Sh::WST, CHP = Sh::CHP;
  constexpr int ACT = Sh::ACT, KR = Sh::KR;
  constexpr int WOFF = 2 * ACT;  // LDS: [2 activation stages][2 weight stages]
  constexpr int NM = Sc::NM, NRD = Sc::NRD;
  static_assert(3 * (KBW + KR) + 4 < 64, "loads in flight fit the vmcnt counter");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  args_in_sgprs(x, w, bias, y, partial, g);

  // KH channel halves of 4 waves each: half h multiplies its share of the unit's slices in its own LDS stages, and
  // the halves' accumulators are added through LDS before the epilogue
  const int tid = threadIdx.x & 255, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) & 3);
  const int half = KH == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 8);
  const int fh = wave & 1, wr = wave >> 1;

  // ---- unit: XCD (slot mod 8) takes units [xcd * per_xcd, ...) ----
  const int slot = int(blockIdx.x);
  const int unit = (slot >> 3) + (slot & 7) * g.per_xcd;
  if (unit >= g.n_units) return;  // workgroup-uniform
  const int q0 = magic_div(unit, g.mg_ig, g.sh_ig), ig = unit - q0 * g.n_ig;
  const int z = magic_div(q0, g.mg_ob, g.sh_ob), ob = q0 - z * g.n_ob;
  const int o0 = ob * kStTO, b0 = ig * g.NI;
  int s_beg = 0, nsu = g.S;  // the unit's slices
  if (g.split > 1) {
    s_beg = (g.S * z) / g.split;
    nsu = (g.S * (z + 1)) / g.split - s_beg;
  }
  // this half's slices: [s_beg + half * nsh, ...), ns of them real; every half runs nsh steps (the barriers are shared)
  const int nsh = KH == 1 ? nsu : (nsu + 1) >> 1;
  const int ns = KH == 1 ? nsu : max(0, min(nsh, nsu - half * nsh));
  s_beg += half * nsh;

  const v4i xr = make_vsharp(x, g.x_bytes), wrs = make_vsharp(w, g.w_bytes);
  const v4i x0 = make_vsharp(x, 0), w0 = make_vsharp(w, 0);  // every offset out of range: loads give zeros
  const unsigned lds0 = lds_addr(lds) + unsigned(half * Sh::LDSH);

  // ---- load offsets first, so the first loads leave before the rest of the set-up ----
  // weights: block wave + NW * kb; lane slot u = (filter u / CPF, chunk u % CPF); per slice += CS * 18
  int w_voff[KBW];
  const int wrow = g.C * 18;
#pragma unroll
  for (int kb = 0; kb < KBW; ++kb) {
    const int u = (wave + NW * kb) * 64 + lane, f = u / CPF, k = u - f * CPF;
    const int val = (o0 + f) * wrow + 16 * k;
    const bool ok = (f < kStTO) & (k < WCH) & (o0 + f < g.O);
    w_voff[kb] = ok ? val : kOut;
  }
  // activation items: e = k * NT + tid < items is (channel ch, image i, row ih) of the slice, whose W halves start at
  // element ((b0 + i) * C + ch) * HW + ih * W; the load starts at the 4-byte boundary at or below it
  int a_voff[KR], a_ch[KR], a_row[KR];
  uint32_t a_sh[KR];  // 16 when the row starts 2 bytes past the load's start, else 0
#pragma unroll
  for (int k = 0; k < KR; ++k) {
    const int e = k * NT + tid;
    const bool ok = e < g.items;
    const int ee = ok ? e : 0;
    const int ch = magic_div(ee, g.mg_nih, g.sh_nih), rem = ee - ch * g.NI * g.H;
    const int i = magic_div(rem, g.mg_h, g.sh_h), ih = rem - i * g.H;
    const int elem = ((b0 + i) * g.C + ch) * g.HW + ih * g.W;
    a_voff[k] = (ok && b0 + i < g.B) ? ((elem * 2) & ~3) : kOut;
    a_sh[k] = uint32_t(elem & 1) << 4;
    // an item past the last one loads zeros (offset kOut) and writes them over the zero row above channel 0
    a_ch[k] = ok ? ch : 0;
    a_row[k] = ok ? i * (g.H + 1) + ih + 1 : 0;
  }
  const int hw2 = g.HW * 2;
  const int a_soff0 = s_beg * CS * hw2;  // + slice * CS * hw2
  const int w_soff0 = s_beg * CS * 18;   // + slice * CS * 18

  struct SliceArgs {
    v4i xs, ws;
    int a_soff, w_soff;
  };
  // slices past the last load through zero-length resources (zeros, no memory traffic) into stages no later step
  // multiplies, so every step issues the same loads and the slot schedule has no branches
  auto slice_args = [&](int s) __attribute__((always_inline)) {
    const bool real = s < ns;
    return SliceArgs{real ? xr : x0, real ? wrs : w0, real ? a_soff0 + s * CS * hw2 : 0,
                     real ? w_soff0 + s * CS * 18 : 0};
  };
  u32x4 ra[KR];  // activation rows of the next slice to write
  auto aload = [&](auto kc, const SliceArgs& sa) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    ra[k] = load16s(sa.xs, a_voff[k], sa.a_soff);
  };
  auto wload = [&](auto kc, auto st_c, const SliceArgs& sa) __attribute__((always_inline)) {
    constexpr int kb = decltype(kc)::value, ST = decltype(st_c)::value;
    dma16s(sa.ws, lds0 + unsigned(WOFF + ST * WST + (wave + NW * kb) * 1024), w_voff[kb], sa.w_soff);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  // ---- prologue loads: activations of slices 0 and 1 (slice 1's into registers of the prologue only), weights of
  // slices 0 and 1 into both stages; bias ----
  u32x4 rb[KR];
  {
    const SliceArgs s0 = slice_args(0), s1 = slice_args(1);
    for_seq([&](auto kc) __attribute__((always_inline)) { aload(kc, s0); }, std::make_integer_sequence<int, KR>{});
    for_seq([&](auto kc) __attribute__((always_inline)) { wload(kc, I0{}, s0); }, std::make_integer_sequence<int, KBW>{});
    for_seq([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      rb[k] = load16s(s1.xs, a_voff[k], s1.a_soff);
    }, std::make_integer_sequence<int, KR>{});
    for_seq([&](auto kc) __attribute__((always_inline)) { wload(kc, I1{}, s1); }, std::make_integer_sequence<int, KBW>{});
  }
  const int f0 = o0 + fh * 16 + 4 * (lane >> 4);  // the lane's first filter
  uint32_t bbits[4];
  {
    const v4i br = make_vsharp(bias, g.split == 1 && bias != nullptr ? 2 * g.O : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) bbits[i] = load2s(br, 2 * min(f0 + i, g.O - 1), 0);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- the rest of the set-up while they travel ----
  unsigned a_dst[KR];
#pragma unroll
  for (int k = 0; k < KR; ++k) a_dst[k] = lds0 + plane_of(a_ch[k], CHP) + unsigned(a_row[k] * P * 2);
  // zero rows of both stages (the row above the stack, the separators, rows past the last image): row z of a
  // channel's nz is 0 (z = 0), z * (H + 1) (1 <= z <= NI), NI * (H + 1) + z - NI (z > NI)
  for (int r = tid; r < 2 * CS * g.nz; r += NT) {
    const int sc = magic_div(r, g.mg_nz, g.sh_nz), zr = r - sc * g.nz;
    const int st = sc >= CS ? 1 : 0, ch = sc - st * CS;
    const int q = zr <= g.NI ? zr * (g.H + 1) : g.NI * (g.H + 1) + zr - g.NI;
    wr16(lds0 + unsigned(st * ACT) + plane_of(ch, CHP) + unsigned(q * P * 2), u32x4{0u, 0u, 0u, 0u});
  }
  // a row's 4 dwords: shifted down by a_sh bits (the first element into place), columns >= W cleared
  auto awrite = [&](auto kc, auto st_c) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value, ST = decltype(st_c)::value;
    const u32x4 v = ra[k];
    const u32x4 o = {__builtin_amdgcn_alignbit(v.y, v.x, a_sh[k]) & g.keep[0],
                     __builtin_amdgcn_alignbit(v.z, v.y, a_sh[k]) & g.keep[1],
                     __builtin_amdgcn_alignbit(v.w, v.z, a_sh[k]) & g.keep[2],
                     __builtin_amdgcn_alignbit(0u, v.w, a_sh[k]) & g.keep[3]};
    wr16(a_dst[k] + unsigned(ST * ACT), o);
  };
  auto touch_ra = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < KR; ++k) touch_v(ra[k]);
  };

  // ---- slices 0 and 1 written into both stages, slice 2's activations into registers ----
  wait_vmcnt<0>();
  touch_ra();
#pragma unroll
  for (int k = 0; k < KR; ++k) touch_v(rb[k]);
  for_seq([&](auto kc) __attribute__((always_inline)) { awrite(kc, I0{}); }, std::make_integer_sequence<int, KR>{});
#pragma unroll
  for (int k = 0; k < KR; ++k) ra[k] = rb[k];
  for_seq([&](auto kc) __attribute__((always_inline)) { awrite(kc, I1{}); }, std::make_integer_sequence<int, KR>{});
  {
    const SliceArgs s2 = slice_args(2);
    for_seq([&](auto kc) __attribute__((always_inline)) { aload(kc, s2); }, std::make_integer_sequence<int, KR>{});
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- fragment addresses: A = the lane's 144-byte weight run; B = pixel block u (P positions apart) of the lane's
  // channel quad h: read q of a slice is at b_rd[h] + 16 * u (+ the stage) ----
  const unsigned a_rd = lds0 + unsigned(WOFF + (fh * 16 + (lane & 15)) * WPITCH + 8 * (lane >> 4) * 18);
  unsigned b_rd[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int ch = 8 * (lane >> 4) + 4 * h + ((lane & 15) >> 2);
    b_rd[h] = lds0 + plane_of(ch, CHP) + unsigned(2 * (wr * RW * P + 4 * (lane & 3)));
  }

  f32x4 acc[3][NBW];
#pragma unroll
  for (int s2 = 0; s2 < 3; ++s2) {
#pragma unroll
    for (int j2 = 0; j2 < NBW; ++j2) acc[s2][j2] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  u32x4 fw[2][9], fb[2][NBR];
  uint32_t d[36];
  auto read_one = [&](auto qc, auto st_c, auto set_c) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value, ST = decltype(st_c)::value, S = decltype(set_c)::value;
    if constexpr (q < 9) {
      const u32x4 v = rd16(a_rd + unsigned(ST * WST + 16 * q));
      d[4 * q] = v.x, d[4 * q + 1] = v.y, d[4 * q + 2] = v.z, d[4 * q + 3] = v.w;
    } else {
      constexpr int u = (q - 9) / 2, h = (q - 9) % 2;
      const u32x2 v = rd_tr(b_rd[h] + unsigned(ST * ACT + 2 * P * u));
      fb[S][u][2 * h] = v.x;
      fb[S][u][2 * h + 1] = v.y;
    }
  };
  auto perm_one = [&](auto pc, auto set_c) __attribute__((always_inline)) {
    constexpr int p = decltype(pc)::value, S = decltype(set_c)::value, t = p / 4, c = p % 4;
    fw[S][t][c] = pick2(d, 18 * c + t, 18 * c + 9 + t);
  };
  auto mfma_one = [&](auto kc, auto set_c) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value, S = decltype(set_c)::value;
    constexpr int t = k / NBW, j = k % NBW, r = t / 3, sc = t % 3;
    acc[sc][j] = E::mfma(fw[S][t], fb[S][(16 * j + r * P) / P], acc[sc][j]);
  };

  // ---- slice 0's fragments into set 0 ----
  stage_barrier();  // slices 0 and 1 are in both stages for every wave
  for_seq([&](auto qc) __attribute__((always_inline)) { read_one(qc, I0{}, I0{}); },
          std::make_integer_sequence<int, NRD>{});
  for_seq([&](auto pc) __attribute__((always_inline)) { perm_one(pc, I0{}); }, std::make_integer_sequence<int, 36>{});

  // ---- step j (parity u = j & 1): multiply slice j from set u; read slice j + 1 (stages u ^ 1) into set u ^ 1;
  // write slice j + 2's activations (in registers since step j - 1) into activation stage u, then load slice j + 3's
  // into the same registers; load slice j + 2's weights into weight stage u ----
  auto step = [&](int j, auto u_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(u_c)::value, nxt = cur ^ 1;
    using Cur = std::integral_constant<int, cur>;
    using Nxt = std::integral_constant<int, nxt>;
    wait_vmcnt<0>();  // this wave's loads issued in step j - 1 (or the prologue) have landed
    touch_ra();
    stage_barrier();  // ... every wave's, and every wave has read slice j's fragments and written slice j + 1
    const SliceArgs sa2 = slice_args(j + 2), sa3 = slice_args(j + 3);
    __builtin_amdgcn_sched_barrier(0);
    for_seq([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      mfma_one(kc, Cur{});
      for_seq([&](auto qc) __attribute__((always_inline)) {
        if constexpr (Sc::rd_slot(decltype(qc)::value) == k) read_one(qc, Nxt{}, Nxt{});
      }, std::make_integer_sequence<int, NRD>{});
      for_seq([&](auto pc) __attribute__((always_inline)) {
        if constexpr (Sc::perm_slot(decltype(pc)::value) == k) perm_one(pc, Nxt{});
      }, std::make_integer_sequence<int, 36>{});
      for_seq([&](auto ac) __attribute__((always_inline)) {
        if constexpr (Sc::awr_slot(decltype(ac)::value) == k) awrite(ac, Cur{});
      }, std::make_integer_sequence<int, KR>{});
      for_seq([&](auto ac) __attribute__((always_inline)) {
        if constexpr (Sc::ald_slot(decltype(ac)::value) == k) aload(ac, sa3);
      }, std::make_integer_sequence<int, KR>{});
      for_seq([&](auto qc) __attribute__((always_inline)) {
        if constexpr (Sc::wld_slot(decltype(qc)::value) == k) wload(qc, Cur{}, sa2);
      }, std::make_integer_sequence<int, KBW>{});
      __builtin_amdgcn_sched_barrier(0);
    }, std::make_integer_sequence<int, NM>{});
  };
  for (int j = 0; j < nsh; j += 2) {
    step(j, I0{});
    if (j + 1 < nsh) step(j + 1, I1{});
  }
  // The last step's activation loads are never written anywhere, but the hardware still writes their registers when
  // the data arrives. The compiler sees an inline-assembly load as writing its registers at issue, so without the
  // touch below it would treat them as free after the loop and place epilogue values there ahead of this wait,
  // where the late data would overwrite them.
  wait_vmcnt<0>();  // the loads of slices past the last one (never used) and the bias loads
  touch_ra();
#pragma unroll
  for (int i = 0; i < 4; ++i) touch_v(bbits[i]);
  if constexpr (KH == 2) {
    // half 1's accumulators through its own LDS (every wave has finished reading it: barrier), added by half 0 in a
    // fixed order (half 0 + half 1), so the result is the same launch to launch
    stage_barrier();
    const unsigned cb = lds0 - unsigned(half * Sh::LDSH) + unsigned(Sh::LDSH) + unsigned((wave * 3 * NBW * 64 + lane) * 16);
    if (half == 1) {
#pragma unroll
      for (int s2 = 0; s2 < 3; ++s2) {
#pragma unroll
        for (int j2 = 0; j2 < NBW; ++j2)
          wr16(cb + unsigned((s2 * NBW + j2) * 64 * 16), __builtin_bit_cast(u32x4, acc[s2][j2]));
      }
    }
    stage_barrier();
    if (half == 1) return;
#pragma unroll
    for (int s2 = 0; s2 < 3; ++s2) {
#pragma unroll
      for (int j2 = 0; j2 < NBW; ++j2) acc[s2][j2] += __builtin_bit_cast(f32x4, rd16(cb + unsigned((s2 * NBW + j2) * 64 * 16)));
    }
  }

  // ---- epilogue: tap-column shifts, then FP32 partials (split > 1) or bias + ReLU + one rounding; positions outside
  // an image (padding columns, separator rows, images past the batch) and filters past O store to kOut (dropped).
  // A 16-position block is two whole rows (P = 8): the neighbour a shift brings in from outside the block is a padding
  // column, whose accumulators are zero, so no term crosses blocks. ----
  auto column = [&](int j) __attribute__((always_inline)) {
    return acc[1][j] + dpp4<kShr1>(acc[0][j]) + dpp4<kShl1>(acc[2][j]);
  };
  const int nf = g.O - f0;  // filters of the lane's four that exist (>= 4: all)
  const int col = lane & 7;
  // stack row of block j is k0 + 2j: image i, row oh (oh < H + 1), tracked as j advances (H + 1 >= 2)
  int i_img = 0, oh = wr * RW + ((lane & 15) >> 3);
  while (oh > g.H) {
    oh -= g.H + 1;
    ++i_img;
  }
  auto element = [&](bool* valid) __attribute__((always_inline)) {
    *valid = (col < g.W) & (oh < g.H) & (i_img < g.NI) & (b0 + i_img < g.B);
    return ((b0 + i_img) * g.O + f0) * g.HW + oh * g.W + col;
  };
  auto advance = [&]() __attribute__((always_inline)) {
    oh += 2;
    if (oh > g.H) {
      oh -= g.H + 1;
      ++i_img;
    }
  };
  if (g.split > 1) {
    const v4i pr = make_vsharp(partial + static_cast<long long>(z) * g.total, g.total * 4);
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const f32x4 out = column(j);
      bool valid;
      const int e = element(&valid);
#pragma unroll
      for (int i = 0; i < 4; ++i) store4(pr, valid && i < nf ? (e + i * g.HW) * 4 : kOut, __float_as_uint(out[i]));
      advance();
    }
    return;
  }
  float bv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bv[i] = E::to_f32(uint16_t(bbits[i]));
  const v4i yr = make_vsharp(y, g.total * 2);
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const f32x4 out = column(j);
    bool valid;
    const int e = element(&valid);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = out[i] + bv[i];
      store2(yr, valid && i < nf ? (e + i * g.HW) * 2 : kOut, E::from_f32(g.relu ? fmaxf(v, 0.0f) : v));
    }
    advance();
  }
}

// (16-position blocks per wave); pitch 8 for rows of up to 7 pixels
struct StackCfg {
  int P, NBW, KH;  // KH: channel halves per workgroup (4 waves each)
};
constexpr StackCfg kStackCfgs[] = {{8, 8, 1}, {8, 4, 1}, {8, 2, 1}, {8, 4, 2}, {8, 2, 2}};
constexpr int kStackN = int(sizeof(kStackCfgs) / sizeof(kStackCfgs[0]));

typedef void (*StackFn)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*, StackGeom);

template <int I>
struct StCfgT {
  static constexpr int P = kStackCfgs[I].P, NBW = kStackCfgs[I].NBW, KH = kStackCfgs[I].KH;
  using Sh = StackShape<P, NBW, KH>;
};

struct StackShapeInfo {
  int P, RB, NT, LDS, KH;
  StackFn fp16, bf16;
};

template <int I>
StackShapeInfo stack_shape_of() {
  using C = StCfgT<I>;
  return StackShapeInfo{C::P, C::Sh::RB, C::Sh::NT * C::KH, C::Sh::LDS, C::KH, &stack_kernel<Fp16, C::P, C::NBW, C::KH>,
                        &stack_kernel<Bf16, C::P, C::NBW, C::KH>};
}

template <int... Is>
StackShapeInfo stack_info(int cfg, std::integer_sequence<int, Is...>) {
  StackShapeInfo si{};
  ((cfg == Is ? void(si = stack_shape_of<Is>()) : void()), ...);
  return si;
}

struct StackPlan {
  StackGeom g;
  StackFn fn;
  int nt, lds;
};

// n / d for n < 2^30: l = ceil(log2 d), mg = floor(2^32 (2^l - d) / d) + 1, q = (umulhi(n, mg) + n) >> l
void magic(int d, unsigned* mg, int* sh) {
  int l = 0;
  while ((1LL << l) < d) ++l;
  *sh = l;
  *mg = unsigned((((1ULL << l) - unsigned(d)) << 32) / unsigned(d) + 1);
}

int stack_prepare(int cfg, const gie_conv_geom* gg, int dtype, int split, StackPlan* sp) {
  if (cfg < 0 || cfg >= kStackN || !gg) return GIE_HIP_EINVAL;
  if (gg->kernel_h != 3 || gg->kernel_w != 3 || gg->stride_h != 1 || gg->stride_w != 1 || gg->pad_h != 1 ||
      gg->pad_w != 1)
    return GIE_HIP_EUNSUPPORTED;
  if (gg->batch <= 0 || gg->in_channels <= 0 || gg->out_channels <= 0 || gg->in_h <= 0 || gg->in_w <= 0)
    return GIE_HIP_EINVAL;
  if (gg->in_channels % 32 != 0) return GIE_HIP_EUNSUPPORTED;  // whole 32-channel slices
  const StackShapeInfo si = stack_info(cfg, std::make_integer_sequence<int, kStackN>{});
  if (gg->in_w + 1 > si.P || gg->in_h + 1 > si.RB) return GIE_HIP_EUNSUPPORTED;
  const long long hw = 1LL * gg->in_h * gg->in_w;
  const long long xb = 2LL * gg->batch * gg->in_channels * hw;
  const long long wb = 18LL * gg->out_channels * gg->in_channels;
  const long long total = 1LL * gg->batch * gg->out_channels * hw;
  if (xb >= (1LL << 30) || wb >= (1LL << 30) || total >= (1LL << 29)) return GIE_HIP_EUNSUPPORTED;
  const int S = gg->in_channels / 32;
  if (split < 1 || split > S) return GIE_HIP_EINVAL;
  StackGeom& g = sp->g;
  g.B = gg->batch, g.C = gg->in_channels, g.H = gg->in_h, g.W = gg->in_w, g.O = gg->out_channels, g.HW = int(hw);
  g.S = S;
  g.NI = std::min(si.RB / (g.H + 1), g.B);
  g.n_ig = (g.B + g.NI - 1) / g.NI;
  g.n_ob = (g.O + kStTO - 1) / kStTO;
  const long long units = 1LL * split * g.n_ob * g.n_ig;
  if (units > (1LL << 30)) return GIE_HIP_EUNSUPPORTED;
  g.n_units = int(units);
  g.per_xcd = (g.n_units + 7) / 8;
  g.x_bytes = int(xb), g.w_bytes = int(wb);
  g.relu = gg->relu;
  g.split = split;
  g.total = int(total);
  g.items = 32 * g.NI * g.H;
  g.nz = si.RB + 2 - g.NI * g.H;
  magic(g.n_ig, &g.mg_ig, &g.sh_ig);
  magic(g.n_ob, &g.mg_ob, &g.sh_ob);
  magic(g.NI * g.H, &g.mg_nih, &g.sh_nih);
  magic(g.H, &g.mg_h, &g.sh_h);
  magic(g.nz, &g.mg_nz, &g.sh_nz);
  // dword d of a row holds columns 2d (low half) and 2d + 1 (high half)
  for (int d = 0; d < 4; ++d) g.keep[d] = (2 * d < g.W ? 0x0000ffffu : 0u) | (2 * d + 1 < g.W ? 0xffff0000u : 0u);
  sp->fn = dtype == GIE_HIP_BF16 ? si.bf16 : si.fp16;
  sp->nt = si.NT;
  sp->lds = si.LDS;
  return GIE_HIP_OK;
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_stack_config_count(void) { return kStackN; }

extern "C" int gie_hip_stack_config_get(int index, gie_stack_config* out) {
  if (index < 0 || index >= kStackN || !out) return GIE_HIP_EINVAL;
  const StackShapeInfo si = stack_info(index, std::make_integer_sequence<int, kStackN>{});
  out->tile_m = kStTO;
  out->rows = si.RB;
  out->pitch = si.P;
  out->tile_k = 32;
  out->threads = si.NT;
  out->lds_bytes = si.LDS;
  out->halves = si.KH;
  out->version = 2;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_stack_check(int config, const gie_conv_geom* g, int* lds_bytes, int* images_per_unit) {
  StackPlan sp;
  if (int rc = stack_prepare(config, g, GIE_HIP_FP16, 1, &sp)) return rc;
  if (lds_bytes) *lds_bytes = sp.lds;
  if (images_per_unit) *images_per_unit = sp.g.NI;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_conv_stack(int config, int dtype, const gie_conv_geom* gg, const void* x, const void* w,
                                  const void* bias, void* y, float* partial, int split, void* stream) {
  if (!gg || !x || !w) return GIE_HIP_EINVAL;
  if (split > 1 ? partial == nullptr : y == nullptr) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if ((bias && (reinterpret_cast<uintptr_t>(bias) & 1u)) || (y && (reinterpret_cast<uintptr_t>(y) & 1u)) ||
      (partial && (reinterpret_cast<uintptr_t>(partial) & 3u)))
    return GIE_HIP_EINVAL;
  // 16-byte weight chunks need a 16-byte aligned w; the 4-byte-aligned row loads need a 4-byte aligned x
  if ((reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(x) & 3u)) return GIE_HIP_EUNSUPPORTED;
  StackPlan sp;
  if (int rc = stack_prepare(config, gg, dtype, split, &sp)) return rc;
  if (int rc = set_lds_limit(reinterpret_cast<const void*>(sp.fn), sp.lds)) return rc;
  hipLaunchKernelGGL(sp.fn, dim3(unsigned(8 * sp.g.per_xcd)), dim3(unsigned(sp.nt)), sp.lds,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x),
                     static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y),
                     partial, sp.g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
