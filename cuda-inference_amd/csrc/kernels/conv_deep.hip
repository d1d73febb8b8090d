// Deep convolution: 3x3, stride 1, padding 1 over small images (in_h <= 8, in_w <= 7) with a long reduction
// (in_channels % 128 == 0), straight from the caller's NCHW x and OIHW w on gfx950 matrix cores
// (v_mfma_f32_16x16x32_{f16,bf16}, FP32 accumulation). One launch, no workspace, no split-K: the whole reduction of an
// output tile runs inside one workgroup.
//
// Unit: (16-filter block, image), one 8-wave workgroup per unit, one unit per CU (config 5: 32 filter blocks x 8
// images = 256 units). Waves 0-3 multiply, waves 4-7 load.
//   * Output tile: 16 filters x 64 positions, the image's rows at pitch 8 (8 rows x 8 columns; column 7 and rows past
//     in_h are padding, dropped at the store) = 4 MFMA blocks of 16 positions (two rows each).
//   * Reduction: C / 32 channel slices in steps of four. Multiplying wave w takes slice 4t + w of step t, so each wave
//     sums a quarter of the reduction over the whole tile; the four partial tiles are added in LDS at the end, in wave
//     order (deterministic), then bias + ReLU + one rounding (the reference's apply_epilogue order,
//     src/kernels/fused_epilogue.cuh:11-16).
//   * Operands (the slab kernel's scheme): A = weights, one lane holding 8 channels of one tap of one filter, taken from
//     its 144-byte OIHW run (8 channels x 9 taps) by 36 v_perm per slice; B = pixels, read from LDS planes with
//     ds_read_b64_tr_b16 (4 channels x 16 positions per 16-lane group, each lane receiving the 4 channels of its
//     position). The three taps of a filter row read the same B fragment; the column shift is done on three
//     accumulator sets by DPP row shifts in the epilogue (acc_s[o] = sum_r W[r][s] . X[o + 8r], y[o] = acc_0[o - 1] +
//     acc_1[o] + acc_2[o + 1]). Column 7 of every plane row holds zeros, which is the left padding of column 0 and
//     the right padding of column in_w - 1, so the shifts need no mask.
//   * LDS planes: per channel 16 granules of 16 bytes; plane row q (input row q - 1, rows 0 and in_h + 1 .. 9 zero) at
//     granule q ^ 2 tau(ch), tau(ch) = (ch & 3) | ((ch >> 3 & 1) << 2) over the channel's index in its slice: the
//     8 channels and 2 rows a 32-lane half of a transposing read touches land in 16 distinct granules, i.e. 64
//     distinct banks. A 16-position window (block j, filter row r) is plane rows 2j + r and 2j + r + 1.
//   * Loader waves: per step, the four slices' weight runs by direct-to-LDS 16-byte loads (each filter's 576-byte run
//     of a slice plus a 16-byte pad, so a lane's 144-byte read of 16 filters spreads over the banks), and the four
//     slices' activation rows by one 16-byte register load per (channel, row) from the 4-byte boundary at or below the
//     row start (rows of 7 halves start at any 2-byte boundary), shifted into place with v_alignbit, masked to the
//     row's columns and written as one 16-byte granule. Two stages: step t + 2 loads into the stage step t read from.
//     One barrier per step joins the multiplying waves (done reading the stage the loaders refill next) and the
//     loaders (the next step's data in LDS).
#include <algorithm>
#include <utility>

#include "slab_common.h"

namespace gie_hip {
namespace {

constexpr int kDpTO = 16;                     // filters per unit
constexpr int kDpP = 8;                       // row pitch (positions)
constexpr int kDpNB = 4;                      // MFMA blocks of 16 positions (8 rows)
constexpr int kDpCS = 32;                     // channels per slice
constexpr int kDpQ = 4;                       // slices per step (one per multiplying wave)
constexpr int kDpRows = 10;                   // plane rows read: input rows -1 .. 8
constexpr int kDpChP = 256;                   // bytes per channel plane: 16 granules of 16
constexpr int kDpAct = kDpQ * kDpCS * kDpChP;  // activation stage: 128 channels = 32 KiB
constexpr int kDpRun = 576 + 16;              // weight run of one filter and slice, plus pad
constexpr int kDpWq = kDpTO * kDpRun;         // one slice's weights
constexpr int kDpWch = kDpQ * kDpWq / 16;     // 16-byte chunks of a step's weights (37 per run)
constexpr int kDpKW = (kDpWch + 255) / 256;   // weight loads per loader lane and step (10)
constexpr int kDpKWh = kDpKW / 2;             // from step 2 on, a loader issues the first kDpKWh, its partner the rest
constexpr int kDpWst = kDpKW * 4 * 1024;      // weight stage: every load block of the four loaders (40 KiB)
constexpr int kDpWOff = 2 * kDpAct;
constexpr int kDpXOff = kDpWOff + 2 * kDpWst;  // partial-tile exchange: 4 waves x 4 blocks x 64 lanes x 16 bytes
constexpr int kDpLds = kDpXOff + kDpQ * kDpNB * 64 * 16;
constexpr int kDpNT = 512;
static_assert(kDpLds <= kLdsLimit, "LDS budget");
static_assert(kDpAct < 65536 && kDpWst < 65536, "stage offsets fit the LDS offset field");

struct DeepGeom {
  int B, C, H, W, O, HW;
  int NS;               // steps: C / 128
  int n_units, per_xcd;
  int x_bytes, w_bytes;
  int relu;
  int total;            // |Y| elements
  int items;            // activation (channel, row) items per step: 128 * H
  unsigned h_magic;     // e / H = (e * h_magic) >> 16 for e < 1024 (h_magic = ceil(2^16 / H))
  unsigned keep[4];     // dword masks keeping a row's W columns
};

// (e * ceil(2^16 / H)) >> 16 == e / H for every H in 1 .. 8 and e < 1024: the product exceeds e * 2^16 / H by at most
// e (H - 1) / H < 1024 * 7 / 8, which stays below 2^16 / H, the distance from e / H to the next integer.
constexpr bool deep_magic_exact() {
  for (unsigned h = 1; h <= 8; ++h)
    for (unsigned e = 0; e < 1024; ++e)
      if (((e * ((65536u + h - 1) / h)) >> 16) != e / h) return false;
  return true;
}
static_assert(deep_magic_exact(), "division by in_h through a multiplier");

// The weight chunk c of a step (c < 2560) splits into slice q = c / 592 and r = c % 592, and r into filter
// f = r / 37 and piece k = r % 37, through multipliers: the products stay below 2^24, so they are 24-bit multiplies.
constexpr bool deep_chunk_magic_exact() {
  for (unsigned c = 0; c < 2560; ++c)
    if (((c * 7085u) >> 22) != c / 592) return false;
  for (unsigned r = 0; r < 592; ++r)
    if (((r * 1772u) >> 16) != r / 37) return false;
  return true;
}
static_assert(deep_chunk_magic_exact(), "chunk decomposition through multipliers");
static_assert(kDpRun == 37 * 16 && kDpWq == 592 * 16 && kDpKW * 256 <= 2560, "chunk decomposition constants");

// v if ok, else the out-of-range offset, with bit operations (a conditional would become an exec-mask branch)
__device__ __forceinline__ unsigned deep_sel(bool ok, unsigned v) {
  const unsigned m = 0u - unsigned(ok);
  return (v & m) | (unsigned(kOut) & ~m);
}

__device__ __forceinline__ int deep_tau(int ch) { return (ch & 3) | (((ch >> 3) & 1) << 2); }
// byte offset of (channel plane, plane row) inside an activation stage; ch is the channel's index in the stage (the
// swizzle uses its index in its slice)
__device__ __forceinline__ int deep_granule(int ch, int row) {
  return ch * kDpChP + ((row ^ (2 * deep_tau(ch & 31))) << 4);
}

// Every kernel argument the set-up reads, requested before the first branch (one round trip to the argument
// segment instead of one per basic block).
__device__ __forceinline__ void deep_args(const void* x, const void* w, const void* bias, const void* y,
                                          const DeepGeom& g) {
  asm volatile("" ::"s"(x), "s"(w), "s"(bias), "s"(y));
  asm volatile("" ::"s"(g.B), "s"(g.C), "s"(g.H), "s"(g.W), "s"(g.O), "s"(g.HW), "s"(g.NS), "s"(g.n_units),
               "s"(g.per_xcd), "s"(g.x_bytes), "s"(g.w_bytes), "s"(g.relu), "s"(g.total), "s"(g.items));
}

// Slot plan of a step (36 MFMAs: tap-major, 4 blocks per tap). The weight fragments are one set: this slice's taps
// 5-8 are transposed in slots 0-7 (their last use in the previous slice was in the previous step, their first use
// here is slot 20), then the next slice's weight runs are read over the same registers (slots 8-16) and its taps 0-4
// transposed in slots 20-35, after their last use here (slot 19). The next slice's 18 pixel-fragment reads fill
// slots 9-34.
struct DeepSched {
  static constexpr int NM = 9 * kDpNB;
  static constexpr int TL = 5;
  static constexpr int early_slot(int p) { return p / 2; }                // p < 16: taps TL .. 8
  static constexpr int wread_slot(int q) { return 8 + q; }               // q < 9
  static constexpr int bread_slot(int q) { return 9 + q * 25 / 18; }     // q < 18
  static constexpr int late_slot(int p) { return 20 + p * 16 / 20; }      // p < 20: taps 0 .. TL-1
};
static_assert(DeepSched::early_slot(4 * (9 - DeepSched::TL) - 1) < DeepSched::wread_slot(0),
              "early transposes read the runs before they are reloaded");
static_assert(DeepSched::late_slot(0) >= kDpNB * DeepSched::TL, "late transposes follow the last use of tap TL - 1");
static_assert(DeepSched::bread_slot(17) < DeepSched::NM && DeepSched::late_slot(4 * DeepSched::TL - 1) < DeepSched::NM,
              "slot plan");

// Offsets of the weight chunks share lw (0..3) of a step issues: chunk c = (4 kb + lw) * 64 + lane is slice q,
// filter f, 16-byte piece k of the run (k = 36 is the pad, never read); out-of-range chunks get kOut.
__device__ __forceinline__ void deep_w_offsets(int lw, int lane, int o0, const DeepGeom& g, int (&w_voff)[kDpKW]) {
  const unsigned wrow = unsigned(g.C) * 18u;  // < 2^24 (deep_prepare)
  const unsigned cb = unsigned(lw * 64 + lane);
#pragma unroll
  for (int kb = 0; kb < kDpKW; ++kb) {
    const unsigned c = cb + 256u * unsigned(kb);
    const unsigned q = __umul24(c, 7085u) >> 22, r = c - __umul24(q, 592u);
    const unsigned f = __umul24(r, 1772u) >> 16, k = r - __umul24(f, 37u);
    const bool ok = (c < unsigned(kDpWch)) & (k < 36u) & (o0 + int(f) < g.O);
    w_voff[kb] = int(deep_sel(ok, __umul24(unsigned(o0) + f, wrow) + __umul24(q, 576u) + 16u * k));
  }
}

// Step t's share lw of the weights into stage st by direct-to-LDS loads: load blocks KB0 .. KB1-1 of the share (past
// the last step they go through a zero-length resource).
template <int KB0 = 0, int KB1 = kDpKW>
__device__ __forceinline__ void deep_load_w(const uint16_t* w, const DeepGeom& g, unsigned lds0, int lw,
                                            const int (&w_voff)[kDpKW], int t, int st) {
  const bool real = t < g.NS;
  const v4i ws = make_vsharp(w, real ? g.w_bytes : 0);
  const int ws_off = real ? t * kDpQ * 576 : 0;
#pragma unroll
  for (int kb = KB0; kb < KB1; ++kb)
    dma16s(ws, lds0 + unsigned(kDpWOff + st * kDpWst + (kb * 4 + lw) * 1024), w_voff[kb], ws_off);
}

template <typename E>
__global__ __launch_bounds__(kDpNT, 1) void deep_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w,
                                                      const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                      DeepGeom g) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  deep_args(x, w, bias, y, g);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slot = int(blockIdx.x);
  const int unit = (slot >> 3) + (slot & 7) * g.per_xcd;  // XCD x takes a contiguous range: few filter blocks, every image
  if (unit >= g.n_units) return;
  const int fblk = unit / g.B, b = unit - fblk * g.B;
  const int o0 = fblk * kDpTO;
  const unsigned lds0 = lds_addr(lds);

  if (wave >= 4) {
    // ====================== loader wave lw = wave - 4 (lt = its thread index among the loaders) ======================
    const int lw = wave - 4, lt = tid - 256;
    const v4i xr = make_vsharp(x, g.x_bytes);
    const v4i x0 = make_vsharp(x, 0);  // every offset out of range: zeros, no traffic
    int w_voff[kDpKW];
    deep_w_offsets(lw, lane, o0, g, w_voff);
    const int a_step = kDpQ * kDpCS * g.HW * 2;
    deep_load_w<0, kDpKWh>(w, g, lds0, lw, w_voff, 0, 0);  // the first loads leave before any other set-up work
    __builtin_amdgcn_sched_barrier(0);
    // activation item e = k * 256 + lt: (channel ch of the step's 128, row r); the row's W halves start at element
    // (b * C + ch) * HW + r * W; the load starts at the 4-byte boundary at or below it
    constexpr int KA = (kDpQ * kDpCS * 8 + 255) / 256;  // up to 8 rows per channel
    const int x_img = b * g.C * g.HW;                    // first element of the image (uniform)
    int a_voff[KA];
    uint32_t a_sh[KA];
    unsigned a_dst[KA];
    bool a_ok[KA];
#pragma unroll
    for (int k = 0; k < KA; ++k) {
      const int e = k * 256 + lt;
      a_ok[k] = e < g.items;
      const int ee = a_ok[k] ? e : 0;
      const int ch = int(__umul24(unsigned(ee), g.h_magic) >> 16), r = ee - ch * g.H;
      const int elem = x_img + int(__umul24(unsigned(ch), unsigned(g.HW)) + __umul24(unsigned(r), unsigned(g.W)));
      a_voff[k] = a_ok[k] ? ((elem * 2) & ~3) : kOut;
      a_sh[k] = uint32_t(elem & 1) << 4;
      a_dst[k] = lds0 + unsigned(deep_granule(ch, r + 1));
    }
    u32x4 ra[KA], rb[KA];
    // step t's activation rows into registers (write_rows puts them in LDS)
    auto load_a = [&](int t, u32x4 (&rr)[KA]) __attribute__((always_inline)) {
      const bool real = t < g.NS;
      const v4i xs = real ? xr : x0;
      const int as = real ? t * a_step : 0;
#pragma unroll
      for (int k = 0; k < KA; ++k) rr[k] = load16s(xs, a_voff[k], as);
    };
    // steps 2 and later: this loader issues load blocks 0 .. kDpKWh-1 of its weight share, multiplying wave lw the rest
    auto load_step = [&](int t, int st, u32x4 (&rr)[KA]) __attribute__((always_inline)) {
      deep_load_w<0, kDpKWh>(w, g, lds0, lw, w_voff, t, st);
      load_a(t, rr);
    };
    auto write_rows = [&](int st, u32x4 (&rr)[KA]) __attribute__((always_inline)) {
#pragma unroll
      for (int k = 0; k < KA; ++k) {
        touch_v(rr[k]);
        const u32x4 v = rr[k];
        const uint32_t sh = a_sh[k];
        const u32x4 o = {__builtin_amdgcn_alignbit(v.y, v.x, sh) & g.keep[0],
                         __builtin_amdgcn_alignbit(v.z, v.y, sh) & g.keep[1],
                         __builtin_amdgcn_alignbit(v.w, v.z, sh) & g.keep[2],
                         __builtin_amdgcn_alignbit(0u, v.w, sh) & g.keep[3]};
        if (a_ok[k]) wr16(a_dst[k] + unsigned(st * kDpAct), o);
      }
    };
    load_a(0, ra);
    load_a(1, rb);  // step 1's weights: the multiplying waves issue them (eight waves load the first two stages)
    // zero the plane rows no load writes (row 0 and rows in_h + 1 .. 9) of both stages, once: loader thread lt
    // takes channel lt % 128 of stage lt / 128
    {
      const unsigned zbase = lds0 + unsigned((lt >> 7) * kDpAct);
      const int zch = lt & 127;
      for (int z = 0; z < kDpRows - g.H; ++z)
        wr16(zbase + unsigned(deep_granule(zch, z == 0 ? 0 : g.H + z)), u32x4{0u, 0u, 0u, 0u});
    }
    wait_vmcnt<KA>();  // step 0's loads (step 1's activation rows may be in flight)
    write_rows(0, ra);
    stage_barrier();  // B0: step 0 in LDS
    wait_vmcnt<0>();
    write_rows(1, rb);
    stage_barrier();  // start of step 0: step 1 in LDS
    for (int t = 0; t + 1 < g.NS; ++t) {
      // step t: the multiplying waves read step t + 1's stage; step t's stage (read during step t - 1) takes t + 2
      if (t + 2 < g.NS) {
        load_step(t + 2, t & 1, ra);
        wait_vmcnt<0>();
        write_rows(t & 1, ra);
      }
      stage_barrier();
    }
    stage_barrier();  // the partial-tile exchange of the multiplying waves
    return;
  }

  // ====================== multiplying wave w: slices 4t + w ======================
  // First, load blocks kDpKWh .. kDpKW-1 of step 0's weight share w and all of step 1's (the loaders issue every
  // other load of the first two stages); from step 2 on this wave issues load blocks kDpKWh .. kDpKW-1 of that share:
  // more waves with loads in flight move a step's bytes from L2 faster
  int w_voff[kDpKW];
  deep_w_offsets(wave, lane, o0, g, w_voff);
  deep_load_w<kDpKWh, kDpKW>(w, g, lds0, wave, w_voff, 0, 0);  // the second half of step 0's share
  deep_load_w(w, g, lds0, wave, w_voff, 1, 1);
  using Sc = DeepSched;
  constexpr int NM = Sc::NM, TL = Sc::TL;
  const int wv = wave;
  const int f0 = o0 + 4 * (lane >> 4);  // the lane's first filter
  uint32_t bbits[4];
  {
    const v4i br = make_vsharp(bias, bias != nullptr ? 2 * g.O : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) bbits[i] = load2s(br, 2 * min(f0 + i, g.O - 1), 0);
  }
  const unsigned a_rd = lds0 + unsigned(kDpWOff + wv * kDpWq + (lane & 15) * kDpRun + (lane >> 4) * 144);
  unsigned b_rd[9][2];
#pragma unroll
  for (int R = 0; R < 9; ++R) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ch = 8 * (lane >> 4) + 4 * h + ((lane & 15) >> 2), q = lane & 3;
      b_rd[R][h] = lds0 + unsigned(deep_granule(wv * kDpCS + ch, R + (q >> 1)) + (q & 1) * 8);
    }
  }
  f32x4 acc[3][kDpNB];
#pragma unroll
  for (int s2 = 0; s2 < 3; ++s2) {
#pragma unroll
    for (int j2 = 0; j2 < kDpNB; ++j2) acc[s2][j2] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  u32x4 fw[9], fb[2][9];
  uint32_t d[36];
  auto read_w = [&](auto qc, auto st_c) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value, ST = decltype(st_c)::value;
    const u32x4 v = rd16(a_rd + unsigned(ST * kDpWst + 16 * q));
    d[4 * q] = v.x, d[4 * q + 1] = v.y, d[4 * q + 2] = v.z, d[4 * q + 3] = v.w;
  };
  auto read_b = [&](auto qc, auto st_c, auto set_c) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value, ST = decltype(st_c)::value, S = decltype(set_c)::value;
    constexpr int R = q / 2, h = q % 2;
    const u32x2 v = rd_tr(b_rd[R][h] + unsigned(ST * kDpAct));
    fb[S][R][2 * h] = v.x;
    fb[S][R][2 * h + 1] = v.y;
  };
  // transpose p of tap t = p / 4: dword p % 4 of the tap's weight fragment (8 channels of one tap per lane)
  auto perm_tap = [&](auto pc) __attribute__((always_inline)) {
    constexpr int p = decltype(pc)::value, t = p / 4, c = p % 4;
    fw[t][c] = pick2(d, 18 * c + t, 18 * c + 9 + t);
  };
  auto mfma_one = [&](auto kc, auto set_c) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value, S = decltype(set_c)::value;
    constexpr int t = k / kDpNB, j = k % kDpNB, r = t / 3, sc = t % 3;
    acc[sc][j] = E::mfma(fw[t], fb[S][2 * j + r], acc[sc][j]);
  };
  using I0 = std::integral_constant<int, 0>;

  wait_vmcnt<kDpKW + 4>();  // this wave's half of step 0's weights (step 1's and the 4 bias loads may be in flight)
  stage_barrier();  // B0: step 0 in LDS
  // step 0's slice into registers: its weight runs, its pixel fragments (set 0), the transposes of taps 0 .. TL-1
  for_seq([&](auto qc) __attribute__((always_inline)) { read_w(qc, I0{}); }, std::make_integer_sequence<int, 9>{});
  for_seq([&](auto qc) __attribute__((always_inline)) { read_b(qc, I0{}, I0{}); },
          std::make_integer_sequence<int, 18>{});
  for_seq([&](auto pc) __attribute__((always_inline)) { perm_tap(pc); }, std::make_integer_sequence<int, 4 * TL>{});

  // step t (u = t mod 2): slice 4t + w multiplies from pixel set u; step t + 1's slice is read from stage 1 - u
  auto step = [&](int tt, auto u_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(u_c)::value, nxt = cur ^ 1;
    using STn = std::integral_constant<int, nxt>;
    wait_vmcnt<0>();  // this wave's loads into step t + 1's stage (and the bias loads, long landed)
    stage_barrier();  // step t + 1 is in LDS; every wave is done with step t - 1 (and with step t's stage)
    __builtin_amdgcn_sched_barrier(0);
    // step t's stage is free: this wave's part of step t + 2's weights
    if (tt + 2 < g.NS) deep_load_w<kDpKWh, kDpKW>(w, g, lds0, wv, w_voff, tt + 2, cur);
    __builtin_amdgcn_sched_barrier(0);
    for_seq([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      mfma_one(kc, std::integral_constant<int, cur>{});
      for_seq([&](auto pc) __attribute__((always_inline)) {
        constexpr int p = decltype(pc)::value;
        if constexpr (Sc::early_slot(p) == k) perm_tap(std::integral_constant<int, 4 * TL + p>{});
      }, std::make_integer_sequence<int, 4 * (9 - TL)>{});
      for_seq([&](auto qc) __attribute__((always_inline)) {
        if constexpr (Sc::wread_slot(decltype(qc)::value) == k) read_w(qc, STn{});
      }, std::make_integer_sequence<int, 9>{});
      for_seq([&](auto qc) __attribute__((always_inline)) {
        if constexpr (Sc::bread_slot(decltype(qc)::value) == k) read_b(qc, STn{}, STn{});
      }, std::make_integer_sequence<int, 18>{});
      for_seq([&](auto pc) __attribute__((always_inline)) {
        if constexpr (Sc::late_slot(decltype(pc)::value) == k) perm_tap(pc);
      }, std::make_integer_sequence<int, 4 * TL>{});
      __builtin_amdgcn_sched_barrier(0);
    }, std::make_integer_sequence<int, NM>{});
  };
  for (int t = 0; t < g.NS; t += 2) {
    step(t, I0{});
    if (t + 1 < g.NS) step(t + 1, std::integral_constant<int, 1>{});
  }

  // ---- epilogue: tap-column shifts, the four partial tiles added in LDS in wave order, bias + ReLU + one rounding --
  const unsigned xch = lds0 + unsigned(kDpXOff) + unsigned(lane * 16);
#pragma unroll
  for (int j = 0; j < kDpNB; ++j) {
    const f32x4 out = acc[1][j] + dpp4<kShr1>(acc[0][j]) + dpp4<kShl1>(acc[2][j]);
    wr16(xch + unsigned((wv * kDpNB + j) * 1024), __builtin_bit_cast(u32x4, out));
  }
  wait_vmcnt<0>();  // the bias loads
  stage_barrier();
  // this wave finishes block j = w: output rows 2w and 2w + 1
  f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int v = 0; v < 4; ++v) sum += __builtin_bit_cast(f32x4, rd16(xch + unsigned((v * kDpNB + wv) * 1024)));
  const int pos = 16 * wv + (lane & 15), row = pos >> 3, col = pos & 7;
  const bool pv = row < g.H && col < g.W;
  const v4i yr = make_vsharp(y, g.total * 2);
  const int e0 = (b * g.O + f0) * g.HW + row * g.W + col;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    touch_v(bbits[i]);
    float v = sum[i] + (bias != nullptr ? E::to_f32(uint16_t(bbits[i])) : 0.0f);
    if (g.relu) v = fmaxf(v, 0.0f);
    store2(yr, pv && f0 + i < g.O ? (e0 + i * g.HW) * 2 : kOut, E::from_f32(v));
  }
}

typedef void (*DeepFn)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, DeepGeom);

int deep_prepare(const gie_conv_geom* gg, DeepGeom* g) {
  if (!gg) return GIE_HIP_EINVAL;
  if (gg->kernel_h != 3 || gg->kernel_w != 3 || gg->stride_h != 1 || gg->stride_w != 1 || gg->pad_h != 1 ||
      gg->pad_w != 1)
    return GIE_HIP_EUNSUPPORTED;
  if (gg->batch <= 0 || gg->in_channels <= 0 || gg->out_channels <= 0 || gg->in_h <= 0 || gg->in_w <= 0)
    return GIE_HIP_EINVAL;
  if (gg->in_h > 2 * kDpNB || gg->in_w > kDpP - 1) return GIE_HIP_EUNSUPPORTED;  // the tile and its zero column
  if (gg->in_channels % (kDpQ * kDpCS) != 0) return GIE_HIP_EUNSUPPORTED;        // whole steps of four slices
  const long long hw = 1LL * gg->in_h * gg->in_w;
  const long long xb = 2LL * gg->batch * gg->in_channels * hw, wb = 18LL * gg->out_channels * gg->in_channels;
  const long long total = 1LL * gg->batch * gg->out_channels * hw;
  if (xb >= (1LL << 30) || wb >= (1LL << 30) || total >= (1LL << 29)) return GIE_HIP_EUNSUPPORTED;
  if (18LL * gg->in_channels >= (1LL << 24)) return GIE_HIP_EUNSUPPORTED;  // a filter's OIHW row: 24-bit multiplies
  const long long units = 1LL * gg->batch * ((gg->out_channels + kDpTO - 1) / kDpTO);
  if (units > (1LL << 24)) return GIE_HIP_EUNSUPPORTED;
  g->B = gg->batch, g->C = gg->in_channels, g->H = gg->in_h, g->W = gg->in_w, g->O = gg->out_channels;
  g->HW = int(hw);
  g->NS = gg->in_channels / (kDpQ * kDpCS);
  g->n_units = int(units);
  g->per_xcd = (g->n_units + 7) / 8;
  g->x_bytes = int(xb), g->w_bytes = int(wb);
  g->relu = gg->relu;
  g->total = int(total);
  g->items = kDpQ * kDpCS * gg->in_h;
  g->h_magic = (65536u + unsigned(gg->in_h) - 1) / unsigned(gg->in_h);
  for (int i = 0; i < 4; ++i) {
    const int lo = 2 * i, hi = 2 * i + 1;  // columns of dword i
    g->keep[i] = (lo < gg->in_w ? 0xffffu : 0u) | (hi < gg->in_w ? 0xffff0000u : 0u);
  }
  return GIE_HIP_OK;
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_deep_check(const gie_conv_geom* g, int* lds_bytes) {
  DeepGeom dg{};
  if (int rc = deep_prepare(g, &dg)) return rc;
  if (lds_bytes) *lds_bytes = kDpLds;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_conv_deep(int dtype, const gie_conv_geom* gg, const void* x, const void* w, const void* bias,
                                 void* y, void* stream) {
  if (!gg || !x || !w || !y) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(y) & 1u) || (bias && (reinterpret_cast<uintptr_t>(bias) & 1u)))
    return GIE_HIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(x) & 3u) || (reinterpret_cast<uintptr_t>(w) & 15u)) return GIE_HIP_EUNSUPPORTED;
  DeepGeom g{};
  if (int rc = deep_prepare(gg, &g)) return rc;
  const DeepFn fn = dtype == GIE_HIP_BF16 ? &deep_kernel<Bf16> : &deep_kernel<Fp16>;
  if (int rc = set_lds_limit(reinterpret_cast<const void*>(fn), kDpLds)) return rc;
  hipLaunchKernelGGL(fn, dim3(unsigned(8 * g.per_xcd)), dim3(kDpNT), kDpLds, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                     static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
