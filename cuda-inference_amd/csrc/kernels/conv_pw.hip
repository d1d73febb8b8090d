// Pointwise convolution (1x1 filter, stride 1, no padding) straight from NCHW on gfx950 matrix cores
// (v_mfma_f32_32x32x16_{f16,bf16}, FP32 accumulation): no repack of either operand.
//
// Per image the convolution is the GEMM Y[b] (O x HW) = W (O x C) * X[b] (C x HW). A workgroup owns 128 output
// channels x 128 consecutive pixels of one image and walks C in slices of 32 channels:
//   * W[o][c] (OIHW with a 1x1 filter) is already K-contiguous: each filter's 32 channels of the slice are four
//     16-byte chunks, stored [filter][4 chunks] with chunk c at slot c ^ ((o >> 2) & 3);
//   * X[b][c][p0 .. p0+127] is one 256-byte run per channel, stored [channel][128 pixels] with the 32-byte blocks
//     of row r XOR-swizzled by 2*(r & 3); the MFMA operand that needs 8 channels of one pixel per lane is read
//     with ds_read_b64_tr_b16 (the gfx950 transpose read: a 16-lane group reads a 4-channel x 16-pixel block
//     and each lane receives 4 channels of its pixel).
// Both operands travel by direct-to-LDS buffer loads (16 blocks of 1 KiB per slice, 4 per wave), four stages,
// three slices in flight. GEMM roles: M = pixels (the transposed X), N = output channels (W), so each lane's
// accumulators hold 4 consecutive pixels of one output channel. 4 waves, each a 64-pixel x 64-channel tile
// (2 x 2 blocks of 32x32, four independent accumulator chains). LDS is 64 KiB, so two workgroups share a CU
// and their load and multiply phases interleave.
// Epilogue: bias + ReLU on the FP32 sums, one RNE rounding (the order of the reference's apply_epilogue,
// src/kernels/fused_epilogue.cuh:11-16), the 16-bit tile staged in LDS and written as whole 256-byte rows of Y.
// Grid: the 8 consecutive workgroup slots of one XCD (blockIdx mod 8) take the output-channel blocks of one
// pixel tile one after another, so each X tile is fetched into that XCD's L2 once.
#include <algorithm>
#include <vector>

#include "lds_pipe.h"

namespace gie_hip {
namespace {

constexpr int kPwTO = 128;  // output channels per workgroup
constexpr int kPwTP = 128;  // pixels per workgroup
constexpr int kPwKC = 32;   // channels per slice
constexpr int kPwNST = 4;   // load stages
constexpr int kPwNW = 4;    // waves
constexpr int kPwNT = kPwNW * 64;
constexpr int kPwWBytes = kPwTO * kPwKC * 2;   // 8 KiB of weights per stage
constexpr int kPwXBytes = kPwKC * kPwTP * 2;   // 8 KiB of activations per stage
constexpr int kPwSB = kPwWBytes + kPwXBytes;   // 16 KiB per stage
constexpr int kPwKL = kPwSB / 1024 / kPwNW;    // load blocks per wave per slice
constexpr int kPwRow = kPwTP * 2 + 16;         // epilogue tile row pitch (bytes)
constexpr int kPwLds = kPwNST * kPwSB;         // 64 KiB
static_assert(kPwTO * kPwRow <= kPwLds, "the epilogue tile reuses the stages");

struct PwGeom {
  int B, C, HW, O, S;
  int n_ptile;  // pixel tiles per image
  int n_tiles;  // pixel tiles over all images
  int n_ot;     // output-channel blocks
  int x_bytes, w_bytes;
  int relu;
};

typedef short v4s __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x2 lds_tr8(unsigned addr) {
  const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<__attribute__((address_space(3))) v4s*>(size_t(addr)));
  return __builtin_bit_cast(u32x2, v);
}
__device__ __forceinline__ u32x4 lds_b128(unsigned addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(size_t(addr));
}

template <typename E>
__global__ __launch_bounds__(kPwNT, 2) void pw_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                      const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                      PwGeom g) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mw = wave & 1, nw = wave >> 1;  // 64-pixel half, 64-channel half

  // ---- tile: slot L -> XCD x = L % 8 takes the channel blocks of pixel tile t one after another ----
  const int L = int(blockIdx.x);
  const int xcd = L & 7, r = L >> 3;
  const int ot = r % g.n_ot, t = (r / g.n_ot) * 8 + xcd;
  if (t >= g.n_tiles) return;  // workgroup-uniform: padding slots of the last group
  const int b = t / g.n_ptile, p0 = (t - b * g.n_ptile) * kPwTP;
  const int o0 = ot * kPwTO;
  const int np = min(kPwTP, g.HW - p0);

  const v4i xr = make_vsharp(x, g.x_bytes);
  const v4i wr = make_vsharp(w, g.w_bytes);
  const unsigned lds0 = lds_addr(lds);

  // ---- load plan: block bi = kb*4 + wave; blocks 0-7 weights, 8-15 activations (1 KiB each) ----
  int l_off[kPwKL], l_step[kPwKL], l_cix[kPwKL];
#pragma unroll
  for (int kb = 0; kb < kPwKL; ++kb) {
    const int bi = kb * kPwNW + wave;
    int off = kOut, step = 0, cix = 0;
    if (bi < 8) {  // weight unit u: filter u >> 2, slot u & 3 holds chunk slot ^ ((o >> 2) & 3)
      const int u = bi * 64 + lane, o = u >> 2, c = (u & 3) ^ ((o >> 2) & 3);
      if (o0 + o < g.O) off = ((o0 + o) * g.C + c * 8) * 2;
      step = kPwKC * 2;
      cix = c * 8;
    } else {  // activation unit u: channel row u >> 4, position u & 15 holds chunk pos ^ (4*(row & 3))
      const int u = (bi - 8) * 64 + lane, row = u >> 4, gc = (u & 15) ^ (4 * (row & 3));
      if (gc * 8 < np) off = ((b * g.C + row) * g.HW + p0 + gc * 8) * 2;
      step = kPwKC * g.HW * 2;
      cix = row;
    }
    l_off[kb] = off;
    l_step[kb] = step;
    l_cix[kb] = cix;
  }
  int next_cs = 0;  // channel base of the next slice to issue
  auto issue = [&](int st) {
#pragma unroll
    for (int kb = 0; kb < kPwKL; ++kb) {
      const bool w_blk = kb * kPwNW + wave < 8;  // wave-uniform
      dma16(w_blk ? wr : xr, lds0 + st * kPwSB + (kb * kPwNW + wave) * 1024,
            next_cs + l_cix[kb] < g.C ? l_off[kb] : kOut);
      l_off[kb] += l_step[kb];
    }
    next_cs += kPwKC;
  };
#pragma unroll
  for (int st = 0; st < kPwNST - 1; ++st) issue(st);

  // ---- fragment addresses (absolute LDS addresses in stage 0) ----
  // B = weights: lane -> channel column nb*32 + lane%32 of this wave's half, 8 input channels 8*(lane/32)
  unsigned b_addr[2][2];  // [nb][k-step]
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int o = nw * 64 + nb * 32 + (lane & 31);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int ch = 2 * kk + (lane >> 5);
      b_addr[nb][kk] = lds0 + unsigned(o * 64 + ((ch ^ ((o >> 2) & 3)) << 4));
    }
  }
  // A = activations transposed: 16-lane group g16 covers pixels n0 .. n0+15 and channel rows k0 .. k0+3; lane s of
  // the group reads 4 pixels n0 + 4*(s & 3) of channel row k0 + (s >> 2)
  unsigned a_addr[2][2][2];  // [mb][k-step][half of the 8 channels]
  {
    const int s = lane & 15, g16 = lane >> 4;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int k0 = kk * 16 + 8 * (g16 >> 1) + 4 * h;
          const int row = k0 + (s >> 2);
          const int col = (mw * 64 + mb * 32 + 16 * (g16 & 1) + 4 * (s & 3)) * 2;  // byte column
          const int blk = (col >> 5) ^ (2 * (row & 3));
          a_addr[mb][kk][h] = lds0 + unsigned(kPwWBytes + row * (kPwTP * 2) + (blk << 5) + (col & 31));
        }
      }
    }
  }

  f32x16 acc[2][2] = {};
  auto slice = [&](int st) {
    const unsigned so = unsigned(st * kPwSB);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 bf[2], af[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) bf[nb] = lds_b128(b_addr[nb][kk] + so);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const u32x2 lo = lds_tr8(a_addr[mb][kk][0] + so), hi = lds_tr8(a_addr[mb][kk][1] + so);
        af[mb] = u32x4{lo.x, lo.y, hi.x, hi.y};
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = E::mfma32(af[mb], bf[nb], acc[mb][nb]);
      }
    }
  };

  // ---- main loop: slice sl from stage sl % 4 while slices sl+1 .. sl+3 load ----
  wait_vmcnt<2 * kPwKL>();  // slice 0 is in
  stage_barrier();
  for (int s0 = 0; s0 < g.S; s0 += kPwNST) {
#pragma unroll
    for (int st = 0; st < kPwNST; ++st) {
      if (s0 + st < g.S) {
        issue((st + kPwNST - 1) % kPwNST);  // slice sl+3 into the stage slice sl-1 used
        slice(st);
        wait_vmcnt<2 * kPwKL>();  // slice sl+1 is in
        stage_barrier();
      }
    }
  }
  wait_vmcnt<0>();
  __syncthreads();

  // ---- epilogue: bias + ReLU + one rounding into a 16-bit [channel][pixel] tile, then whole rows of Y ----
  {
    const int ol = lane & 31;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int oc = nw * 64 + nb * 32 + ol;  // tile channel
      const float bv = (bias != nullptr && o0 + oc < g.O) ? E::to_f32(bias[o0 + oc]) : 0.0f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t h[2];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            float v0 = acc[mb][nb][4 * q + 2 * j] + bv, v1 = acc[mb][nb][4 * q + 2 * j + 1] + bv;
            if (g.relu) {
              v0 = fmaxf(v0, 0.0f);
              v1 = fmaxf(v1, 0.0f);
            }
            h[j] = uint32_t(E::from_f32(v0)) | (uint32_t(E::from_f32(v1)) << 16);
          }
          const int px = mw * 64 + mb * 32 + 8 * q + 4 * (lane >> 5);  // 4 consecutive pixels
          *reinterpret_cast<u32x2*>(lds + oc * kPwRow + px * 2) = u32x2{h[0], h[1]};
        }
      }
    }
  }
  __syncthreads();
  // 128 rows x 256 bytes: 16 bytes per thread per pass, 16 rows per pass
#pragma unroll
  for (int pass = 0; pass < kPwTO * kPwTP * 2 / 16 / kPwNT; ++pass) {
    const int idx = pass * kPwNT + tid, row = idx >> 4, ck = idx & 15;
    if (o0 + row < g.O && ck * 8 < np) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(lds + row * kPwRow + ck * 16);
      *reinterpret_cast<u32x4*>(y + (static_cast<long long>(b) * g.O + o0 + row) * g.HW + p0 + ck * 8) = v;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Weight-stationary streaming variant (C <= 256). The per-tile kernel above re-reads a 128 x 32 weight slice
// and an X slice from L2 for every 128 x 128 output tile, and its 2 x 2 MFMA blocks per wave need ~256 B/clk of
// LDS reads at the MFMA rate (more than the LDS delivers). Here one workgroup per CU (8 waves, two per SIMD) keeps
// 256 filters x all C input channels in VGPRs for its whole life and streams one contiguous range of 64-pixel
// blocks of the flattened B*H*W pixel axis through a three-stage LDS ring:
//   * the weights come in once per workgroup: 256 filters x C by LDS-DMA into the LDS the ring and the output
//     tiles use later, each filter's OIHW row as 16-byte slots permuted by the filter index (kc ^ (f % RC)), so the
//     loads read whole rows and every wave's B-operand reads (filters 64*(w%4) .. +63, W[o][16j + 8*(lane/32) ..])
//     have at most two-way bank conflicts;
//   * block i = X[b][0 .. C)[p .. p+63] as two [channel][32 pixels] halves with 64-byte rows (16-byte chunks by
//     LDS-DMA; a block may straddle two images, each 8-pixel chunk is addressed on its own, H*W % 8 == 0);
//   * wave w takes pixel half w/4 against its 64 filters: A fragments by ds_read_b64_tr_b16 (rows k..k+3 of a
//     16-lane group are 64 bytes apart, the two groups of a half-wave 32 bytes: no bank conflicts), 2 MFMA chains;
//     the bias enters as one more k-step (A = 1 at k = 0, B = bias), after the real ones;
//   * epilogue: ReLU + one rounding; the two waves of a SIMD (same 64 filters, the two pixel halves) run half a
//     block apart and put their 64 x 32 halves into one 64 x 64 LDS tile of the block, and the second of them writes
//     the tile as 16-byte stores of 128-byte runs (8 filter rows per instruction): 34.7-35.1 us against 35.1-37.4
//     for each wave storing its own half as 64-byte runs with a four-stage ring (config 3, same process,
//     alternating batches, two boxes), although the 128-byte runs, 32 bytes into a line in three planes out of four
//     (784-pixel planes), write 1.05x the bytes of the 64-byte ones. The stores are device-scope (store16_wt): 34.77
//     against 35.17 us with write-back stores (which had won with 64-byte runs).
// Only X travels from L2 to LDS per block. The loads into the ring and the stores are issued through inline
// assembly in a fixed order so the waits can count them (vmcnt counts both, in issue order). The workgroups that
// share a pixel range (the 256-filter blocks of O) sit on one XCD (slot L -> XCD L % 8), so each X block comes
// from HBM once.
constexpr int kSwO = 256;   // filters per workgroup
constexpr int kSwP = 64;    // pixels per block (two halves of 32)
constexpr int kSwNST = 3;   // LDS ring stages
constexpr int kSwNW = 8;    // waves
constexpr int kSwNT = kSwNW * 64;
constexpr int kSwTile = 8192;  // output tile of one filter group and block: 64 filters x 64 pixels x 2 B
constexpr int kSwTiles = 4 * 2 * kSwTile;  // four filter groups, two tiles each (block parity)

struct PwsGeom {
  int C, HW, O, N;     // N = B*H*W pixels
  int n_ob;            // 256-filter blocks
  int n_ranges;        // pixel ranges (workgroups per filter block)
  int n_blk;           // 64-pixel blocks over N
  int x_bytes, w_bytes, y_bytes;
  unsigned hw_magic;   // n / HW = (umulhi(n, magic) + ((n - umulhi) >> 1)) >> (shift - 1)
  int hw_shift;
  int relu;
};

__device__ __forceinline__ unsigned div_hw(unsigned n, const PwsGeom& g) {
  const unsigned t = __umulhi(n, g.hw_magic);
  return (t + ((n - t) >> 1)) >> (g.hw_shift - 1);
}

// transposing 8-byte LDS read through a pointer, so constant offsets fold into the instruction's offset field
typedef __attribute__((address_space(3))) const unsigned char lds_cu8;
__device__ __forceinline__ u32x2 lds_tr8p(lds_cu8* p) {
  const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<__attribute__((address_space(3))) v4s*>(const_cast<__attribute__((address_space(3))) unsigned char*>(p)));
  return __builtin_bit_cast(u32x2, v);
}

// two FP32 values -> two 16-bit values in one register (gfx950 v_cvt_pk_{f16,bf16}_f32, round to nearest even)
template <typename E>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<Fp16>(float a, float b) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), h2));
}
template <>
__device__ __forceinline__ uint32_t pack2<Bf16>(float a, float b) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), b2));
}

// packed ReLU on two rounded 16-bit values: max(round(v), 0) == round(max(v, 0)) (rounding is monotonic and
// keeps the sign); v_pk_max_f16 for FP16, the FP32 max before rounding for BF16 (no packed BF16 max)
template <typename E>
__device__ __forceinline__ uint32_t relu2(uint32_t h) {
  if constexpr (E::kDtype == GIE_HIP_FP16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(h2, h), (h2){0, 0}));
  } else {
    return h;
  }
}

// v if ok, else the out-of-range offset, with bit operations (a conditional would become an exec-mask branch)
__device__ __forceinline__ unsigned sel_or_out(bool ok, unsigned v) {
  const unsigned m = 0u - unsigned(ok);
  return (v & m) | (unsigned(kOut) & ~m);
}

// BIG: H*W >= 64, so a 64-pixel block spans at most two images and the per-lane pixel offsets follow from the
// block's (image, pixel) pair, computed once per block in scalar registers; otherwise each lane divides.
template <typename E, int KS, bool RELU, bool BIG>
__global__ __launch_bounds__(kSwNT, 1) void pws_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                       const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                       PwsGeom g) {
  constexpr int KL = KS / 4;              // 1 KiB ring units per wave per block (2*KS units over 8 waves)
  constexpr int HB = KS * 1024;           // bytes per pixel half of a stage: 16*KS channels x 32 pixels x 2 B
  constexpr int SB = 2 * HB;              // bytes per stage
  constexpr int WL = KS * 8 * 1024 / (kSwNW * 1024);  // 1 KiB weight units per wave (256 x 16KS x 2 B in all)
  constexpr int ST_W = 8;                 // stores per block of a pixel-half-1 wave (half 0 stores none)
  constexpr int NST = kSwNST;
  constexpr int W_OFF = SB;               // weights land on stages 1 .. NST-1 and the output tiles
  constexpr bool kBf = E::kDtype == GIE_HIP_BF16;
  static_assert(KS == 4 || KS == 8 || KS == 16, "16-channel k-steps");
  static_assert((NST - 1) * SB + kSwTiles >= KS * 8 * 1024, "the weights fit the space they are staged in");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fg = wave & 3, ph = wave >> 2;  // filter group (64 filters), pixel half of each block
  static_assert(kSwP == 64, "BIG (one image wrap at most per block) assumes 64-pixel blocks and H*W >= 64");

  // ---- workgroup -> (filter block, pixel range); the n_ob workgroups of one range share an XCD ----
  const int L = int(blockIdx.x);
  const int xcd = L & 7, rr = L >> 3;
  const int ob = rr % g.n_ob, range = (rr / g.n_ob) * 8 + xcd;
  if (range >= g.n_ranges) return;  // workgroup-uniform padding slot
  const int blk0 = int((long long)g.n_blk * range / g.n_ranges);
  const int nblk = int((long long)g.n_blk * (range + 1) / g.n_ranges) - blk0;

  const v4i xr = make_vsharp(x, g.x_bytes);
  const v4i yr = make_vsharp(y, g.y_bytes);
  const v4i wr = make_vsharp(w, g.w_bytes);
  const v4i br = make_vsharp(bias, bias != nullptr ? g.O * 2 : 0);
  const unsigned lds0 = lds_addr(lds);
  const unsigned hw = unsigned(g.HW);
  const int o0 = kSwO * ob;

  // ---- ring loads: unit u = wave + 8*kb of a stage holds pixel half u / KS, channels 16*(u % KS) .. +15;
  //      lane: channel 16*(u % KS) + lane/4, pixel chunk lane%4 ----
  unsigned cx_off[KL], dx[KL];  // channel row offset (x_bytes past C: out of range), first pixel in the block
#pragma unroll
  for (int kb = 0; kb < KL; ++kb) {
    const int u = wave + kSwNW * kb;
    const int c = 16 * (u % KS) + (lane >> 2);
    cx_off[kb] = c < g.C ? unsigned(c) * hw * 2u : unsigned(g.x_bytes);
    dx[kb] = 32u * unsigned(u / KS) + 8u * unsigned(lane & 3);
  }
  const unsigned x_wrap = unsigned(g.C - 1) * hw * 2u;  // pixel p + d >= HW: same channel of the next image
  const unsigned y_wrap = unsigned(g.O - 1) * hw * 2u;
  // first pixel of block i: image b0 and pixel p0 (uniform), pixels left in the tensor from there
  struct Base {
    unsigned b0, p0, rem;
    bool whole;  // the block lies inside one image and the tensor: every lane's pixels valid, no image wrap
  };
  auto base_of = [&](int i) {
    Base r;
    const unsigned n0 = unsigned(blk0 + i) * kSwP;
    r.b0 = div_hw(n0, g);
    r.p0 = n0 - r.b0 * hw;
    r.rem = i < nblk ? unsigned(g.N) - n0 : 0u;
    r.whole = BIG && r.p0 + kSwP <= hw && r.rem >= kSwP;
    return r;
  };
  // lane constants of the common (whole-block) case: ring-load offset past the block's first pixel, per unit
  unsigned x_lane[KL];
#pragma unroll
  for (int kb = 0; kb < KL; ++kb) x_lane[kb] = dx[kb] * 2u + cx_off[kb];
  auto issue_unit = [&](int i, int st, const Base& bb, int kb) {
    if (bb.whole) {  // uniform: one add
      dma16(xr, lds0 + st * SB + (wave + kSwNW * kb) * 1024, int((bb.b0 * unsigned(g.C) * hw + bb.p0) * 2u + x_lane[kb]));
    } else {
      unsigned off;
      if constexpr (BIG) {
        const unsigned xs0 = (bb.b0 * unsigned(g.C) * hw + bb.p0) * 2u;
        off = sel_or_out(dx[kb] < bb.rem, xs0 + dx[kb] * 2u + (bb.p0 + dx[kb] >= hw ? x_wrap : 0u));
      } else {
        const unsigned n = unsigned(blk0 + i) * kSwP + dx[kb];
        const unsigned b = div_hw(n, g), p = n - b * hw;
        off = sel_or_out(i < nblk && n < unsigned(g.N), (b * unsigned(g.C) * hw + p) * 2u);
      }
      dma16(xr, lds0 + st * SB + (wave + kSwNW * kb) * 1024, int(off + cx_off[kb]));
    }
  };
  auto issue = [&](int i, int st, const Base& bb) {
#pragma unroll
    for (int kb = 0; kb < KL; ++kb) issue_unit(i, st, bb, kb);
  };

  // ---- prologue 1: block 0 into stage 0, the weights into the rest of LDS, the lane's bias values ----
  issue(0, 0, base_of(0));
  // weights: [256 filters][RC 16-byte slots], filter f's chunk kc (channels 8kc .. 8kc+7) in slot kc ^ (f % RC), so
  // a load instruction covers two whole OIHW rows (1 KiB contiguous) and the 32 filters of a B-operand read spread
  // over the banks
  constexpr int RC = 2 * KS;  // 16-byte chunks per filter row
#pragma unroll
  for (int t = 0; t < WL; ++t) {
    const int e = 64 * (wave + kSwNW * t) + lane, f = e / RC, kc = (e % RC) ^ (f % RC);
    const int o = o0 + f;
    dma16(wr, lds0 + W_OFF + (wave + kSwNW * t) * 1024, (o < g.O && 8 * kc < g.C) ? (o * g.C + 8 * kc) * 2 : kOut);
  }
  uint32_t braw[2];
  int o_lane[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    o_lane[nb] = o0 + 64 * fg + 32 * nb + (lane & 31);
    braw[nb] = load2_asm(br, o_lane[nb] < g.O && lane < 32 ? o_lane[nb] * 2 : kOut);
  }
  wait_vm<0>();
  touch_v(braw[0]);
  touch_v(braw[1]);
  __syncthreads();
  u32x4 wf[2][KS];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const int f = 64 * fg + 32 * nb + (lane & 31), kc = 2 * j + (lane >> 5);
      wf[nb][j] = lds_b128(lds0 + W_OFF + unsigned(f * RC + (kc ^ (f % RC))) * 16u);
    }
  stage_barrier();  // every wave holds its weights (lgkmcnt(0) in the barrier): the ring may overwrite them

  // ---- prologue 2: blocks 1 .. NST-2 in flight ----
#pragma unroll
  for (int st = 1; st < NST - 1; ++st) issue(st, st, base_of(st));

  // Ring load D(i+1) has landed for this wave once at most (loads issued after it) remain: the later ring loads
  // (NST-2 blocks) and the store batches issued since. Block j's ring load goes out during the MFMAs of block
  // j-NST+1; pixel half 1 stores block j-1 (both halves) before the MFMAs of block j and pixel half 0 stores nothing,
  // so at the end of block i that is min(i, NST - 2) store batches for half 1, none for half 0.
  auto wait_next = [&](int i) {
    static_assert(NST >= 3 && NST <= 6, "wait_next enumerates the warm-up blocks of a 3- to 6-stage ring");
    const int k = ph == 0 ? 0 : (i < NST - 2 ? i : NST - 2);
    if (k == 0) wait_vm<KL * (NST - 2)>();
    else if (k == 1) wait_vm<KL * (NST - 2) + ST_W * 1>();
    else if (k == 2) wait_vm<KL * (NST - 2) + ST_W * (2 < NST - 2 ? 2 : NST - 2)>();
    else if (k == 3) wait_vm<KL * (NST - 2) + ST_W * (3 < NST - 2 ? 3 : NST - 2)>();
    else wait_vm<KL * (NST - 2) + ST_W * (NST - 2)>();
  };
  static_assert(KL * (NST - 2) + ST_W * (NST - 2) < 64, "vmcnt range");

  // The bias enters as one more MFMA k-step after the real ones: A = 1 at k = 0 for every pixel, B = bias at
  // k = 0 for the lane's filter (lanes 0-31 carry k = 0..7). The single non-zero product is exact, so the sum is
  // acc + bias rounded once, the order of the reference's epilogue.
  const uint32_t one = kBf ? 0x3F80u : 0x3C00u;
  const u32x4 a_one = lane < 32 ? u32x4{one, 0u, 0u, 0u} : u32x4{0u, 0u, 0u, 0u};
  const u32x4 b_bias[2] = {u32x4{braw[0] & 0xffffu, 0u, 0u, 0u}, u32x4{braw[1] & 0xffffu, 0u, 0u, 0u}};

  // ---- epilogue: both pixel halves of a block leave together, as 128-byte runs ----
  // The accumulators hold, per lane, filter o_lane[nb] and pixels 8q + 4*(lane/32) + 0..3 of the wave's half. The two
  // waves of a filter group (w and w+4, one SIMD) write their halves into the group's tile of the block: [64 filters]
  // [64 pixels], 128-byte rows, the 16-byte segment s of row r (pixels 8s .. 8s+7) at s ^ ((r / 2) & 7), so the 8-byte
  // writes of 32 rows see 2-way bank conflicts and the 16-byte row reads none. Half 0 writes block i's half after its
  // MFMAs; half 1 writes block i's half at the start of block i+1 (after the barrier that follows half 0's writes),
  // reads the whole tile and stores it, 8 lanes per 128-byte run of a filter's output row, 8 rows per store
  // instruction. Each group has a tile per block parity: half 0 writes block i+1's tile while half 1 still reads
  // block i's, and block i+2 reuses block i's tile only after the barrier that ends block i+1.
  const unsigned stg = lds0 + unsigned(NST * SB) + unsigned(fg) * 2u * unsigned(kSwTile);
  typedef __attribute__((address_space(3))) u32x2 lds_u32x2_t;
  typedef __attribute__((address_space(3))) const u32x4 lds_cu32x4_t;
  lds_u32x2_t* w_q[4];  // granule writes (q, nb): row 32nb + lane%32, segment 4ph + q, 8-byte half lane/32
  {
    const unsigned r = unsigned(lane) & 31u, m = (r >> 1) & 7u, h = unsigned(lane) >> 5;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w_q[q] = reinterpret_cast<lds_u32x2_t*>(size_t(stg + r * 128u + (((4u * unsigned(ph) + unsigned(q)) ^ m) << 4) + (h << 3)));
  }
  // row read t covers rows 8t + lane/8, segment lane%8, stored at (lane%8) ^ (lane/16 + 4 (t%2))
  lds_cu32x4_t* r_base[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    r_base[par] = reinterpret_cast<lds_cu32x4_t*>(size_t(
        stg + (unsigned(lane) >> 3) * 128u + (((unsigned(lane) & 7u) ^ ((unsigned(lane) >> 4) + 4u * unsigned(par))) << 4)));
  // y offset of the row of read t: filter o0 + 64fg + 8t + lane/8 (y_bytes past O: out of range)
  unsigned o_row[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int o = o0 + 64 * fg + 8 * t + (lane >> 3);
    o_row[t] = o < g.O ? unsigned(o) * hw * 2u : unsigned(g.y_bytes);
  }
  const unsigned d_y = 8u * unsigned(lane & 7);  // the lane's first pixel of a row segment
  unsigned st_x = 0;                            // y offset of that pixel
  auto seg_offset = [&](int i, const Base& bb) {
    if (bb.whole) {
      st_x = (bb.b0 * unsigned(g.O) * hw + bb.p0) * 2u + d_y * 2u;
    } else if constexpr (BIG) {
      const unsigned ys0 = (bb.b0 * unsigned(g.O) * hw + bb.p0) * 2u;
      st_x = sel_or_out(d_y < bb.rem, ys0 + d_y * 2u + (bb.p0 + d_y >= hw ? y_wrap : 0u));
    } else {
      const unsigned n = unsigned(blk0 + i) * kSwP + d_y;
      const unsigned b = div_hw(n, g), p = n - b * hw;
      st_x = sel_or_out(n < unsigned(g.N), (b * unsigned(g.O) * hw + p) * 2u);
    }
  };
  auto put = [&](const f32x16 (&acc)[2], int q, int nb, int par) {
    uint32_t h[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float v0 = acc[nb][4 * q + 2 * e], v1 = acc[nb][4 * q + 2 * e + 1];
      if (RELU && kBf) {
        v0 = fmaxf(v0, 0.f);
        v1 = fmaxf(v1, 0.f);
      }
      h[e] = pack2<E>(v0, v1);
      if (RELU && !kBf) h[e] = relu2<E>(h[e]);
    }
    w_q[q][nb * 512 + par * 1024] = u32x2{h[0], h[1]};  // + 32 rows for the second 32-filter block, + 8 KiB per parity
  };
  auto stage_half = [&](const f32x16 (&acc)[2], int i) {
    const int par = i & 1;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) put(acc, q, nb, par);
    // A wave's LDS accesses complete in issue order, so the reads see the writes once the compiler keeps that order
    // (the tile is written as 8-byte and read as 16-byte vectors, which type-based alias analysis would separate).
    asm volatile("" ::: "memory");
  };
  auto epilogue = [&](const f32x16 (&acc)[2], int i) {  // pixel half 1: its half of block i, then the block to y
    seg_offset(i, base_of(i));
    stage_half(acc, i);
    const int par = i & 1;
    u32x4 v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = r_base[t & 1][t * 64 + par * 512];  // + 1 KiB per 8 rows, + 8 KiB per parity
#pragma unroll
    for (int t = 0; t < 8; ++t) store16_wt(yr, int(st_x + o_row[t]), v[t]);
  };

  // ---- A-fragment addresses: 16-lane group g16 reads pixels 16*(g16&1) .. +15 of channel rows k0 .. k0+3,
  //      k0 = 16j + 8*(g16>>1) + 4h; lane s of the group: row k0 + s/4, pixels +4*(s%4) ----
  unsigned a_lane;
  {
    const int s = lane & 15, g16 = lane >> 4;
    a_lane = unsigned(ph * HB + (8 * (g16 >> 1) + (s >> 2)) * 64 + (16 * (g16 & 1) + 4 * (s & 3)) * 2);
  }
  lds_cu8* const a_base = reinterpret_cast<lds_cu8*>(size_t(lds0 + a_lane));
  // The two waves that share a SIMD (w and w+4: same filters, other pixel half) work out of phase: half 0 runs
  // the MFMAs of block i and then its epilogue, half 1 the epilogue of block i-1 and then the MFMAs of block i,
  // so one wave's epilogue overlaps the other's MFMAs and each wave needs one accumulator set.
  f32x16 acc[2];
  auto compute = [&](int i) {
    lds_cu8* ab = a_base + (i % NST) * SB;
    const int i_ld = i + NST - 1, st_ld = (i + NST - 1) % NST;  // the ring load that goes out meanwhile
    const Base b_ld = base_of(i_ld);
    acc[0] = f32x16{};
    acc[1] = f32x16{};
    // A fragments two k-steps ahead of the MFMAs that use them (LDS latency exceeds two MFMA issues)
    constexpr int PF = 2;
    u32x4 af[PF + 1];
    auto read_a = [&](int j) {
      const u32x2 lo = lds_tr8p(ab + j * 1024), hi = lds_tr8p(ab + j * 1024 + 256);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    };
#pragma unroll
    for (int j = 0; j < PF; ++j) af[j] = read_a(j);
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      if (j + PF < KS) af[(j + PF) % (PF + 1)] = read_a(j + PF);
      acc[0] = E::mfma32(af[j % (PF + 1)], wf[0][j], acc[0]);
      acc[1] = E::mfma32(af[j % (PF + 1)], wf[1][j], acc[1]);
      // ring-load units between the MFMAs (issued in a burst they would wait behind the stores in the memory
      // pipeline before the MFMAs could start)
      if constexpr (KS >= 2 * KL) {
        if (j % 2 == 1 && j / 2 < KL) issue_unit(i_ld, st_ld, b_ld, j / 2);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the reads PF steps ahead (the scheduler would cluster them)
    }
    acc[0] = E::mfma32(a_one, b_bias[0], acc[0]);
    acc[1] = E::mfma32(a_one, b_bias[1], acc[1]);
  };

  for (int i = 0; i < nblk; ++i) {
    if (ph == 1 && i > 0) epilogue(acc, i - 1);
    compute(i);
    if (ph == 0) stage_half(acc, i);
    wait_next(i);  // block i+1 has landed (this wave's part)
    stage_barrier();
  }
  if (ph == 1) epilogue(acc, nblk - 1);
  wait_vm<0>();  // ring loads past the range still target this workgroup's LDS
}

// geometry checks shared by the capability query and the launch
int pw_prepare(const gie_conv_geom* gg, PwGeom* g) {
  if (!gg) return GIE_HIP_EINVAL;
  if (gg->kernel_h != 1 || gg->kernel_w != 1 || gg->stride_h != 1 || gg->stride_w != 1 || gg->pad_h != 0 ||
      gg->pad_w != 0)
    return GIE_HIP_EUNSUPPORTED;
  if (gg->batch <= 0 || gg->in_channels <= 0 || gg->in_h <= 0 || gg->in_w <= 0 || gg->out_channels <= 0)
    return GIE_HIP_EINVAL;
  const long long hw = static_cast<long long>(gg->in_h) * gg->in_w;
  // whole 16-byte chunks: 8 channels of a filter, 8 pixels of a channel row
  if (gg->in_channels % 8 != 0 || hw % 8 != 0) return GIE_HIP_EUNSUPPORTED;
  const long long xb = hw * gg->batch * gg->in_channels * 2, wb = static_cast<long long>(gg->out_channels) * gg->in_channels * 2;
  const long long yn = hw * gg->batch * gg->out_channels;
  if (xb + hw * 2 * kPwKC >= 0x7fffffffLL || wb >= 0x7fffffffLL || yn >= 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  g->B = gg->batch;
  g->C = gg->in_channels;
  g->HW = int(hw);
  g->O = gg->out_channels;
  g->S = (g->C + kPwKC - 1) / kPwKC;
  g->n_ptile = int((hw + kPwTP - 1) / kPwTP);
  const long long tiles = static_cast<long long>(g->n_ptile) * g->B;
  g->n_ot = (g->O + kPwTO - 1) / kPwTO;
  const long long slots = (tiles + 7) / 8 * 8 * g->n_ot;
  if (tiles > 0x7fffffffLL || slots > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  g->n_tiles = int(tiles);
  g->x_bytes = int(xb);
  g->w_bytes = int(wb);
  g->relu = gg->relu ? 1 : 0;
  return GIE_HIP_OK;
}

// geometry checks of the streaming variant, shared by its capability query and its launch
int pws_prepare(const gie_conv_geom* gg, int cu_count, PwsGeom* g, int* ks) {
  PwGeom base;
  if (int rc = pw_prepare(gg, &base)) return rc;
  if (gg->in_channels > 16 * 16) return GIE_HIP_EUNSUPPORTED;  // weights of 256 filters x C must fit the VGPRs
  const long long n = static_cast<long long>(gg->batch) * gg->in_h * gg->in_w;
  const long long yb = n * gg->out_channels * 2;
  if (yb >= 0x7fffffffLL || n >= 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  g->C = gg->in_channels;
  g->HW = base.HW;
  g->O = gg->out_channels;
  g->N = int(n);
  g->n_ob = (g->O + kSwO - 1) / kSwO;
  g->n_blk = int((n + kSwP - 1) / kSwP);
  const int target = std::max(1, cu_count / g->n_ob);  // one workgroup per CU
  g->n_ranges = std::max(1, std::min(g->n_blk, target));
  const long long slots = static_cast<long long>((g->n_ranges + 7) / 8) * 8 * g->n_ob;
  if (slots > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  g->x_bytes = base.x_bytes;
  g->w_bytes = base.w_bytes;
  g->y_bytes = int(yb);
  // n / HW for 32-bit n: l = ceil(log2 HW), magic = floor(2^32 (2^l - HW) / HW) + 1 (HW >= 8)
  int l = 0;
  while ((1LL << l) < g->HW) ++l;
  g->hw_shift = l;
  g->hw_magic = unsigned((((1ULL << l) - unsigned(g->HW)) << 32) / unsigned(g->HW) + 1);
  g->relu = base.relu;
  const int k16 = (g->C + 15) / 16;
  *ks = k16 <= 4 ? 4 : k16 <= 8 ? 8 : 16;
  return GIE_HIP_OK;
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_pw_check(const gie_conv_geom* g, int* lds_bytes) {
  PwGeom pg;
  const int rc = pw_prepare(g, &pg);
  if (rc == GIE_HIP_OK && lds_bytes) *lds_bytes = kPwLds;
  return rc;
}

extern "C" int gie_hip_conv_pw(int dtype, const gie_conv_geom* gg, const void* x, const void* w, const void* bias,
                               void* y, void* stream) {
  if (!gg || !x || !w || !y) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if (bias && (reinterpret_cast<uintptr_t>(bias) & 1u)) return GIE_HIP_EINVAL;
  PwGeom g;
  if (int rc = pw_prepare(gg, &g)) return rc;
  // 16-byte chunks straight from the caller's tensors and 16-byte row stores into y
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(w) & 15u) ||
      (reinterpret_cast<uintptr_t>(y) & 15u))
    return GIE_HIP_EUNSUPPORTED;
  using Fn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, PwGeom);
  const Fn fn = dtype == GIE_HIP_BF16 ? &pw_kernel<Bf16> : &pw_kernel<Fp16>;
  const long long slots = static_cast<long long>((g.n_tiles + 7) / 8) * 8 * g.n_ot;
  hipLaunchKernelGGL(fn, dim3(unsigned(slots)), dim3(kPwNT), kPwLds, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                     static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}

extern "C" int gie_hip_pws_check(const gie_conv_geom* g, int* lds_bytes) {
  PwsGeom pg;
  int ks = 0;
  const int rc = pws_prepare(g, 256, &pg, &ks);
  if (rc == GIE_HIP_OK && lds_bytes) *lds_bytes = kSwNST * 2 * ks * 1024 + kSwTiles;
  return rc;
}

extern "C" int gie_hip_conv_pws(int dtype, const gie_conv_geom* gg, const void* x, const void* w, const void* bias,
                                void* y, void* stream) {
  if (!gg || !x || !w || !y) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if (bias && (reinterpret_cast<uintptr_t>(bias) & 1u)) return GIE_HIP_EINVAL;
  PwsGeom g;
  int ks = 0;
  if (int rc = pws_prepare(gg, current_device_cus(), &g, &ks)) return rc;
  // 16-byte chunks into LDS, 16-byte weight loads, 8-byte stores
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(w) & 15u) ||
      (reinterpret_cast<uintptr_t>(y) & 7u))
    return GIE_HIP_EUNSUPPORTED;
  using Fn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, PwsGeom);
  static const Fn table[2][3][2][2] = {
      {{{&pws_kernel<Fp16, 4, false, false>, &pws_kernel<Fp16, 4, false, true>},
        {&pws_kernel<Fp16, 4, true, false>, &pws_kernel<Fp16, 4, true, true>}},
       {{&pws_kernel<Fp16, 8, false, false>, &pws_kernel<Fp16, 8, false, true>},
        {&pws_kernel<Fp16, 8, true, false>, &pws_kernel<Fp16, 8, true, true>}},
       {{&pws_kernel<Fp16, 16, false, false>, &pws_kernel<Fp16, 16, false, true>},
        {&pws_kernel<Fp16, 16, true, false>, &pws_kernel<Fp16, 16, true, true>}}},
      {{{&pws_kernel<Bf16, 4, false, false>, &pws_kernel<Bf16, 4, false, true>},
        {&pws_kernel<Bf16, 4, true, false>, &pws_kernel<Bf16, 4, true, true>}},
       {{&pws_kernel<Bf16, 8, false, false>, &pws_kernel<Bf16, 8, false, true>},
        {&pws_kernel<Bf16, 8, true, false>, &pws_kernel<Bf16, 8, true, true>}},
       {{&pws_kernel<Bf16, 16, false, false>, &pws_kernel<Bf16, 16, false, true>},
        {&pws_kernel<Bf16, 16, true, false>, &pws_kernel<Bf16, 16, true, true>}}}};
  const Fn fn = table[dtype == GIE_HIP_BF16 ? 1 : 0][ks == 4 ? 0 : ks == 8 ? 1 : 2][g.relu ? 1 : 0][g.HW >= kSwP ? 1 : 0];
  const int lds = kSwNST * 2 * ks * 1024 + kSwTiles;  // ring + two 8 KiB output tiles per filter group
  if (int rc = set_lds_limit(reinterpret_cast<const void*>(fn), lds)) return rc;
  const long long slots = static_cast<long long>((g.n_ranges + 7) / 8) * 8 * g.n_ob;
  hipLaunchKernelGGL(fn, dim3(unsigned(slots)), dim3(kSwNT), lds, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                     static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
