// Band convolution straight from NCHW on gfx950 matrix cores (v_mfma_f32_32x32x16_{f16,bf16}, FP32
// accumulation): no activation repack. Weights come channel-blocked, wb [O][S][KH*KW][32] (S = ceil(C / 32)
// slices of 32 channels, zero padded; gie_hip_repack_w_blocked writes it).
//
// GEMM view (reference naming): M = out_channels, N = batch*out_h*out_w output pixels, K = kh*kw*32*S. A workgroup
// owns 32 output channels x one band of R output rows of one image. The band's pixels are laid out in rows of
// OWP = 2^k >= out_w columns (the columns past out_w are computed and dropped), cut into NG groups of 32: one
// 32x32 MFMA block each, R = NG*32 / OWP. Blocks are numbered image-band fastest, so the workgroups that share an
// XCD (blockIdx mod 8) share few images and all of each filter block.
// Per channel slice an LDS stage holds
//   * the band's input rows, each input pixel's 32 channels as four 16-byte chunks (chunk c at slot
//     c ^ ((pos >> 2) & 3), so any 16 consecutive positions hit 16 distinct bank groups); image padding is zero;
//   * the weights [32][KH*KW][4 slots], slot = chunk ^ ((o >> 2) & 3).
// Activations travel NCHW -> registers -> LDS: per slice the band's input rows of each channel are one
// contiguous run, read with 8-byte loads (4 pixels x 4 channels per thread, or 2-byte loads when alignment does
// not allow) and written transposed with 8-byte LDS stores. Weights travel by direct-to-LDS buffer loads. Both
// are prefetched: the weights NST-1 slices ahead, the activations one slice ahead.
// Waves: (group pair) x (channel half). Each wave multiplies one weight fragment against its two pixel groups for
// every tap of its 16 channels; the two halves are summed through LDS at the end. When a band row is one 16-lane
// DPP row (OWP == 16, stride 1, out_w + kw - 1 <= 16) the fragment of tap column s is the column-0 fragment shifted
// s lanes (row_shl): one LDS read per filter row instead of KW (the lanes shifted in are dropped columns).
// Epilogue: bias + ReLU on the FP32 sums, one RNE rounding, NCHW stores; or FP32 partials partial[z][NCHW] for
// split-K (reduced by splitk_reduce.hip), over channel slices [floor(S*z/split), floor(S*(z+1)/split)) as the
// reference partitions K (src/kernels/tensor_core_mma.cu:112-115, :231-234).
#include <algorithm>
#include <type_traits>
#include <utility>
#include <vector>

#include "lds_pipe.h"

namespace gie_hip {
namespace {

constexpr int kCS = 32;   // channels per slice
constexpr int kTO = 32;   // output channels per workgroup (one 32-row MFMA block)
constexpr int kKxMax = 2; // transposition rounds per thread (DMA form)
constexpr int kKlMin = 2, kKlMax = 6;  // DMA form: load blocks per wave per slice
constexpr int kKuMax = 3;               // register form: activation units per thread

struct BandGeom {
  int B, C, H, W, O, S, OH, OW, SH, SW, PH, PW;
  int HW, OHW, Y;   // input and output pixels per image plane; output elements
  int lgOWP;        // log2 of the padded output row width
  int R, n_bands;   // output rows per band; bands per image
  int IR, IWP;      // LDS input rows per band and their pitch (positions)
  int XTB;          // bytes of one transposed activation buffer: positions (multiple of 4) x 64
  int NCH, NBX;     // DMA form: 16-byte chunks per channel run; 1 KiB activation blocks per slice
  int x_bytes, wb_bytes;
  int relu;
  float inv_w, inv_nch;
};

template <int KH, int KW, int NG, int NST>
struct BShape {
  static constexpr int RS = KH * KW;
  static constexpr int NP = (NG + 1) / 2;  // group pairs
  static constexpr int NW = 2 * NP;        // waves: group pair x channel half
  static constexpr int NT = NW * 64;
  static constexpr int NBW = 2 * RS;               // 1 KiB weight blocks per slice: 32 filters x RS taps x 64 B
  static constexpr int KBW = (NBW + NW - 1) / NW;  // register form: weight loads per wave per slice (+ dummies)
  static_assert(NST >= 2 && NST <= 4, "two to four load stages");
  static_assert(NG >= 1 && NG <= 8, "one to eight pixel groups");
};

// Vector-memory loads into registers that the compiler does not see as loads: their results are valid only after
// a counted wait (wait_a), which also makes every later use depend on it.
__device__ __forceinline__ uint32_t load_u16(v4i rsrc, int voff) {
  uint32_t v;
  asm volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rsrc));
  return v;
}
template <int N>
__device__ __forceinline__ void wait_vm_asm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}
template <typename T>
__device__ __forceinline__ void touch(T& v) {
  asm volatile("" : "+v"(v));
}

// Lane i of each 16-lane row takes lane i + S (row_shl:S); lanes past the row read zero.
template <int S>
__device__ __forceinline__ u32x4 shl_rows(u32x4 v) {
  if constexpr (S == 0) {
    return v;
  } else {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = uint32_t(__builtin_amdgcn_mov_dpp(int(v[i]), 0x100 + S, 0xf, 0xf, true));
    return r;
  }
}
__device__ __forceinline__ u32x4 shl_rows_n(u32x4 v, int s) {
  switch (s) {
    case 0: return v;
    case 1: return shl_rows<1>(v);
    case 2: return shl_rows<2>(v);
    case 3: return shl_rows<3>(v);
    case 4: return shl_rows<4>(v);
    case 5: return shl_rows<5>(v);
    case 6: return shl_rows<6>(v);
    default: return shl_rows<7>(v);
  }
}

// LDS accesses by absolute 32-bit LDS address (the workgroup's base already folded into the address), so the
// only arithmetic left in the loop is the instruction's immediate offset
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
__device__ __forceinline__ u32x4 lds_ld16(unsigned addr) { return *reinterpret_cast<const lds_u32x4*>(size_t(addr)); }
__device__ __forceinline__ u32x2 lds_ld8(unsigned addr) { return *reinterpret_cast<const lds_u32x2*>(size_t(addr)); }
__device__ __forceinline__ void lds_st8(unsigned addr, u32x2 v) { *reinterpret_cast<lds_u32x2*>(size_t(addr)) = v; }

// Four channels of one pixel from four channel rows of four pixels (a_j = the 32-bit half holding the pixel):
// {c0 | c1 << 16, c2 | c3 << 16}
__device__ __forceinline__ u32x2 pixel4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t sel) {
  return u32x2{__builtin_amdgcn_perm(a1, a0, sel), __builtin_amdgcn_perm(a3, a2, sel)};
}

// DMA = true: activations travel by direct-to-LDS loads of each channel's contiguous input run into the load stage
// (KL = load blocks per wave per slice, weights and runs together) and are transposed LDS -> LDS one slice ahead.
// DMA = false: 2-byte register loads (KL = activation units per thread) written transposed; weights by
// direct-to-LDS loads. The DMA form needs 16-byte aligned x and runs that start on 8-byte boundaries.
template <typename E, int KH, int KW, int NG, int NST, int KL, bool DMA, bool SHIFT>
__global__ __launch_bounds__((NG + 1) / 2 * 128) void band_kernel(const uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ wb,
                                                                  const uint16_t* __restrict__ bias,
                                                                  uint16_t* __restrict__ y,
                                                                  float* __restrict__ partial, BandGeom g,
                                                                  int split) {
  using Sh = BShape<KH, KW, NG, NST>;
  constexpr int RS = Sh::RS, NW = Sh::NW, NT = Sh::NT, NBW = Sh::NBW, KBW = Sh::KBW;
  static_assert(!DMA || NST >= 3, "the DMA form transposes one slice ahead of the loads");
  static_assert((DMA ? KL : 16 * KL + KBW) < 64, "loads per slice must fit the vmcnt counter");
  constexpr int KX = DMA ? kKxMax : KL;          // transposition rounds
  constexpr int NLB = DMA ? KL : KBW;             // load blocks per wave per slice
  constexpr int SB = NLB * NW * 1024;             // bytes of one load stage
  constexpr int XT0 = NST * SB;                   // the two transposed activation buffers follow the stages
  constexpr int UNR = NST % 2 == 0 ? NST : 2 * NST;  // loop unroll: stage and buffer indices are constants
  // LDS instruction offsets are 16-bit: stage st is reached as base[(st*SB) >> 16] + ((st*SB) & 0xffff)
  static_assert((NST - 1) * SB < 2 * 65536, "two base registers reach every stage");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pr = wave >> 1, hh = wave & 1;
  // the last pair of an odd NG has one group: it multiplies that group twice (no branch in the loop; its SIMD
  // does no more MFMAs than the others) and drops the copy
  const bool two = (NG % 2 == 0) || (pr < Sh::NP - 1);

  // grid (image-band, 32-filter block, split): consecutive workgroups share images, so the eight XCDs
  // (blockIdx mod 8) each see few images and every filter block
  const int ib = int(blockIdx.x), ot = int(blockIdx.y);
  const int b = g.n_bands == 1 ? ib : ib / g.n_bands, band = ib - b * g.n_bands;
  const int o0 = ot * kTO, oh0 = band * g.R;
  const int z = int(blockIdx.z);
  const int s_beg = (g.S * z) / split, ns = (g.S * (z + 1)) / split - s_beg;

  const v4i xr = make_vsharp(x, g.x_bytes);
  const v4i wr = make_vsharp(wb, g.wb_bytes);
  const unsigned lds0 = lds_addr(lds);

  const int ih_base = oh0 * g.SH - g.PH;  // input row of LDS row 0
  const int ih_lo = max(ih_base, 0), ih_hi = min(ih_base + g.IR, g.H);
  const int L = max(ih_hi - ih_lo, 0) * g.W;  // pixels of each channel's run
  const int nq = (L + 3) >> 2;
  const bool run_whole = (L & 3) == 0;
  const int ebase = (b * g.C + s_beg * kCS) * g.HW + ih_lo * g.W;  // element of channel 0's run (uniform)

  // ---- loads into the stages: per wave NLB blocks of 1 KiB per slice, issued in slice order; each lane keeps
  // its next source offset and channel index and advances them by one slice per issue ----
  int l_off[NLB], l_step[NLB], l_cix[NLB];
#pragma unroll
  for (int kb = 0; kb < NLB; ++kb) {
    const int bi = kb * NW + wave;
    int off = kOut, step = 0, cix = -(1 << 30);
    if (bi < NBW) {
      // weight block: the chunk that belongs at LDS unit u = (o*RS + t)*4 + slot
      const int u = bi * 64 + lane;
      const int ou = u >> 2, o = ou / RS, t = ou - o * RS, slot = u & 3;
      if (o0 + o < g.O)
        off = ((o0 * g.S + s_beg) * RS) * 64 + int(__umul24(unsigned(o), unsigned(g.S * RS * 64))) + t * 64 +
              ((slot ^ ((o >> 2) & 3)) << 4);
      step = RS * 64;
    } else if (DMA && bi < NBW + g.NBX) {
      // activation run chunk: channel c's run starts 8-byte aligned; chunk k covers its bytes [16k - d, 16k+16-d)
      const int u = (bi - NBW) * 64 + lane;
      if (u < kCS * g.NCH) {
        const int c = fdiv(u, g.NCH, g.inv_nch), k = u - c * g.NCH;
        const int e = ebase + int(__umul24(unsigned(c), unsigned(g.HW)));
        off = ((2 * e) & ~15) + 16 * k;
        step = 2 * kCS * g.HW;
        cix = s_beg * kCS + c;
      }
    }
    l_off[kb] = off;
    l_step[kb] = step;
    l_cix[kb] = cix;
  }
  auto issue_one = [&](int kb, int st) {  // block kb of the next slice in order into stage st
    const bool w_blk = kb * NW + wave < NBW;  // wave-uniform
    dma16(w_blk ? wr : xr, lds0 + st * SB + (kb * NW + wave) * 1024, l_cix[kb] < g.C ? l_off[kb] : kOut);
    l_off[kb] += l_step[kb];
    l_cix[kb] += kCS;
  };
  // the first NST-1 slices start loading now; the rest of the set-up runs under their latency
#pragma unroll
  for (int st = 0; st < NST - 1; ++st) {
#pragma unroll
    for (int kb = 0; kb < NLB; ++kb) issue_one(kb, st);
  }

  // ---- activation transposition plan: unit (channel quad cq, pixel quad q) -> four 8-byte position writes ----
  const int units = 8 * nq;
  unsigned t_rd[KX][4], t_wr[KX][4];
  unsigned t_rd_hi[4], t_wr1[4];  // round 0: reads from stages past 64 KiB, stores into buffer 1
  bool t_ok[KX], t_px[KX][4];
  int t_cb[KX];
#pragma unroll
  for (int k = 0; k < KX; ++k) {
    const int u = k * NT + tid, cq = u & 7, q = u >> 3;
    t_ok[k] = q < nq;
    t_cb[k] = s_beg * kCS + 4 * cq;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      t_rd[k][j] = DMA ? lds0 : unsigned(kOut);
      t_wr[k][j] = lds0;
      t_px[k][j] = false;
    }
    if (k > 0 && k * NT >= units) continue;  // workgroup-uniform: no unit in this round
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = 4 * cq + j;
      const int e0 = ebase + int(__umul24(unsigned(c), unsigned(g.HW)));  // channel c's run
      if constexpr (DMA) {
        // units past the run read offset 0 of the stage (harmless) and write nothing
        if (t_ok[k])
          t_rd[k][j] = lds0 + unsigned(NBW * 1024) + __umul24(unsigned(c), unsigned(g.NCH * 16)) +
                       unsigned((2 * e0) & 15) + unsigned(8 * q);
      } else {
        if (t_ok[k]) t_rd[k][j] = unsigned(2 * (e0 + 4 * q));  // global byte offset of slice 0
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int px = 4 * q + i;
      t_px[k][i] = t_ok[k] && px < L;
      const int rr = fdiv(px, g.W, g.inv_w);
      const int pos = int(__umul24(unsigned(ih_lo - ih_base + rr), unsigned(g.IWP))) + (px - rr * g.W) + g.PW;
      t_wr[k][i] = lds0 + unsigned(XT0 + pos * 64 + ((((cq >> 1) ^ ((pos >> 2) & 3))) << 4) + ((cq & 1) << 3));
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    t_rd_hi[j] = t_rd[0][j] + 65536u;
    t_wr1[j] = t_wr[0][j] + unsigned(g.XTB);
    // opaque to the compiler, which would otherwise fold them back into base + a constant too large for the
    // instruction offset
    touch(t_rd_hi[j]);
    touch(t_wr1[j]);
  }
  // four channels of pixel i of the unit from four channel rows of the quad
  auto unit_pixels = [&](const u32x2 (&v)[4], u32x2 (&d)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
      d[i] = (i & 2) ? pixel4(v[0].y, v[1].y, v[2].y, v[3].y, sel) : pixel4(v[0].x, v[1].x, v[2].x, v[3].x, sel);
    }
  };
  auto unit_store = [&](int k, int xb, const u32x2 (&d)[4]) {
    if (t_ok[k]) {
      unsigned w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = k == 0 ? (xb ? t_wr1[i] : t_wr[0][i]) : t_wr[k][i] + unsigned(xb * g.XTB);
      if (run_whole) {  // workgroup-uniform: every pixel of a valid unit lies in the run
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_st8(w[i], d[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (t_px[k][i]) lds_st8(w[i], d[i]);
      }
    }
  };
  auto raw_read = [&](int k, int j, int st) {  // transposition read of channel row j of unit round k, stage st
    const unsigned so = unsigned(st * SB);
    const unsigned a = (k == 0 && so >= 65536u) ? t_rd_hi[j] + (so - 65536u) : t_rd[k][j] + so;
    return lds_ld8(a);
  };
  // DMA form: LDS -> LDS transposition of the slice in stage st into transposed buffer xb
  auto transpose = [&](int st, int xb) {
#pragma unroll
    for (int k = 0; k < KX; ++k) {
      if (k == 0 || k * NT < units) {
        u32x2 v[4], d[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = raw_read(k, j, st);
        unit_pixels(v, d);
        unit_store(k, xb, d);
      }
    }
  };
  // register form: 2-byte loads of slice sl, then (after the counted wait) transposed stores
  uint32_t rb[DMA ? 1 : KL][16];
  auto issue_a = [&](int sl) {
    if constexpr (!DMA) {
      const int cs = sl * kCS;
#pragma unroll
      for (int k = 0; k < KL; ++k) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int off = (t_cb[k] + cs + j < g.C) ? int(t_rd[k][j]) + cs * g.HW * 2 : kOut;
#pragma unroll
          for (int i = 0; i < 4; ++i) rb[k][j * 4 + i] = load_u16(xr, off + 2 * i);
        }
      }
    }
  };
  auto wait_a = [&](auto n_c) {
    wait_vm_asm<decltype(n_c)::value>();
    if constexpr (!DMA) {
#pragma unroll
      for (int k = 0; k < KL; ++k) {
#pragma unroll
        for (int j = 0; j < 16; ++j) touch(rb[k][j]);
      }
    }
  };
  auto write_a = [&](int xb) {
    if constexpr (!DMA) {
#pragma unroll
      for (int k = 0; k < KL; ++k) {
        u32x2 d[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          d[i] = u32x2{(rb[k][i] & 0xffffu) | (rb[k][4 + i] << 16), (rb[k][8 + i] & 0xffffu) | (rb[k][12 + i] << 16)};
        unit_store(k, xb, d);
      }
    }
  };

  // ---- fragment addresses (per transposed buffer, so no address arithmetic runs in the loop) ----
  const int chunk = 2 * hh + (lane >> 5);
  const int ol = lane & 31;
  const unsigned a_off = lds0 + unsigned(ol * RS * 64 + ((chunk ^ ((ol >> 2) & 3)) << 4));
  unsigned a_off_hi = a_off + 65536u;
  touch(a_off_hi);
  constexpr int NTB = SHIFT ? KH : RS;  // B fragment reads per group per slice
  unsigned b_off[2][2][NTB];
  const int owp_mask = (1 << g.lgOWP) - 1;
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    const int f = (2 * pr + (two ? gi : 0)) * 32 + (lane & 31);
    const int orow = f >> g.lgOWP, ocol = f & owp_mask;
#pragma unroll
    for (int tb = 0; tb < NTB; ++tb) {
      const int r = SHIFT ? tb : tb / KW, s = SHIFT ? 0 : tb % KW;
      const int pos = int(__umul24(unsigned(orow * g.SH + r), unsigned(g.IWP))) + ocol * g.SW + s;
      const unsigned o = lds0 + unsigned(XT0 + pos * 64 + ((chunk ^ ((pos >> 2) & 3)) << 4));
      b_off[0][gi][tb] = o;
      b_off[1][gi][tb] = o + unsigned(g.XTB);
      touch(b_off[1][gi][tb]);
    }
  }

  // four independent accumulator chains per wave: [pixel group][tap parity]
  f32x16 acc[2][2] = {};
  // DMA form: the first unit's weight fragments of the next slice, read before the barrier that ends a slice
  // (its weights landed an iteration earlier)
  constexpr int NAc = SHIFT ? KW : 1;
  u32x4 fa_next[NAc];
  auto prefetch_a = [&](int st) {
    const unsigned so = unsigned(st * SB);
    const unsigned a_base = so >= 65536u ? a_off_hi : a_off;
#pragma unroll
    for (int s = 0; s < NAc; ++s) fa_next[s] = lds_ld16(a_base + (so & 0xffffu) + s * 64);
  };
  // One iteration: multiply the slice in stage st / transposed buffer xb. DMA form: the next slice in order is
  // loaded into stage ist (its blocks spread over the slice) and the slice in stage tst is transposed into buffer
  // txb (reads first, stores mid-slice). Fragments are read one unit (filter row, or tap) ahead of their MFMAs.
  auto slice = [&](int st, int xb, int ist, int tst, int txb) {
    const unsigned so = unsigned(st * SB);
    const unsigned a_base = so >= 65536u ? a_off_hi : a_off;
    const unsigned wofs = so & 0xffffu;
    constexpr int NU = SHIFT ? KH : RS;  // pipeline units
    constexpr int NA = SHIFT ? KW : 1;   // weight fragments per unit
    u32x4 fa[2][NA], fq[2][2];
    auto fetch = [&](int u, int bsel) {
#pragma unroll
      for (int s = 0; s < NA; ++s) fa[bsel][s] = lds_ld16(a_base + wofs + (u * NA + s) * 64);
      fq[bsel][0] = lds_ld16(b_off[xb][0][u]);
      fq[bsel][1] = lds_ld16(b_off[xb][1][u]);
    };
    if constexpr (DMA) {
      // unit 0's weight fragments were read before the barrier that opened this slice
#pragma unroll
      for (int s = 0; s < NA; ++s) fa[0][s] = fa_next[s];
      fq[0][0] = lds_ld16(b_off[xb][0][0]);
      fq[0][1] = lds_ld16(b_off[xb][1][0]);
    } else {
      fetch(0, 0);
    }
    u32x2 tv[KX][4];
    if constexpr (DMA) {
#pragma unroll
      for (int k = 0; k < KX; ++k) {
        if (k == 0 || k * NT < units) {
#pragma unroll
          for (int j = 0; j < 4; ++j) tv[k][j] = raw_read(k, j, tst);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      if (u + 1 < NU) fetch(u + 1, (u + 1) & 1);
      if constexpr (DMA) {
#pragma unroll
        for (int kb = (NLB * u + NU - 1) / NU; kb < (NLB * (u + 1) + NU - 1) / NU; ++kb) issue_one(kb, ist);
      }
#pragma unroll
      for (int s = 0; s < NA; ++s) {
        const int p = (u * NA + s) & 1;
        acc[0][p] = E::mfma32(fa[u & 1][s], shl_rows_n(fq[u & 1][0], s), acc[0][p]);
        acc[1][p] = E::mfma32(fa[u & 1][s], shl_rows_n(fq[u & 1][1], s), acc[1][p]);
      }
      if constexpr (DMA) {
        if (u == NU - 1) prefetch_a(tst);  // the next slice sits in stage tst
        if (u == NU / 2) {
#pragma unroll
          for (int k = 0; k < KX; ++k) {
            if (k == 0 || k * NT < units) {
              u32x2 d[4];
              unit_pixels(tv[k], d);
              unit_store(k, txb, d);
            }
          }
        }
      }
    }
  };

  // ---- prologue: zero both transposed buffers (positions outside the image are never written), then the
  // first slice's activations ----
  for (int i = tid * 16; i < 2 * g.XTB; i += NT * 16)
    *reinterpret_cast<u32x4*>(lds + XT0 + i) = u32x4{0u, 0u, 0u, 0u};
  if constexpr (DMA) {
    // slices 0 and 1 are in (slice 0 is transposed now, slice 1 in the first iteration)
    wait_vm_asm<NST == 4 ? KL : 0>();
    __syncthreads();
    transpose(0, 0);
    prefetch_a(0);
  } else {
    issue_a(0);
    wait_a(std::integral_constant<int, 0>{});
    __syncthreads();
    write_a(0);
  }
  stage_barrier();

  // ---- main loop: slice sl multiplies from stage sl % NST and transposed buffer sl % 2 ----
  for (int s0 = 0; s0 < ns; s0 += UNR) {
#pragma unroll
    for (int su = 0; su < UNR; ++su) {
      if (s0 + su < ns) {
        const int st = su % NST, xb = su & 1;
        if constexpr (DMA) {
          slice(st, xb, (st + NST - 1) % NST, (st + 1) % NST, xb ^ 1);
          // the next iteration transposes slice sl+2: its loads (issued one iteration ago with NST = 4) are in
          wait_vm_asm<NST == 4 ? KL : 0>();
        } else {
          issue_a(s0 + su + 1);
#pragma unroll
          for (int kb = 0; kb < NLB; ++kb) issue_one(kb, (st + NST - 1) % NST);
          slice(st, xb, 0, 0, 0);
          // every MFMA of the slice issues before the wait below (they keep running while the wave waits)
          __builtin_amdgcn_sched_barrier(0);
          // this slice's activation loads are in, and with them (older) the weights of slice sl+1
          wait_a(std::integral_constant<int, NST >= 3 ? KBW : 0>{});
          write_a(xb ^ 1);
        }
        stage_barrier();
      }
    }
  }
  wait_vmcnt<0>();
  __syncthreads();

  // ---- epilogue: the two channel halves of each group meet in LDS; each wave finishes one group ----
  const f32x16 acc0 = acc[0][0] + acc[0][1], acc1 = acc[1][0] + acc[1][1];
  float* const red = reinterpret_cast<float*>(lds);
  float* const bias_s = red + NW * 1024;
  if (tid < kTO) bias_s[tid] = (bias != nullptr && o0 + tid < g.O) ? E::to_f32(bias[o0 + tid]) : 0.0f;
  {
    float* const dst = red + wave * 1024 + lane;
    if (hh == 0) {
      if (two) {
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[r * 64] = acc1[r];
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[r * 64] = acc0[r];
    }
  }
  __syncthreads();
  const int grp = 2 * pr + hh;
  if (grp >= NG) return;
  f32x16 accf = hh == 0 ? acc0 : acc1;
  {
    const float* const src = red + (wave ^ 1) * 1024 + lane;
#pragma unroll
    for (int r = 0; r < 16; ++r) accf[r] += src[r * 64];
  }
  const int f = grp * 32 + (lane & 31);
  const int orow = f >> g.lgOWP, ocol = f & owp_mask, oh = oh0 + orow;
  if (ocol >= g.OW || oh >= g.OH) return;
  const int ybase = (b * g.O + o0) * g.OHW + oh * g.OW + ocol;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int olr = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (o0 + olr >= g.O) continue;
    const int idx = ybase + olr * g.OHW;
    if (split == 1) {
      float v = accf[r] + bias_s[olr];
      if (g.relu) v = fmaxf(v, 0.0f);
      y[idx] = E::from_f32(v);
    } else {
      partial[static_cast<long long>(z) * g.Y + idx] = accf[r];
    }
  }
}

typedef void (*BandFn)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*, BandGeom, int);

constexpr int kDmaForms = kKlMax - kKlMin + 1;

struct BandConfig {
  gie_band_config info;
  int ng, nst, nw, nbw, kbw;
  BandFn dma[2][2][kDmaForms];  // [fp16, bf16][per-tap reads, row shifts][load blocks per wave - kKlMin]
  BandFn reg[2][2][kKuMax];     // [fp16, bf16][per-tap reads, row shifts][activation units per thread - 1]
};

// a DMA form exists for the load-block counts whose stages fit in LDS with two base registers
template <int NG, int NST, int KL>
constexpr bool dma_form_fits() {
  constexpr int sb = KL * 2 * ((NG + 1) / 2) * 1024;
  return NST >= 3 && (NST - 1) * sb < 2 * 65536 && NST * sb < kLdsLimit;
}
template <typename E, int KH, int KW, int NG, int NST, bool SHIFT, int K>
BandFn dma_fn() {
  if constexpr (dma_form_fits<NG, NST, K + kKlMin>()) return &band_kernel<E, KH, KW, NG, NST, K + kKlMin, true, SHIFT>;
  else return nullptr;
}
template <typename E, int KH, int KW, int NG, int NST, bool SHIFT, int... Ks>
void fill_dma(BandFn* out, std::integer_sequence<int, Ks...>) {
  ((out[Ks] = dma_fn<E, KH, KW, NG, NST, SHIFT, Ks>()), ...);
}
template <typename E, int KH, int KW, int NG, int NST, bool SHIFT, int... Ks>
void fill_reg(BandFn* out, std::integer_sequence<int, Ks...>) {
  ((out[Ks] = &band_kernel<E, KH, KW, NG, NST, Ks + 1, false, SHIFT>), ...);
}

template <typename E, int KH, int KW, int NG, int NST>
void fill_dtype(BandConfig& c, int d) {
  using D = std::make_integer_sequence<int, kDmaForms>;
  using U = std::make_integer_sequence<int, kKuMax>;
  fill_dma<E, KH, KW, NG, NST, false>(c.dma[d][0], D{});
  fill_dma<E, KH, KW, NG, NST, true>(c.dma[d][1], D{});
  fill_reg<E, KH, KW, NG, NST, false>(c.reg[d][0], U{});
  fill_reg<E, KH, KW, NG, NST, true>(c.reg[d][1], U{});
}

template <int KH, int KW, int NG, int NST>
BandConfig make_band(int version) {
  using S = BShape<KH, KW, NG, NST>;
  BandConfig c{};
  c.info.tile_m = kTO;
  c.info.tile_n = NG * 32;
  c.info.tile_k = kCS;
  c.info.kernel_h = KH;
  c.info.kernel_w = KW;
  c.info.threads = S::NT;
  c.info.stages = NST;
  c.info.version = version;
  c.ng = NG;
  c.nst = NST;
  c.nw = S::NW;
  c.nbw = S::NBW;
  c.kbw = S::KBW;
  fill_dtype<Fp16, KH, KW, NG, NST>(c, 0);
  fill_dtype<Bf16, KH, KW, NG, NST>(c, 1);
  return c;
}

const std::vector<BandConfig>& band_configs() {
  static const std::vector<BandConfig> t = [] {
    std::vector<BandConfig> v;
    //                KH KW NG NST
    v.push_back(make_band<3, 3, 7, 4>(2));
    v.push_back(make_band<3, 3, 8, 3>(2));
    return v;
  }();
  return t;
}

// The two ways a geometry can run: the DMA form (when the pointer and run alignment allow) and the register
// form (always, when its loads and LDS fit).
struct BandPlan {
  BandGeom g;
  bool shift;
  int dma_kl, dma_lds;  // 0 when the DMA form does not fit
  int reg_ku, reg_lds;  // 0 when the register form does not fit
};

int band_prepare(const BandConfig& c, const gie_conv_geom* gg, BandPlan* bp) {
  if (!gg) return GIE_HIP_EINVAL;
  if (gg->kernel_h != c.info.kernel_h || gg->kernel_w != c.info.kernel_w) return GIE_HIP_EUNSUPPORTED;
  BandGeom* g = &bp->g;
  *g = BandGeom{};
  g->B = gg->batch;
  g->C = gg->in_channels;
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
  if (g->B <= 0 || g->C <= 0 || g->H <= 0 || g->W <= 0 || g->O <= 0 || g->SH <= 0 || g->SW <= 0 || g->PH < 0 ||
      g->PW < 0 || g->OH <= 0 || g->OW <= 0)
    return GIE_HIP_EINVAL;
  const int KH = c.info.kernel_h, KW = c.info.kernel_w;
  g->S = (g->C + kCS - 1) / kCS;
  const long long hw = static_cast<long long>(g->H) * g->W, ohw = static_cast<long long>(g->OH) * g->OW;
  const long long xb = hw * g->B * g->C * 2, wbb = static_cast<long long>(g->O) * g->S * KH * KW * 64;
  const long long yn = ohw * g->B * g->O;
  // 32-bit offsets: channel indices run up to 32*S per image, so leave a slice of headroom past the tensor
  if (xb + hw * 2 * kCS >= 0x7fffffffLL || wbb >= 0x7fffffffLL || yn >= 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  g->HW = int(hw);
  g->OHW = int(ohw);
  g->Y = int(yn);
  g->x_bytes = int(xb);
  g->wb_bytes = int(wbb);
  int lg = 0;
  while ((1 << lg) < g->OW) ++lg;
  if ((c.ng * 32) % (1 << lg) != 0) return GIE_HIP_EUNSUPPORTED;  // a band is whole padded rows
  g->lgOWP = lg;
  const int owp = 1 << lg;
  g->R = c.ng * 32 / owp;
  g->n_bands = (g->OH + g->R - 1) / g->R;
  g->IR = (g->R - 1) * g->SH + KH;
  g->IWP = g->W + 2 * g->PW;
  g->inv_w = 1.0f / float(g->W);
  bp->shift = owp == 16 && g->SW == 1 && g->OW + KW - 1 <= 16 && KW <= 8;
  // positions the B reads reach: the real rows, plus the dropped columns' reach past the last row (the row-shift
  // form reads tap column 0 only)
  const long long tail = bp->shift ? owp - 1 : static_cast<long long>(owp - 1) * g->SW + KW - 1;
  const long long reach = std::max<long long>(static_cast<long long>(g->IR) * g->IWP - 1,
                                              static_cast<long long>(g->IR - 1) * g->IWP + tail);
  const long long xtb = (reach + 1 + 3) / 4 * 4 * 64;
  if (xtb > kLdsLimit) return GIE_HIP_EUNSUPPORTED;
  g->XTB = int(xtb);
  const long long run = static_cast<long long>(std::min(g->IR, g->H)) * g->W;  // longest channel run
  if (run >= (1 << 21)) return GIE_HIP_EUNSUPPORTED;                            // exact fast divisions
  const long long units = 8 * ((run + 3) / 4);                                  // transposition units
  const long long nt = c.nw * 64;
  const long long epi = static_cast<long long>(c.nw) * 4096 + kTO * 4;
  // register form
  const long long ku = (units + nt - 1) / nt;
  const long long reg_lds = std::max<long long>(c.nst * (c.kbw * c.nw * 1024LL) + 2 * xtb, epi);
  bp->reg_ku = (ku <= kKuMax && reg_lds <= kLdsLimit) ? int(ku) : 0;
  bp->reg_lds = bp->reg_ku ? int(reg_lds) : 0;
  // DMA form: each channel's run as 16-byte chunks from the 16-byte boundary at or below its start
  // (+8: the last pixel quad of a run may read up to 6 bytes past it)
  const long long nch = (8 + 2 * run + 8 + 15) / 16;
  const long long nbx = (kCS * nch + 63) / 64;
  const long long kl = std::max<long long>((c.nbw + nbx + c.nw - 1) / c.nw, kKlMin);
  const long long dma_lds = std::max<long long>(c.nst * kl * c.nw * 1024LL + 2 * xtb, epi);
  const bool dma_fits = c.nst >= 3 && kl <= kKlMax && units <= kKxMax * nt && dma_lds <= kLdsLimit &&
                        (c.nst - 1) * kl * c.nw * 1024LL < 2 * 65536;
  bp->dma_kl = dma_fits ? int(kl) : 0;
  bp->dma_lds = dma_fits ? int(dma_lds) : 0;
  g->NCH = int(nch);
  g->NBX = int(nbx);
  g->inv_nch = 1.0f / float(nch);
  if (!bp->reg_ku && !bp->dma_kl) return GIE_HIP_EUNSUPPORTED;
  const long long blocks = static_cast<long long>((g->O + kTO - 1) / kTO) * g->B * g->n_bands;
  if (blocks > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  return GIE_HIP_OK;
}

// The DMA form reads 16-byte chunks of each channel's run: x 16-byte aligned with a 16-byte multiple of bytes
// (every chunk that holds data lies inside x), and every run starting on an 8-byte boundary.
bool dma_form_ok(const BandGeom& g, const void* x) {
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || g.x_bytes % 16 != 0 || g.HW % 4 != 0) return false;
  for (int band = 0; band < g.n_bands; ++band) {
    const int ih_lo = std::max(band * g.R * g.SH - g.PH, 0);
    if ((static_cast<long long>(ih_lo) * g.W) % 4 != 0) return false;
  }
  return true;
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_band_config_count(void) { return int(band_configs().size()); }

extern "C" int gie_hip_band_config_get(int index, gie_band_config* out) {
  if (index < 0 || index >= int(band_configs().size()) || !out) return GIE_HIP_EINVAL;
  *out = band_configs()[size_t(index)].info;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_band_check(int config, const gie_conv_geom* g, int* lds_bytes) {
  if (config < 0 || config >= int(band_configs().size()) || !g) return GIE_HIP_EINVAL;
  BandPlan bp;
  const int rc = band_prepare(band_configs()[size_t(config)], g, &bp);
  if (rc == GIE_HIP_OK && lds_bytes) *lds_bytes = std::max(bp.dma_lds, bp.reg_lds);
  return rc;
}

extern "C" int gie_hip_conv_band(int config, int dtype, const gie_conv_geom* gg, const void* x, const void* wb,
                                 const void* bias, void* y, float* partial, int split, void* stream) {
  if (config < 0 || config >= int(band_configs().size()) || !gg || !x || !wb) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if (split < 1 || split > 64) return GIE_HIP_EINVAL;
  if (split == 1 && !y) return GIE_HIP_EINVAL;
  if (split > 1 && (!partial || (reinterpret_cast<uintptr_t>(partial) & 15u) != 0)) return GIE_HIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(x) & 1u) || (reinterpret_cast<uintptr_t>(wb) & 15u)) return GIE_HIP_EINVAL;
  if (bias && (reinterpret_cast<uintptr_t>(bias) & 1u)) return GIE_HIP_EINVAL;
  if (y && (reinterpret_cast<uintptr_t>(y) & 1u)) return GIE_HIP_EINVAL;
  const BandConfig& c = band_configs()[size_t(config)];
  BandPlan bp;
  if (int rc = band_prepare(c, gg, &bp)) return rc;
  const BandGeom& g0 = bp.g;
  if (split > g0.S) return GIE_HIP_EUNSUPPORTED;
  if (split > 1 && static_cast<long long>(split) * g0.Y >= 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  const int d = dtype == GIE_HIP_BF16 ? 1 : 0, sh = bp.shift ? 1 : 0;
  BandGeom g = g0;
  BandFn fn = nullptr;
  int lds = 0;
  if (bp.dma_kl && dma_form_ok(g, x) && c.dma[d][sh][bp.dma_kl - kKlMin]) {
    fn = c.dma[d][sh][bp.dma_kl - kKlMin];
    lds = bp.dma_lds;
  } else if (bp.reg_ku) {
    fn = c.reg[d][sh][bp.reg_ku - 1];
    lds = bp.reg_lds;
  }
  if (!fn) return GIE_HIP_EUNSUPPORTED;
  if (int rc = set_lds_limit(reinterpret_cast<const void*>(fn), lds)) return rc;
  const long long blocks = static_cast<long long>((g.O + kTO - 1) / kTO) * g.B * g.n_bands;
  const long long n_ot = (g.O + kTO - 1) / kTO;
  if (n_ot > 65535) return GIE_HIP_EUNSUPPORTED;
  hipLaunchKernelGGL(fn, dim3(unsigned(blocks / n_ot), unsigned(n_ot), unsigned(split)), dim3(c.info.threads), lds,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x),
                     static_cast<const uint16_t*>(wb), static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y),
                     partial, g, split);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
