// Stem convolution (7x7 filter, stride 2, padding 3, in_channels <= 4) straight from NCHW on gfx950 matrix cores
// (v_mfma_f32_32x32x16_{f16,bf16}, FP32 accumulation): no repack, no padded channels, one launch.
//
// The generic implicit GEMM pads C to 8 channels per tap (K = 49 * 8 = 392 for C = 3); the stem's reduction is
// only C * 49 = 147 long and the layer is bound by writing Y (64 filters per pixel), so this kernel keeps the
// reduction short and spends its effort on the stores.
//   * K order: one group of 8 per (channel c, filter row kh): a zero, then the filter columns kw = 0 .. 6. With
//     stride 2 the 7 input pixels of one (c, kh) group are the input columns 2*ow - 3 .. 2*ow + 3, so k = kw + 1
//     meets column 2*ow - 4 + k: the group's 16-byte pixel operand is the 4 dwords of the row that start at column
//     2*ow - 4 as they lie in LDS, with their first half (column 2*ow - 4, weight zero) cleared by one AND so that
//     an Inf or NaN outside the window cannot reach the sum. 7*C groups plus one bias group (weights = bias, pixels
//     = 1.0 at its first k), in k-steps of two groups: K = 176 for C = 3 (147 useful).
//   * A workgroup (one per CU, persistent) owns 64 filters and walks tiles of R = 4 (2 for wide rows) output rows of
//     one image (R * out_w pixels, contiguous in each output plane). The tile's 2R+5 input rows per channel sit in LDS with 4 zero
//     dwords on each side (the horizontal padding); rows above or below the image are loaded as zeros. Wave 7
//     streams rows: tile i+2's rows go straight into the third of three row buffers (buffer_load ... lds) while
//     waves 0..6 multiply tile i (tile 0's rows come from waves 0..6 at the start, tile 1's from wave 7). Waves 0..6 hold the 64 filters' operands in registers (2 x 32 columns x K);
//     per 32-pixel block: two ds_read2_b32 and one AND per k-step, two MFMA chains. One barrier per tile.
//   * MFMA roles: rows = pixels, columns = filters, so each lane's accumulators hold 4-pixel runs of one filter.
//     Epilogue: ReLU, RNE rounding (the order of the reference's apply_epilogue,
//     src/kernels/fused_epilogue.cuh:11-16), then the wave's two adjacent 32-pixel blocks staged in LDS as one
//     64-filter x 64-pixel tile and written by 16-byte stores, every 8 lanes one 128-byte run of a filter's output
//     row (whole lines: a tile starts on a 128-byte boundary of each plane when R * out_w * 2 and the plane size are
//     multiples of 128). Where the LDS cannot hold an 8 KiB tile per wave, one block at a time in 64-byte runs.
//   * Grid: one 8-wave workgroup per CU; tiles are split into 8 contiguous ranges, one per XCD (blockIdx mod 8),
//     so the input rows shared by neighbouring tiles are read into one L2.
#include <algorithm>

#include "lds_pipe.h"

namespace gie_hip {
namespace {

constexpr int kStNT = 512;             // threads per workgroup: waves 0..6 multiply, wave 7 streams rows
constexpr int kStCW = 7;               // multiplying waves
constexpr int kStLoader = 7;           // the row-streaming wave
constexpr int kStBufs = 3;             // row buffers: tile i read, i+1 landed, i+2 in flight
constexpr int kStPad = 4;              // zero dwords left of each row (and at least 2 to its right)
constexpr int kStLdsMax = 160 * 1024;

struct StemGeom {
  int N, C, H, W, O, OH, OW;
  int R;          // output rows per tile (4, or 2 for rows too wide for LDS)
  int n_rt;       // tiles per image
  int n_tiles;    // tiles per filter group
  int NB;         // 32-pixel blocks per tile
  int G;          // workgroups per filter group (a multiple of 8)
  int per_xcd;    // tiles per XCD range
  int CPR;        // 16-byte chunks per input row (in_w / 8 <= 64)
  int RS;         // LDS row stride in dwords: in_w / 2 + 8
  int buf_bytes;  // one row buffer: C * WR * RS * 4
  int rows_off;   // LDS byte offset of the row buffers (after the MFMA operands)
  int tile_off;   // LDS byte offset of the multiplying waves' output tiles (8 KiB each, 4 KiB without `wide`)
  int wide;       // 128-byte output runs: each wave takes two adjacent 32-pixel blocks (host-side choice)
  int x_bytes, y_bytes;
};

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

// two FP32 sums -> optional ReLU -> two rounded 16-bit values in one register; for FP16 the ReLU is one
// v_pk_max_f16 on the rounded pair (rounding is monotonic and keeps the sign, so max(round(v), 0) ==
// round(max(v, 0))), for BF16 the FP32 max before rounding
template <typename E, bool RELU>
__device__ __forceinline__ uint32_t relu2(float v0, float v1) {
  if constexpr (RELU && E::kDtype == GIE_HIP_FP16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t,
                              __builtin_elementwise_max(__builtin_bit_cast(h2, pack2<E>(v0, v1)), (h2){0, 0}));
  } else {
    if (RELU) v0 = fmaxf(v0, 0.0f), v1 = fmaxf(v1, 0.0f);
    return pack2<E>(v0, v1);
  }
}

template <typename E>
constexpr uint32_t one_bits() {
  return E::kDtype == GIE_HIP_FP16 ? 0x3C00u : 0x3F80u;
}

template <typename E, int C, int R, bool RELU, bool WIDE>
__global__ __launch_bounds__(kStNT) void stem_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                    StemGeom g) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int NG = 7 * C;             // (channel, filter row) groups
  constexpr int KS = (NG + 2) / 2;      // k-steps: NG groups + the bias group, two groups per step
  constexpr int FW = C * 49;            // weights per filter
  constexpr int WR = 2 * R + 5;         // input rows per tile and channel
  constexpr int NROW = C * WR;          // input rows per tile
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = lane >> 5, col = lane & 31;
  const int og = blockIdx.x / g.G, L = blockIdx.x - og * g.G;
  const int f0 = og * 64;
  const int nf = min(64, g.O - f0);
  auto rows = [&](int i) { return smem + g.rows_off + (i % kStBufs) * g.buf_bytes; };

  // ---- tiles of this workgroup: XCD range, then every (G/8)-th tile of it
  const int xcd = L & 7, step = g.G >> 3;
  const int t0 = xcd * g.per_xcd + (L >> 3);
  const int t_end = min(g.n_tiles, (xcd + 1) * g.per_xcd);
  const int n_my = t0 < t_end ? (t_end - t0 + step - 1) / step : 0;
  const int row_bytes = g.W * 2;
  const size_t y_plane = size_t(g.OH) * g.OW;
  const v4i xr = make_vsharp(x, g.x_bytes);
  const v4i yr = make_vsharp(y, g.y_bytes);

  // the rows of tile i into row buffer i % 3 (streaming wave): one load per row, lanes < in_w / 8 active (an
  // inactive lane writes nothing), rows above or below the image read as zeros
  auto load_rows = [&](int i) {
    const int t = t0 + i * step;
    const int n = t / g.n_rt, oh0 = (t - n * g.n_rt) * R;
    unsigned char* dst = rows(i) + kStPad * 4;
    if (lane < g.CPR) {
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int lr = 0; lr < WR; ++lr) {
          const int ih = 2 * oh0 - 3 + lr;
          const int voff = ih >= 0 && ih < g.H ? ((n * C + c) * g.H + ih) * row_bytes + lane * 16 : kOut;
          dma16(xr, lds_addr(dst + (c * WR + lr) * g.RS * 4), voff);
        }
    }
  };
  // tile 0's rows come from the multiplying waves (row q to wave q % 7, issued before their weight loads and waited
  // with them), tile 1's from the streaming wave, so the first tile's 39 loads are not issued by one wave
  if (wave == kStLoader) {
    if (n_my > 1) load_rows(1);
  } else if (n_my > 0 && lane < g.CPR) {
    const int n = t0 / g.n_rt, oh0 = (t0 - n * g.n_rt) * R;
    unsigned char* dst = rows(0) + kStPad * 4;
    for (int q = wave; q < NROW; q += kStCW) {
      const int c = q / WR, lr = q - c * WR;
      const int ih = 2 * oh0 - 3 + lr;
      const int voff = ih >= 0 && ih < g.H ? ((n * C + c) * g.H + ih) * row_bytes + lane * 16 : kOut;
      dma16(xr, lds_addr(dst + (c * WR + lr) * g.RS * 4), voff);
    }
  }
  // the horizontal padding of every row buffer: zero once, never written again
  for (int idx = tid; idx < kStBufs * NROW * 8; idx += kStNT) {
    const int rw = idx >> 3, d = idx & 7;
    const int dw = d < kStPad ? d : kStPad + g.W / 2 + (d - kStPad);
    reinterpret_cast<uint32_t*>(smem + g.rows_off)[rw * g.RS + dw] = 0u;
  }

  // ---- the MFMA operands of the workgroup's 64 filters, built straight from OIHW: operand (filter f, k-step s,
  // half h) is group grp = 2s + h, the 7 taps of one filter row (channel grp / 7, row grp % 7), which are 7
  // consecutive halves of the filter's OIHW run starting at element 7 grp. One 16-byte load from the 4-byte boundary
  // at or below them and 16-bit shifts put them in the order (0, kw 0, ..., kw 6): k = kw + 1 meets input column
  // 2 ow - 4 + k, so the pixel operand is the row's 16 bytes from column 2 ow - 4 as they lie in LDS. The bias group
  // holds (bias, 0, ...); groups past it are zero. Stored [f][s][h] x 16 bytes at the start of LDS.
  u32x4* frag = reinterpret_cast<u32x4*>(smem);
  if (wave != kStLoader) {  // (the streaming wave keeps its vector-memory counter to the row loads)
    constexpr int kMT = kStCW * 64;                         // threads of the multiplying waves
    constexpr int kItems = 64 * KS * 2;                     // operands
    constexpr int kPer = (kItems + kMT - 1) / kMT;          // operands per thread
    const v4i wrs = make_vsharp(w, g.O * FW * 2);           // dwords past w read as zeros
    u32x4 v[kPer];
    uint32_t sh[kPer], bv[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {  // every load in flight before the first is used
      const int idx = tid + k * kMT, f = idx / (2 * KS), grp = idx - f * 2 * KS;
      const bool real = idx < kItems && f < nf;
      const int e = (f0 + f) * FW + 7 * grp;
      v[k] = load16_asm(wrs, real && grp < NG ? (2 * e) & ~3 : kOut);
      sh[k] = uint32_t(e & 1) << 4;
      bv[k] = real && grp == NG && bias != nullptr ? uint32_t(bias[f0 + f]) : 0u;
    }
    wait_vm<0>();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int idx = tid + k * kMT, f = idx / (2 * KS), grp = idx - f * 2 * KS;
      if (idx >= kItems) break;
      touch_v(v[k]);
      const u32x4 d = v[k];
      const uint32_t q0 = __builtin_amdgcn_alignbit(d.y, d.x, sh[k]), q1 = __builtin_amdgcn_alignbit(d.z, d.y, sh[k]);
      const uint32_t q2 = __builtin_amdgcn_alignbit(d.w, d.z, sh[k]), q3 = __builtin_amdgcn_alignbit(0u, d.w, sh[k]);
      // q0..q3 = halves (p0, p1), (p2, p3), (p4, p5), (p6, -): the operand is (0, p0), (p1, p2), (p3, p4), (p5, p6)
      u32x4 op = {q0 << 16, __builtin_amdgcn_alignbit(q1, q0, 16), __builtin_amdgcn_alignbit(q2, q1, 16),
                  __builtin_amdgcn_alignbit(q3, q2, 16)};
      if (grp >= NG || f >= nf) op = u32x4{bv[k], 0u, 0u, 0u};  // the bias group, or zero
      frag[idx] = op;
    }
  }
  __syncthreads();

  if (wave == kStLoader) {
    // ---- streaming wave: before the barrier that ends tile i, tile i+1's rows must have landed; tile i+2's are
    // issued first and may stay in flight (this wave issues no other vector-memory operation in the loop)
    stage_barrier();  // B0 (tile 0's rows: the multiplying waves waited for them; tile 1's may be in flight)
    for (int i = 0; i < n_my; ++i) {
      if (i + 2 < n_my) {
        load_rows(i + 2);
        wait_vm<NROW>();  // the NROW loads just issued may stay in flight
      } else {
        wait_vm<0>();
      }
      stage_barrier();
    }
    return;
  }

  u32x4 wa[2][KS];
#pragma unroll
  for (int fh = 0; fh < 2; ++fh)
#pragma unroll
    for (int s = 0; s < KS; ++s) wa[fh][s] = frag[((fh * 32 + col) * KS + s) * 2 + hi];
  // Row each k-step reads, from the lane's (output row 0, column 0) position: group 2s's row r0(s) (a constant per
  // step, times the row stride: uniform), plus for the hi half (group 2s + 1) one row further, or WR - 6 rows (the
  // next channel's first filter row) when group 2s is a channel's last filter row. The bias and zero groups read
  // group 2s's row or group 0's (any valid address: replaced below). Two per-lane displacements instead of one
  // offset register per step.
  const int rs4 = g.RS * 4;
  const int h_next = hi * rs4, h_chan = hi * (WR - 6) * rs4;
  stage_barrier();  // tile 0's rows are in

  // ---- multiplying waves: 32-pixel blocks of tile i from row buffer i % 3, two at a time (below)
  const int npix = R * g.OW;
  const float inv_ow = 1.0f / float(g.OW);
  // Output tile of this wave in LDS.
  // 64-byte runs (!WIDE, one 32-pixel block at a time): row r (64 bytes) holds filter f0 + r; its 8-byte granule q sits
  // at q ^ (2 * ((r / 4) & 3)). Writes: lane (hi, col) puts pixels 8a + 4hi .. +3 of filter 32fh + col into granule
  // 2a + hi of row 32fh + col. Reads: read t of lane l covers row 16t + l/4, 16-byte segment l%4 (stored at
  // segment (l%4) ^ ((l/16) & 3)).
  // 128-byte runs (WIDE, two adjacent blocks): row r (128 bytes) holds filter f0 + r for the pair's 64 pixels; its
  // 16-byte segment s (pixels 8s .. 8s+7) sits at s ^ ((r / 2) & 7). Writes: lane (hi, col) puts pixels 8a + 4hi .. +3
  // of block bh into the 8-byte half hi of segment 4bh + a of row 32fh + col (2-way bank conflict, as above). Reads:
  // read t of lane l covers row 8t + l/8, segment l%8, stored at (l%8) ^ ((l/16) + 4 (t%2)) (conflict-free).
  constexpr unsigned kTB = WIDE ? 8192u : 4096u;
  typedef __attribute__((address_space(3))) u32x2 lds_u32x2_t;
  typedef __attribute__((address_space(3))) const u32x4 lds_cu32x4_t;
  const unsigned stg = lds_addr(smem + g.tile_off) + unsigned(wave) * kTB;
  constexpr int NQ = WIDE ? 8 : 4;  // write pointers: one per (block, a) segment
  lds_u32x2_t* w_q[NQ];
  lds_cu32x4_t* r_base[WIDE ? 2 : 1];
  if constexpr (WIDE) {
    const unsigned m = (unsigned(col) >> 1) & 7u;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      w_q[q] = reinterpret_cast<lds_u32x2_t*>(
          size_t(stg + unsigned(col) * 128u + ((unsigned(q) ^ m) << 4) + (unsigned(hi) << 3)));
#pragma unroll
    for (int par = 0; par < 2; ++par)
      r_base[par] = reinterpret_cast<lds_cu32x4_t*>(size_t(
          stg + (unsigned(lane) >> 3) * 128u + (((unsigned(lane) & 7u) ^ ((unsigned(lane) >> 4) + 4u * par)) << 4)));
  } else {
#pragma unroll
    for (int a = 0; a < 4; ++a)
      w_q[a] = reinterpret_cast<lds_u32x2_t*>(size_t(
          stg + unsigned(col) * 64u + (((unsigned(a) ^ ((unsigned(lane) >> 2) & 3u)) << 1 | unsigned(hi)) << 3)));
    r_base[0] = reinterpret_cast<lds_cu32x4_t*>(
        size_t(stg + (unsigned(lane) >> 2) * 64u + (((unsigned(lane) & 3u) ^ ((unsigned(lane) >> 4) & 3u)) << 4)));
  }
  constexpr int NS = WIDE ? 8 : 4;  // store instructions per tile of the wave: rows per read, 16 (64-byte) or 8
  int f_off[NS];                    // byte offset of the filter plane of each read's row
  bool f_ok[NS];
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    const int f = f0 + (WIDE ? 8 * t + (lane >> 3) : 16 * t + (lane >> 2));
    f_ok[t] = f < g.O;
    f_off[t] = int(size_t(f_ok[t] ? f : 0) * y_plane * 2);
  }
  for (int i = 0; i < n_my; ++i) {
    const int t = t0 + i * step;
    const int n = t / g.n_rt, oh0 = (t - n * g.n_rt) * R;
    const unsigned char* rb = rows(i);
    const int p_end = min(npix, (g.OH - oh0) * g.OW);  // pixels of the tile inside the image
    const int y_tile = int((size_t(n) * g.O * y_plane + size_t(oh0) * g.OW) * 2);  // byte offset of (n, 0, oh0, 0)
    // row dwords ow-2 .. ow+1 (input columns 2*ow-4 .. 2*ow+3) of every k-step's row: padded dwords ow+2 .. ow+5
    auto load = [&](int blk, uint32_t (&d)[KS][4]) {
      const int p = blk * 32 + col;
      const int pc = p < npix ? p : 0;
      const int r = fdiv(pc, g.OW, inv_ow), ow = pc - r * g.OW;
      const unsigned char* bp = rb + (2 * r * g.RS + ow + 2) * 4;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int g0 = 2 * s;
        const int r0 = g0 < NG ? (g0 / 7) * WR + g0 % 7 : 0;
        const int dl = g0 + 1 < NG ? (g0 % 7 == 6 ? h_chan : h_next) : 0;
        const uint32_t* q = reinterpret_cast<const uint32_t*>(bp + r0 * rs4 + dl);
        d[s][0] = q[0], d[s][1] = q[1], d[s][2] = q[2], d[s][3] = q[3];
      }
    };
    auto multiply = [&](const uint32_t (&d)[KS][4], f32x16& acc0, f32x16& acc1) {
      acc0 = f32x16{0}, acc1 = f32x16{0};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        // halves h0..h7 = input columns 2*ow-4 .. 2*ow+3 meet weights (0, kw 0, ..., kw 6): the operand is the
        // window as read, h0 zeroed (its weight is zero, but an Inf or NaN there would still reach the sum)
        u32x4 b = {d[s][0] & 0xffff0000u, d[s][1], d[s][2], d[s][3]};
        const int grp = 2 * s + hi;
        if (2 * s + 1 >= NG) {  // this step holds the bias group (and possibly the zero group)
          if (grp == NG) b = u32x4{one_bits<E>(), 0u, 0u, 0u};
          else if (grp > NG) b = u32x4{0u, 0u, 0u, 0u};
        }
        acc0 = E::mfma32(b, wa[0][s], acc0);  // rows: pixels; columns: filters
        acc1 = E::mfma32(b, wa[1][s], acc1);
      }
    };
    // epilogue: lane (hi, col) holds filter col of each 32-filter half and pixels 8a + 4hi + (0..3), a = 0..3.
    // ReLU and the rounding in registers, then the wave's 64 x 32 tile goes through its own 4 KiB of LDS so that
    // every 4 lanes write one 64-byte run of a filter's output row (16 runs per store instruction; measured
    // faster than 16-byte runs of 32 filters per instruction straight from the registers). The stores are
    // device-scope (store16_wt): 24.5 us per launch on the 64 x 3 x 224 x 224 stem against 25.7 with stores that
    // leave dirty L2 lines to be written back at the end of the launch.
    // the rounded 64 x 32 tile of block half bh (WIDE) or of the block into the wave's LDS tile
    auto stage = [&](int bh, const f32x16& acc0, const f32x16& acc1) {
#pragma unroll
      for (int fh = 0; fh < 2; ++fh) {
        const f32x16& acc = fh ? acc1 : acc0;
#pragma unroll
        for (int a = 0; a < 4; ++a)
          w_q[WIDE ? 4 * bh + a : a][fh * (WIDE ? 512 : 256)] =  // + 32 rows for the second 32-filter half
              u32x2{relu2<E, RELU>(acc[4 * a], acc[4 * a + 1]), relu2<E, RELU>(acc[4 * a + 2], acc[4 * a + 3])};
      }
      // the tile is written as 8-byte and read as 16-byte vectors: keep the compiler from reordering them (the
      // wave's LDS accesses complete in issue order)
      asm volatile("" ::: "memory");
    };
    // the staged tile to y: 16-byte stores, every 4 (8 when WIDE) lanes one 64- (128-) byte run of a filter's output
    // row; px0 = the tile's first pixel. The stores are device-scope (store16_wt): 24.5 us per launch on the
    // 64 x 3 x 224 x 224 stem against 25.7 with stores that leave dirty L2 lines to be written back at the end of the
    // launch (64-byte runs). Runs of 128 bytes, so each store writes whole lines instead of halves whose other half
    // comes from another wave's block: 24.96 against 25.79 us (same process, 16 alternating batches).
    auto flush = [&](int px0) {
      u32x4 v[NS];
#pragma unroll
      for (int t = 0; t < NS; ++t) v[t] = WIDE ? r_base[t & 1][t * 64] : r_base[0][t * 64];  // + 1 KiB per read
      const int p0 = px0 + 8 * (lane & (WIDE ? 7 : 3));  // the lane's 8 pixels of one output row (out_w % 8 == 0)
#pragma unroll
      for (int t = 0; t < NS; ++t) {
        const int voff = p0 < p_end && f_ok[t] ? y_tile + f_off[t] + p0 * 2 : kOut;
        store16_wt(yr, voff, v[t]);
      }
    };
    if constexpr (WIDE) {
      // wave w takes the block pairs (2p, 2p + 1), p = w, w + 7, ...: the second block's rows are read before the
      // first block's tile is staged; both leave together as 128-byte runs
      for (int pk = wave; 2 * pk < g.NB; pk += kStCW) {
        const int ba = 2 * pk, bb = ba + 1;
        uint32_t d[KS][4];
        f32x16 acc0, acc1;
        load(ba, d);
        multiply(d, acc0, acc1);
        if (bb < g.NB) {
          load(bb, d);
          stage(0, acc0, acc1);
          multiply(d, acc0, acc1);
          stage(1, acc0, acc1);
        } else {
          stage(0, acc0, acc1);  // the second half's pixels are past the tile: never stored
        }
        flush(ba * 32);
      }
    } else {
      // blocks in pairs (wave, wave + 7), (wave + 14, wave + 21), ...: the second block's rows are read before the
      // first block's stores are issued
      for (int ba = wave; ba < g.NB; ba += 2 * kStCW) {
        const int bb = ba + kStCW;
        uint32_t d[KS][4];
        f32x16 acc0, acc1;
        load(ba, d);
        multiply(d, acc0, acc1);
        if (bb < g.NB) {
          load(bb, d);
          stage(0, acc0, acc1);
          flush(ba * 32);
          multiply(d, acc0, acc1);
          stage(0, acc0, acc1);
          flush(bb * 32);
        } else {
          stage(0, acc0, acc1);
          flush(ba * 32);
        }
      }
    }
    stage_barrier();  // tile i's rows are no longer read; tile i+1's have landed
  }
}

// Geometry of a stem launch; GIE_HIP_EUNSUPPORTED when the problem is not one this kernel runs. max_r caps the
// output rows per tile (4, or 2 for a variant whose 4-row form does not fit the register file).
int stem_prepare(const gie_conv_geom* gg, int cus, StemGeom* g, int* lds, int max_r = 4) {
  if (!gg) return GIE_HIP_EINVAL;
  if (gg->kernel_h != 7 || gg->kernel_w != 7 || gg->stride_h != 2 || gg->stride_w != 2 || gg->pad_h != 3 ||
      gg->pad_w != 3)
    return GIE_HIP_EUNSUPPORTED;
  if (gg->in_channels < 1 || gg->in_channels > 4 || gg->batch < 1 || gg->out_channels < 1 || gg->in_h < 1 ||
      gg->in_w < 16 || gg->in_w % 16 != 0 || gg->in_w > 512)
    return GIE_HIP_EUNSUPPORTED;
  if (gg->out_h != (gg->in_h - 1) / 2 + 1 || gg->out_w != gg->in_w / 2) return GIE_HIP_EINVAL;
  const long long nx = 1LL * gg->batch * gg->in_channels * gg->in_h * gg->in_w;
  const long long ny = 1LL * gg->batch * gg->out_channels * gg->out_h * gg->out_w;
  if (2 * nx >= (1LL << 31) || 2 * ny >= (1LL << 31)) return GIE_HIP_EUNSUPPORTED;  // 32-bit byte offsets
  g->N = gg->batch, g->C = gg->in_channels, g->H = gg->in_h, g->W = gg->in_w, g->O = gg->out_channels;
  g->OH = gg->out_h, g->OW = gg->out_w;
  g->CPR = g->W / 8;
  g->RS = g->W / 2 + 2 * kStPad;
  const int ks = (7 * g->C + 2) / 2;
  g->rows_off = 64 * ks * 2 * 16;  // the MFMA operands
  int R = 0;
  for (int r : {4, 2})
    if (r <= max_r && g->rows_off + kStBufs * g->C * (2 * r + 5) * g->RS * 4 + kStCW * 4096 <= kStLdsMax) {
      R = r;
      break;
    }
  if (R == 0) return GIE_HIP_EUNSUPPORTED;
  g->R = R;
  g->n_rt = (g->OH + R - 1) / R;
  g->n_tiles = g->N * g->n_rt;
  g->NB = (R * g->OW + 31) / 32;
  g->G = std::max(8, std::min((g->n_tiles + 7) / 8 * 8, cus / 8 * 8));
  g->per_xcd = (g->n_tiles + 7) / 8;
  g->buf_bytes = g->C * (2 * R + 5) * g->RS * 4;
  g->x_bytes = int(2 * nx);
  g->y_bytes = int(2 * ny);
  const long long grid = 1LL * g->G * ((g->O + 63) / 64);
  if (grid >= (1LL << 31)) return GIE_HIP_EUNSUPPORTED;
  g->tile_off = g->rows_off + kStBufs * g->buf_bytes;
  // 128-byte output runs where the LDS holds an 8 KiB tile per multiplying wave
  g->wide = g->tile_off + kStCW * 8192 <= kStLdsMax ? 1 : 0;
  if (lds) *lds = g->tile_off + kStCW * (g->wide ? 8192 : 4096);
  return GIE_HIP_OK;
}

using StemFn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, StemGeom);

// BF16 with four channels and ReLU runs 2-row tiles: its 4-row form needs more than the 256 registers a wave has at
// two waves per SIMD, and a spill would add scratch traffic to the vector-memory counter the row-streaming wave
// counts. That form is never instantiated.
constexpr bool stem_two_rows_only(bool bf16, int c, bool relu) { return bf16 && c == 4 && relu; }

template <typename E, int R, bool RELU, bool WIDE>
StemFn stem_fn(int c) {
  switch (c) {
    case 1: return &stem_kernel<E, 1, R, RELU, WIDE>;
    case 2: return &stem_kernel<E, 2, R, RELU, WIDE>;
    case 3: return &stem_kernel<E, 3, R, RELU, WIDE>;
    default:
      if constexpr (R == 4 && stem_two_rows_only(E::kDtype == GIE_HIP_BF16, 4, RELU)) return nullptr;
      else return &stem_kernel<E, 4, R, RELU, WIDE>;
  }
}

template <typename E, bool WIDE>
StemFn stem_fn(int c, int r, bool relu) {
  if (r == 4) return relu ? stem_fn<E, 4, true, WIDE>(c) : stem_fn<E, 4, false, WIDE>(c);
  return relu ? stem_fn<E, 2, true, WIDE>(c) : stem_fn<E, 2, false, WIDE>(c);
}

template <typename E>
StemFn stem_fn(int c, int r, bool relu, bool wide) {
  return wide ? stem_fn<E, true>(c, r, relu) : stem_fn<E, false>(c, r, relu);
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_stem_check(const gie_conv_geom* g, int* lds_bytes) {
  StemGeom sg;
  return stem_prepare(g, 256, &sg, lds_bytes);
}

extern "C" int gie_hip_conv_stem(int dtype, const gie_conv_geom* gg, const void* x, const void* w, const void* bias,
                                 void* y, void* stream) {
  if (!gg || !x || !w || !y) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if (bias && (reinterpret_cast<uintptr_t>(bias) & 1u)) return GIE_HIP_EINVAL;
  StemGeom g;
  int lds = 0;
  const bool bf = dtype == GIE_HIP_BF16;
  const int max_r = stem_two_rows_only(bf, gg->in_channels, gg->relu != 0) ? 2 : 4;
  if (int rc = stem_prepare(gg, current_device_cus(), &g, &lds, max_r)) return rc;
  // 16-byte input row and weight loads, 16-byte output stores
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(w) & 15u) ||
      (reinterpret_cast<uintptr_t>(y) & 15u))
    return GIE_HIP_EUNSUPPORTED;
  const StemFn fn = bf ? stem_fn<Bf16>(g.C, g.R, gg->relu != 0, g.wide != 0)
                       : stem_fn<Fp16>(g.C, g.R, gg->relu != 0, g.wide != 0);
  if (fn == nullptr) return GIE_HIP_EUNSUPPORTED;
  if (int rc = set_lds_limit(reinterpret_cast<const void*>(fn), lds)) return rc;
  const unsigned grid = unsigned(g.G * ((g.O + 63) / 64));
  hipLaunchKernelGGL(fn, dim3(grid), dim3(kStNT), lds, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                     static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
