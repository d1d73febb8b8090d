// Narrow convolution: 3x3 filter, stride 1, padding 1, for layers with few output pixels and a long reduction
// (config 5: N = 8 * 7 * 7 = 392 pixels, K = 512 * 9 = 4608) on gfx950 matrix cores (v_mfma_f32_32x32x16_{f16,bf16},
// FP32 accumulation). One launch, no repack and no split-K partials in HBM.
//
// The matrix-core families tile N in 128-pixel steps and split K across workgroups, which leaves this shape bound
// by fixed costs: the weight repack (4.7 MB read and written), FP32 partials and their reduce, three launches.
// Here a workgroup owns 32 filters x 32 output pixels and the whole reduction:
//   * K in the weights' own order (channel, tap): a filter's OIHW row is K-contiguous, so each lane's 8 weights of
//     a k-step are one 16-byte load straight from w (no repack);
//   * the activations of the images the block touches (at most a few, C x H x W each) are copied to LDS once; the
//     pixel operand (8 consecutive k = (channel, tap) pairs of the lane's pixel) is gathered from there with
//     tables built once per workgroup in LDS and held in registers: for each of the 9 k-steps of a 16-channel
//     unit, the offset of every element relative to the unit's first channel, and per element pair a mask that
//     zeroes the taps in the padding;
//   * the 8 waves split the channels (C / 8 each, in 16-channel units), then the 8 partial tiles are summed in LDS
//     in wave order (deterministic) and the sum gets bias + ReLU and one RNE rounding (the order of the
//     reference's apply_epilogue, src/kernels/fused_epilogue.cuh:11-16).
// Grid: tiles (filter block, pixel block) in 8 contiguous ranges, one per XCD (blockIdx mod 8), so the
// workgroups of one filter block share an L2.
#include <algorithm>

#include "lds_pipe.h"

namespace gie_hip {
namespace {

constexpr int kNaNT = 512;             // 8 waves
constexpr int kNaWaves = 8;
constexpr int kNaLdsMax = 160 * 1024;

struct NarrowGeom {
  int B, C, H, W, O, HW, NPIX, K;
  int x_bytes;
  int n_pb;      // 32-pixel blocks
  int n_tiles;   // filter blocks x pixel blocks
  int per_xcd;   // tiles per XCD range
  int cw;        // channels per wave (a multiple of 16)
  int tab_off;   // LDS byte offset of the gather tables (after the staged activations)
};

template <typename E, bool RELU>
__global__ __launch_bounds__(kNaNT) void narrow_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                      const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                      NarrowGeom g) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = lane >> 5, col = lane & 31;
  const int L = blockIdx.x, xcd = L & 7;
  const int t = xcd * g.per_xcd + (L >> 3);
  if ((L >> 3) >= g.per_xcd || t >= g.n_tiles) return;  // workgroup-uniform padding slot
  const int fb = t / g.n_pb, pb = t - fb * g.n_pb;
  const int p0 = pb * 32, f0 = fb * 32;

  // ---- the activations of the images this pixel block touches, one contiguous NCHW range, into LDS
  const int img_lo = p0 / g.HW;
  const int img_hi = min(p0 + 31, g.NPIX - 1) / g.HW;
  // (buffer_load ... lds: 64 chunks of 16 bytes per instruction, all in flight at once; lanes past the range are
  // inactive and write nothing)
  {
    const int n16 = (img_hi - img_lo + 1) * g.C * g.HW / 8;  // C % 128 == 0: whole 16-byte chunks
    const v4i xr = make_vsharp(x, g.x_bytes);
    const int src0 = img_lo * g.C * g.HW * 2;
    for (int j = wave; j * 64 < n16; j += kNaWaves) {
      const int ci = j * 64 + lane;
      if (ci < n16) dma16(xr, lds_addr(smem + j * 1024), src0 + ci * 16);
    }
    wait_vmcnt<0>();
  }

  // ---- gather tables, built once per workgroup in LDS (every wave multiplies the same 32 pixels): element j of
  // k-step s of a 16-channel unit is k = 16s + 8hi + j of the unit, channel k / 9, tap k % 9. For lane (hi, col):
  // its LDS offset (halves) relative to the unit's first channel of the lane's image, and per element pair a
  // mask that zeroes the taps in the padding.
  int* tab_rel = reinterpret_cast<int*>(smem + g.tab_off);                 // [hi][col][72]
  uint8_t* tab_ok = smem + g.tab_off + 2 * 32 * 72 * 4;                     // [hi][col][72]
  uint32_t* tab_msk = reinterpret_cast<uint32_t*>(smem + g.tab_off + 2 * 32 * 72 * 5);  // [hi][col][36]
  {
    const int th = tid >> 8, tc = (tid >> 3) & 31, part = tid & 7;
    const int p = p0 + tc;
    const int pc = p < g.NPIX ? p : p0;
    const int img = pc / g.HW, q = pc - img * g.HW;
    const int oh = q / g.W, ow = q - oh * g.W;
    const int lbase = (img - img_lo) * g.C * g.HW;
#pragma unroll
    for (int u = 0; u < 9; ++u) {
      const int e = part * 9 + u, k = 16 * (e >> 3) + 8 * th + (e & 7);
      const int c = k / 9, tp = k - c * 9;
      const int ih = oh + tp / 3 - 1, iw = ow + tp % 3 - 1;
      const bool ok = ih >= 0 && ih < g.H && iw >= 0 && iw < g.W;
      tab_rel[(th * 32 + tc) * 72 + e] = lbase + c * g.HW + (ok ? ih * g.W + iw : 0);
      tab_ok[(th * 32 + tc) * 72 + e] = ok ? 1 : 0;
    }
  }
  __syncthreads();  // (also: the activations are in)
  for (int i = tid; i < 2 * 32 * 36; i += kNaNT) {
    const int lc = i / 36, pr = i - lc * 36;
    tab_msk[i] = (tab_ok[lc * 72 + 2 * pr] ? 0xffffu : 0u) | (tab_ok[lc * 72 + 2 * pr + 1] ? 0xffff0000u : 0u);
  }
  __syncthreads();
  int rel[72];
  uint32_t msk[36];
  {
    const u32x4* tr = reinterpret_cast<const u32x4*>(tab_rel + (hi * 32 + col) * 72);
    const u32x4* tm = reinterpret_cast<const u32x4*>(tab_msk + (hi * 32 + col) * 36);
#pragma unroll
    for (int v = 0; v < 18; ++v) {
      const u32x4 r = tr[v];
      rel[4 * v] = int(r.x), rel[4 * v + 1] = int(r.y), rel[4 * v + 2] = int(r.z), rel[4 * v + 3] = int(r.w);
    }
#pragma unroll
    for (int v = 0; v < 9; ++v) {
      const u32x4 m = tm[v];
      msk[4 * v] = m.x, msk[4 * v + 1] = m.y, msk[4 * v + 2] = m.z, msk[4 * v + 3] = m.w;
    }
  }

  // ---- this wave's channels [wave * cw, +cw) in units of 16: 9 k-steps of 16 each
  const uint16_t* xl = reinterpret_cast<const uint16_t*>(smem);
  const uint16_t* wrow = w + size_t(min(f0 + col, g.O - 1)) * g.K + 8 * hi;  // rows past O: any valid row
  f32x16 acc = {0};
  const int c_beg = wave * g.cw;
  // the next unit's weights are loaded while this unit is multiplied
  u32x4 a[9], an[9];
#pragma unroll
  for (int s = 0; s < 9; ++s) an[s] = *reinterpret_cast<const u32x4*>(wrow + c_beg * 9 + 16 * s);
  for (int cu = c_beg; cu < c_beg + g.cw; cu += 16) {
#pragma unroll
    for (int s = 0; s < 9; ++s) a[s] = an[s];
    const int cn = cu + 16 < c_beg + g.cw ? cu + 16 : cu;  // past the last unit: reload this one (any valid row)
#pragma unroll
    for (int s = 0; s < 9; ++s) an[s] = *reinterpret_cast<const u32x4*>(wrow + cn * 9 + 16 * s);
    const uint16_t* xu = xl + cu * g.HW;
#pragma unroll
    for (int s = 0; s < 9; ++s) {
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = xu[rel[s * 8 + j]];
      const u32x4 b = u32x4{(h[0] | (h[1] << 16)) & msk[4 * s], (h[2] | (h[3] << 16)) & msk[4 * s + 1],
                            (h[4] | (h[5] << 16)) & msk[4 * s + 2], (h[6] | (h[7] << 16)) & msk[4 * s + 3]};
      acc = E::mfma32(a[s], b, acc);  // rows: filters; columns: pixels
    }
  }

  // ---- the 8 partial tiles summed in wave order, bias + ReLU, one rounding, NCHW stores
  __syncthreads();  // the activations are no longer read
  float* red = reinterpret_cast<float*>(smem);  // [wave][16][64]
#pragma unroll
  for (int i = 0; i < 16; ++i) red[(wave * 16 + i) * 64 + lane] = acc[i];
  __syncthreads();
  for (int e = tid; e < 16 * 64; e += kNaNT) {
    const int i = e >> 6, l = e & 63;
    float sum = 0.0f;
#pragma unroll
    for (int wv = 0; wv < kNaWaves; ++wv) sum += red[(wv * 16 + i) * 64 + l];
    const int f = f0 + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3), pp = p0 + (l & 31);
    if (f < g.O && pp < g.NPIX) {
      if (bias != nullptr) sum += E::to_f32(bias[f]);
      if (RELU) sum = fmaxf(sum, 0.0f);
      const int im = pp / g.HW, qq = pp - im * g.HW;
      y[(size_t(im) * g.O + f) * g.HW + qq] = E::from_f32(sum);
    }
  }
}

int narrow_prepare(const gie_conv_geom* gg, NarrowGeom* g, int* lds) {
  if (!gg) return GIE_HIP_EINVAL;
  if (gg->kernel_h != 3 || gg->kernel_w != 3 || gg->stride_h != 1 || gg->stride_w != 1 || gg->pad_h != 1 ||
      gg->pad_w != 1)
    return GIE_HIP_EUNSUPPORTED;
  if (gg->batch < 1 || gg->in_h < 1 || gg->in_w < 1 || gg->out_channels < 1 || gg->in_channels < 128 ||
      gg->in_channels % 128 != 0)
    return GIE_HIP_EUNSUPPORTED;
  if (gg->out_h != gg->in_h || gg->out_w != gg->in_w) return GIE_HIP_EINVAL;
  const long long hw = 1LL * gg->in_h * gg->in_w;
  const long long npix = gg->batch * hw;
  if (npix >= (1LL << 24) || 1LL * gg->out_channels * gg->in_channels * 9 >= (1LL << 31) ||
      2 * npix * gg->in_channels >= (1LL << 31) || npix * gg->out_channels >= (1LL << 31))
    return GIE_HIP_EUNSUPPORTED;
  // images one 32-pixel block can touch, staged whole in LDS
  const long long n_img = std::min<long long>(gg->batch, 31 / hw + 2);
  const long long x_lds = (n_img * gg->in_channels * hw * 2 + 15) / 16 * 16;
  const long long tab = 2 * 32 * 72 * 5 + 2 * 32 * 36 * 4;  // offsets, valid flags, pair masks
  const long long need = std::max<long long>(x_lds + tab, kNaWaves * 16 * 64 * 4);
  if (need > kNaLdsMax) return GIE_HIP_EUNSUPPORTED;
  g->B = gg->batch, g->C = gg->in_channels, g->H = gg->in_h, g->W = gg->in_w, g->O = gg->out_channels;
  g->HW = int(hw), g->NPIX = int(npix), g->K = gg->in_channels * 9;
  g->n_pb = int((npix + 31) / 32);
  g->n_tiles = (g->O + 31) / 32 * g->n_pb;
  g->per_xcd = (g->n_tiles + 7) / 8;
  g->cw = g->C / kNaWaves;
  g->tab_off = int(x_lds);
  g->x_bytes = int(npix * gg->in_channels * 2);
  if (lds) *lds = int(need);
  return GIE_HIP_OK;
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_narrow_check(const gie_conv_geom* g, int* lds_bytes) {
  NarrowGeom ng;
  return narrow_prepare(g, &ng, lds_bytes);
}

extern "C" int gie_hip_conv_narrow(int dtype, const gie_conv_geom* gg, const void* x, const void* w, const void* bias,
                                   void* y, void* stream) {
  if (!gg || !x || !w || !y) return GIE_HIP_EINVAL;
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  if ((bias && (reinterpret_cast<uintptr_t>(bias) & 1u)) || (reinterpret_cast<uintptr_t>(y) & 1u))
    return GIE_HIP_EINVAL;
  NarrowGeom g;
  int lds = 0;
  if (int rc = narrow_prepare(gg, &g, &lds)) return rc;
  // 16-byte activation chunks and weight rows
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(w) & 15u)) return GIE_HIP_EUNSUPPORTED;
  using Fn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, NarrowGeom);
  const bool bf = dtype == GIE_HIP_BF16;
  const Fn fn = bf ? (gg->relu ? &narrow_kernel<Bf16, true> : &narrow_kernel<Bf16, false>)
                   : (gg->relu ? &narrow_kernel<Fp16, true> : &narrow_kernel<Fp16, false>);
  if (int rc = set_lds_limit(reinterpret_cast<const void*>(fn), lds)) return rc;
  hipLaunchKernelGGL(fn, dim3(unsigned(8 * g.per_xcd)), dim3(kNaNT), lds, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                     static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), g);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
