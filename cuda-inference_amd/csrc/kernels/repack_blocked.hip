// Channel-blocked repack feeding the halo-tiled MFMA kernel, both tensors in one dispatch:
//   activations x [B][C][H*W] (NCHW)  -> xb [B][S][H*W][32]
//   weights     w [O][C][KH*KW] (OIHW) -> wb [O][S][KH*KW][32]
// with S = ceil(C / 32) channel slices of 32 and the channels past C zero. Within one slice every image row
// (activations) or every filter (weights) is one contiguous run of 64-byte pixel/tap records, so the kernel's
// per-slice loads use every byte of each cache line they fetch.
//
// Both are pure 16-bit permutations (the reference's transpose_c_hw, src/kernels/tensor_core_mma.cu:61-82,
// 309-310, with the channel index split into slice and lane) and HBM-bound: each element is read once and written
// once.
//   * activations: one workgroup per (image, slice, 64 pixels). Reads: 32 channel rows of 128 contiguous bytes
//     (8-byte loads when H*W % 4 == 0 and x is 8-byte aligned, else 2-byte loads). LDS tile [32][64]. Writes: the
//     tile's 4 KiB are contiguous in xb, 16 bytes per thread.
//   * weights: one workgroup per output channel. Its C*KH*KW values are contiguous in OIHW: 16-byte loads when
//     aligned, else 2-byte loads, into LDS; writes are 16-byte [tap][8 channels] vectors in xb order.
// Source pointers may be only 2-byte aligned (caller tensors); destinations are workspace slices (256-B aligned).
#include "device_common.h"

namespace gie_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kTilePx = 64;
constexpr int kTileRow = kTilePx + 4;  // LDS row pitch (elements): 8-byte aligned rows, conflict-free columns
constexpr int kWBuf = 16384;           // weight elements staged per workgroup (C*KH*KW above this: direct path)

struct BlockedJob {
  const uint16_t* __restrict__ x;
  uint16_t* __restrict__ xb;
  const uint16_t* __restrict__ w;
  uint16_t* __restrict__ wb;
  int B, C, HW, S, O, RS;
  int n_pt;      // 64-pixel tiles per (image, slice)
  long long n_act;
  int xvec;      // 8-byte activation loads
  int wvec;      // 16-byte weight loads
  int wlds;      // weights staged through LDS
};

__device__ __forceinline__ void act_tile(const BlockedJob& j, long long blk, uint16_t (*tile)[kTileRow]) {
  const int t = threadIdx.x;
  const int pt = int(blk % j.n_pt);
  const long long rest = blk / j.n_pt;
  const int s = int(rest % j.S), b = int(rest / j.S);
  const int p0 = pt * kTilePx;
  const uint16_t* src = j.x + static_cast<long long>(b) * j.C * j.HW;
  if (j.xvec) {  // 16 lanes x 8 bytes = one 128-byte run of a channel row
    const int px = p0 + (t & 15) * 4;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ch = (t >> 4) + h * 16, c = s * 32 + ch;
      u32x2 v = u32x2{0u, 0u};
      if (c < j.C && px < j.HW) v = *reinterpret_cast<const u32x2*>(src + static_cast<long long>(c) * j.HW + px);
      *reinterpret_cast<u32x2*>(&tile[ch][(t & 15) * 4]) = v;
    }
  } else {
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      const int ch = (t >> 6) + h * 4, pl = t & 63, c = s * 32 + ch, px = p0 + pl;
      tile[ch][pl] = (c < j.C && px < j.HW) ? src[static_cast<long long>(c) * j.HW + px] : uint16_t(0);
    }
  }
  __syncthreads();
  const int pl = t >> 2, k = t & 3, px = p0 + pl;
  if (px >= j.HW) return;
  u32x4 v;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    v[q] = uint32_t(tile[k * 8 + 2 * q][pl]) | (uint32_t(tile[k * 8 + 2 * q + 1][pl]) << 16);
  *reinterpret_cast<u32x4*>(j.xb + ((static_cast<long long>(b) * j.S + s) * j.HW + px) * 32 + k * 8) = v;
}

__device__ __forceinline__ void weight_filter(const BlockedJob& j, int o, uint16_t* buf) {
  const int n = j.C * j.RS;
  const uint16_t* src = j.w + static_cast<long long>(o) * n;
  const int chunks = j.S * j.RS * 4;  // 16-byte output vectors of this filter
  uint16_t* dst = j.wb + static_cast<long long>(o) * chunks * 8;
  if (j.wlds) {
    if (j.wvec) {
      for (int i = threadIdx.x * 8; i < n; i += kThreads * 8)
        *reinterpret_cast<u32x4*>(buf + i) = *reinterpret_cast<const u32x4*>(src + i);
    } else {
      for (int i = threadIdx.x; i < n; i += kThreads) buf[i] = src[i];
    }
    __syncthreads();
  }
  const uint16_t* from = j.wlds ? buf : src;
  for (int q = threadIdx.x; q < chunks; q += kThreads) {
    const int k = q & 3, tr = q >> 2;  // tr = s * RS + rs
    const int s = tr / j.RS, rs = tr - s * j.RS;
    u32x4 v;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int c = s * 32 + k * 8 + 2 * d;
      const uint32_t lo = c < j.C ? from[c * j.RS + rs] : 0u;
      const uint32_t hi = c + 1 < j.C ? from[(c + 1) * j.RS + rs] : 0u;
      v[d] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(dst + q * 8) = v;
  }
}

__global__ __launch_bounds__(kThreads) void repack_blocked_kernel(BlockedJob j) {
  __shared__ __attribute__((aligned(16))) uint16_t buf[kWBuf > 32 * kTileRow ? kWBuf : 32 * kTileRow];
  const long long blk = blockIdx.x;
  if (blk < j.n_act) act_tile(j, blk, reinterpret_cast<uint16_t(*)[kTileRow]>(buf));
  else weight_filter(j, int(blk - j.n_act), buf);
}

// Weights only, one thread per 16-byte output vector (filter o, slice s, tap rs, 8-channel group k): its 8
// halves w[o][s*32 + 8k + j][rs] are gathered straight from global memory (all 8 loads in flight, no LDS
// round trip or barrier: the weight repack sits on the critical path of every band call).
__global__ __launch_bounds__(kThreads) void repack_w_direct_kernel(const uint16_t* __restrict__ w,
                                                                  uint16_t* __restrict__ wb, int C, int RS,
                                                                  int S, long long n_vec) {
  const long long q = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (q >= n_vec) return;
  const int per_o = S * RS * 4;
  const int o = int(q / per_o), r = int(q - static_cast<long long>(o) * per_o);
  const int k = r & 3, tr = r >> 2, s = tr / RS, rs = tr - s * RS;
  const int c0 = s * 32 + k * 8;
  const uint16_t* src = w + (static_cast<long long>(o) * C + c0) * RS + rs;
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = c0 + j < C ? uint32_t(src[j * RS]) : 0u;
  *reinterpret_cast<u32x4*>(wb + q * 8) = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                                                h[6] | (h[7] << 16)};
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

namespace {

// x == nullptr: weights only (n_act = 0)
int repack_blocked(const void* x, void* xb, const void* w, void* wb, const gie_conv_geom* g, void* stream) {
  if (!g || !w || !wb || (x && !xb)) return GIE_HIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(xb) & 15u) || (reinterpret_cast<uintptr_t>(wb) & 15u)) return GIE_HIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(x) & 1u) || (reinterpret_cast<uintptr_t>(w) & 1u)) return GIE_HIP_EINVAL;
  BlockedJob j;
  j.x = static_cast<const uint16_t*>(x);
  j.xb = static_cast<uint16_t*>(xb);
  j.w = static_cast<const uint16_t*>(w);
  j.wb = static_cast<uint16_t*>(wb);
  j.B = g->batch;
  j.C = g->in_channels;
  j.O = g->out_channels;
  if (j.B <= 0 || j.C <= 0 || j.O <= 0 || g->in_h <= 0 || g->in_w <= 0 || g->kernel_h <= 0 || g->kernel_w <= 0)
    return GIE_HIP_EINVAL;
  const long long hw = static_cast<long long>(g->in_h) * g->in_w;
  const long long rs = static_cast<long long>(g->kernel_h) * g->kernel_w;
  if (hw > 0x7fffffffLL || rs * j.C > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  j.HW = int(hw);
  j.RS = int(rs);
  j.S = (j.C + 31) / 32;
  j.n_pt = int((hw + kTilePx - 1) / kTilePx);
  j.n_act = x ? static_cast<long long>(j.B) * j.S * j.n_pt : 0;
  j.xvec = (x && hw % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 7u) == 0) ? 1 : 0;
  j.wlds = (rs * j.C <= kWBuf) ? 1 : 0;
  j.wvec = ((reinterpret_cast<uintptr_t>(w) & 15u) == 0 && (rs * j.C) % 8 == 0) ? 1 : 0;
  const long long blocks = j.n_act + j.O;
  if (blocks > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  hipLaunchKernelGGL(repack_blocked_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), j);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}

}  // namespace

extern "C" int gie_hip_repack_blocked(const void* x, void* xb, const void* w, void* wb, const gie_conv_geom* g,
                                      void* stream) {
  if (!x) return GIE_HIP_EINVAL;
  return repack_blocked(x, xb, w, wb, g, stream);
}

extern "C" int gie_hip_repack_w_blocked(const void* w, void* wb, const gie_conv_geom* g, void* stream) {
  if (!g || !w || !wb) return GIE_HIP_EINVAL;
  if ((reinterpret_cast<uintptr_t>(wb) & 15u) || (reinterpret_cast<uintptr_t>(w) & 1u)) return GIE_HIP_EINVAL;
  if (g->in_channels <= 0 || g->out_channels <= 0 || g->kernel_h <= 0 || g->kernel_w <= 0) return GIE_HIP_EINVAL;
  const long long rs = static_cast<long long>(g->kernel_h) * g->kernel_w;
  const int S = (g->in_channels + 31) / 32;
  const long long n_vec = static_cast<long long>(g->out_channels) * S * rs * 4;
  if (rs * g->in_channels > 0x7fffffffLL || S * rs * 4 > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  const long long blocks = (n_vec + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  hipLaunchKernelGGL(repack_w_direct_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w), static_cast<uint16_t*>(wb),
                     g->in_channels, int(rs), S, n_vec);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
