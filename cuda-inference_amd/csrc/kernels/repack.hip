// Layout repacks feeding the implicit GEMM: activations NCHW -> NHWC (channels padded to a multiple of 8 with
// zeros) and weights OIHW -> O,(R,S),C with the same padding, so one 16-byte vector = 8 channels of one pixel
// (or one tap) and the GEMM K index is ordered (r, s, c).
//
// Both are pure 16-bit permutations (bit-exact with the reference's transpose_c_hw indexing,
// src/kernels/tensor_core_mma.cu:61-82,309-310) and HBM-bound: every element is read once and written once.
//   * activations, channels >= 16: a 64(pixel) x 64(channel) tile goes through LDS; global reads are
//     coalesced along pixels (128 B per wave-row), global writes are 16-byte vectors along channels.
//   * activations, channels < 16 (the 7x7 stem, C=3): one thread per pixel, C strided 2-byte reads that are
//     coalesced across the wave, C_pad/8 16-byte writes.
//   * weights: one thread per (o, tap, 8-channel chunk), 8 strided reads from a small L2-resident tensor and
//     one 16-byte write.
// Source pointers may be only 2-byte aligned (caller tensors); destinations are workspace slices (256-B aligned).
#include "device_common.h"

namespace gie_hip {
namespace {

constexpr int kTile = 64;
constexpr int kThreads = 256;

struct ActJob {
  const uint16_t* __restrict__ x;
  uint16_t* __restrict__ xn;
  int batch, C, HW, Cp;
  int tiles_hw, tiles_c;  // tiled path
  int small;              // 1: one thread per pixel
};

struct WJob {
  const uint16_t* __restrict__ w;
  uint16_t* __restrict__ wk;
  int O, C, RS, Cp;
};

inline long long act_blocks(const ActJob& j) {
  return j.small ? (static_cast<long long>(j.batch) * j.HW + kThreads - 1) / kThreads
                 : static_cast<long long>(j.tiles_hw) * j.tiles_c * j.batch;
}
inline long long w_blocks(const WJob& j) {
  return (static_cast<long long>(j.O) * j.RS * (j.Cp / 8) + kThreads - 1) / kThreads;
}

__device__ __forceinline__ void act_tiled(const ActJob& j, long long blk, uint16_t (*tile)[kTile + 2]) {
  const int t = threadIdx.x;
  const int th = int(blk % j.tiles_hw);
  const long long rest = blk / j.tiles_hw;
  const int tc = int(rest % j.tiles_c);
  const int b = int(rest / j.tiles_c);
  const int hw0 = th * kTile, c0 = tc * kTile;
  const uint16_t* src = j.x + static_cast<long long>(b) * j.C * j.HW;
  uint16_t* dst = j.xn + static_cast<long long>(b) * j.Cp * j.HW;
  {
    const int hw = hw0 + (t & 63);
#pragma unroll 4
    for (int cc = t >> 6; cc < kTile; cc += kThreads / 64) {
      const int c = c0 + cc;
      tile[cc][t & 63] = (c < j.C && hw < j.HW) ? src[static_cast<long long>(c) * j.HW + hw] : uint16_t(0);
    }
  }
  __syncthreads();
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int hl = (t >> 3) + pass * 32;
    const int ch = (t & 7) * 8;
    const int hw = hw0 + hl, c = c0 + ch;
    if (hw < j.HW && c < j.Cp) {
      u32x4 v;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[q] = uint32_t(tile[ch + 2 * q][hl]) | (uint32_t(tile[ch + 2 * q + 1][hl]) << 16);
      *reinterpret_cast<u32x4*>(dst + static_cast<long long>(hw) * j.Cp + c) = v;
    }
  }
}

__device__ __forceinline__ void act_small(const ActJob& j, long long blk) {
  const long long i = blk * kThreads + threadIdx.x;
  if (i >= static_cast<long long>(j.batch) * j.HW) return;
  const int b = int(i / j.HW), hw = int(i - static_cast<long long>(b) * j.HW);
  const uint16_t* src = j.x + static_cast<long long>(b) * j.C * j.HW + hw;
  uint16_t* dst = j.xn + i * j.Cp;
  for (int c8 = 0; c8 < j.Cp; c8 += 8) {
    u32x4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = c8 + 2 * q;
      const uint32_t lo = c < j.C ? src[static_cast<long long>(c) * j.HW] : 0u;
      const uint32_t hi = c + 1 < j.C ? src[static_cast<long long>(c + 1) * j.HW] : 0u;
      v[q] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(dst + c8) = v;
  }
}

__device__ __forceinline__ void weight_chunk(const WJob& j, long long blk) {
  const long long i = blk * kThreads + threadIdx.x;
  const int cv = j.Cp / 8;
  if (i >= static_cast<long long>(j.O) * j.RS * cv) return;
  const int c8 = int(i % cv) * 8;
  const long long orow = i / cv;  // o * RS + rs
  const int rs = int(orow % j.RS), o = int(orow / j.RS);
  const uint16_t* src = j.w + static_cast<long long>(o) * j.C * j.RS + rs;
  u32x4 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = c8 + 2 * q;
    const uint32_t lo = c < j.C ? src[static_cast<long long>(c) * j.RS] : 0u;
    const uint32_t hi = c + 1 < j.C ? src[static_cast<long long>(c + 1) * j.RS] : 0u;
    v[q] = lo | (hi << 16);
  }
  *reinterpret_cast<u32x4*>(j.wk + orow * j.Cp + c8) = v;
}

// One output channel per workgroup: its C*RS filter taps are contiguous in OIHW, so they are read with
// coalesced loads into LDS and leave as 16-byte [rs][8 channels] vectors (used when C*RS fits kWElems).
constexpr int kWElems = 8192;

__device__ __forceinline__ void weight_filter(const WJob& j, long long o, uint16_t* buf) {
  const int n = j.C * j.RS;
  const uint16_t* src = j.w + o * n;
  for (int i = threadIdx.x; i < n; i += kThreads) buf[i] = src[i];
  __syncthreads();
  const int cv = j.Cp / 8;
  uint16_t* dst = j.wk + o * static_cast<long long>(j.RS) * j.Cp;
  for (int t = threadIdx.x; t < j.RS * cv; t += kThreads) {
    const int rs = t / cv, c8 = (t - rs * cv) * 8;
    u32x4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = c8 + 2 * q;
      const uint32_t lo = c < j.C ? buf[c * j.RS + rs] : 0u;
      const uint32_t hi = c + 1 < j.C ? buf[(c + 1) * j.RS + rs] : 0u;
      v[q] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(dst + rs * j.Cp + c8) = v;
  }
}

inline bool w_per_filter(const WJob& j) { return j.C * j.RS <= kWElems; }

inline long long w_launch_blocks(const WJob& j) { return w_per_filter(j) ? j.O : w_blocks(j); }

__device__ __forceinline__ void weight_any(const WJob& j, long long blk, uint16_t* buf) {
  if (j.C * j.RS <= kWElems) weight_filter(j, blk, buf);
  else weight_chunk(j, blk);
}

__global__ __launch_bounds__(kThreads) void repack_act_kernel(ActJob j) {
  __shared__ uint16_t tile[kTile][kTile + 2];
  if (j.small) act_small(j, blockIdx.x);
  else act_tiled(j, blockIdx.x, tile);
}

__global__ __launch_bounds__(kThreads) void repack_w_kernel(WJob j) {
  __shared__ uint16_t buf[kWElems];
  weight_any(j, blockIdx.x, buf);
}

// Both repacks in one dispatch: blocks [0, n_act) repack activations, the rest repack weights.
__global__ __launch_bounds__(kThreads) void repack_both_kernel(ActJob a, WJob w, long long n_act) {
  __shared__ uint16_t buf[kWElems > kTile * (kTile + 2) ? kWElems : kTile * (kTile + 2)];
  const long long blk = blockIdx.x;
  if (blk < n_act) {
    if (a.small) act_small(a, blk);
    else act_tiled(a, blk, reinterpret_cast<uint16_t(*)[kTile + 2]>(buf));
  } else {
    weight_any(w, blk - n_act, buf);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int make_act(const void* x, void* xn, int batch, int C, int HW, int Cp, ActJob* j) {
  if (!x || !xn || batch <= 0 || C <= 0 || HW <= 0 || Cp < C || Cp % 8 != 0 || !aligned16(xn)) return GIE_HIP_EINVAL;
  j->x = static_cast<const uint16_t*>(x);
  j->xn = static_cast<uint16_t*>(xn);
  j->batch = batch;
  j->C = C;
  j->HW = HW;
  j->Cp = Cp;
  j->small = Cp <= 16 ? 1 : 0;
  j->tiles_hw = ceil_div_i(HW, kTile);
  j->tiles_c = ceil_div_i(Cp, kTile);
  return GIE_HIP_OK;
}

int make_w(const void* w, void* wk, int O, int C, int RS, int Cp, WJob* j) {
  if (!w || !wk || O <= 0 || C <= 0 || RS <= 0 || Cp < C || Cp % 8 != 0 || !aligned16(wk)) return GIE_HIP_EINVAL;
  j->w = static_cast<const uint16_t*>(w);
  j->wk = static_cast<uint16_t*>(wk);
  j->O = O;
  j->C = C;
  j->RS = RS;
  j->Cp = Cp;
  return GIE_HIP_OK;
}

int launched() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_repack_act_nchw_to_nhwc(const void* x, void* xn, int batch, int channels, int hw, int c_pad,
                                               void* stream) {
  ActJob j;
  if (int rc = make_act(x, xn, batch, channels, hw, c_pad, &j)) return rc;
  const long long blocks = act_blocks(j);
  if (blocks > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  hipLaunchKernelGGL(repack_act_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, static_cast<hipStream_t>(stream), j);
  return launched();
}

extern "C" int gie_hip_repack_w_oihw_to_orsc(const void* w, void* wk, int out_channels, int channels, int rs, int c_pad,
                                             void* stream) {
  WJob j;
  if (int rc = make_w(w, wk, out_channels, channels, rs, c_pad, &j)) return rc;
  const long long blocks = w_launch_blocks(j);
  if (blocks > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  hipLaunchKernelGGL(repack_w_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, static_cast<hipStream_t>(stream), j);
  return launched();
}

extern "C" int gie_hip_repack_act_and_w(const void* x, void* xn, const void* w, void* wk, const gie_conv_geom* g,
                                        void* stream) {
  if (!g) return GIE_HIP_EINVAL;
  ActJob a;
  WJob wj;
  if (int rc = make_act(x, xn, g->batch, g->in_channels, g->in_h * g->in_w, g->c_pad, &a)) return rc;
  if (int rc = make_w(w, wk, g->out_channels, g->in_channels, g->kernel_h * g->kernel_w, g->c_pad, &wj)) return rc;
  const long long na = act_blocks(a), nw = w_launch_blocks(wj);
  if (na + nw > 0x7fffffffLL) return GIE_HIP_EUNSUPPORTED;
  hipLaunchKernelGGL(repack_both_kernel, dim3(unsigned(na + nw)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     a, wj, na);
  return launched();
}

extern "C" const char* gie_hip_status_string(int status) {
  if (status == GIE_HIP_OK) return "ok";
  if (status == GIE_HIP_EINVAL) return "invalid argument";
  if (status == GIE_HIP_EUNSUPPORTED) return "unsupported by this kernel configuration";
  return hipGetErrorString(static_cast<hipError_t>(status));
}
