// Layout repacks feeding the implicit GEMM: activations NCHW -> NHWC (channels padded to a multiple of 8 with
// zeros) and weights OIHW -> O,(R,S),C with the same padding, so one 16-byte vector = 8 channels of one pixel
// (or one tap) and the GEMM K index is ordered (r, s, c).
//
// Both are pure 16-bit permutations (bit-exact with the reference's transpose_c_hw indexing,
// src/kernels/tensor_core_mma.cu:61-82,309-310) and HBM-bound: every element is read once and written once.
//   * activations, channels > 16, H*W % 4 == 0, x 8-byte aligned (the common case): pixels of all images are
//     one flat index (b*HW + hw; a 4-pixel group never straddles two images). Each lane moves an 8-channel x
//     4-pixel block: eight 8-byte loads along pixels (16 lanes read 128 contiguous bytes of one channel row),
//     a register transpose, and four 16-byte NHWC stores (4 lanes write 64 contiguous bytes of one pixel).
//     No LDS, no barrier.
//   * activations, other channel counts > 16: a 64(pixel) x 64(channel) tile goes through LDS; global reads
//     are coalesced along pixels (128 B per wave-row), global writes are 16-byte vectors along channels.
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
  int vec;                // 1: register-transpose path
  long long vtiles_p;     // register-transpose path: 64-pixel tiles over batch*HW
  int vtiles_c;           // ... and 128-channel tiles over Cp
};

constexpr int kVecPx = 64;   // pixels per register-transpose workgroup tile (16 lanes x 4 pixels)
constexpr int kVecCh = 128;  // channels per tile (4 waves x 4 lanes x 8 channels)

struct WJob {
  const uint16_t* __restrict__ w;
  uint16_t* __restrict__ wk;
  int O, C, RS, Cp;
  int vec_load;  // 1: every filter starts 16-byte aligned
};

inline long long act_blocks(const ActJob& j) {
  if (j.vec) return j.vtiles_p * j.vtiles_c;
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

__device__ __forceinline__ void act_vec(const ActJob& j, long long blk) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const long long tp = blk % j.vtiles_p;
  const int tc = int(blk / j.vtiles_p);
  const long long P = tp * kVecPx + (lane & 15) * 4;           // first of this lane's 4 pixels (b*HW + hw)
  const int c8 = tc * kVecCh + wave * 32 + (lane >> 4) * 8;    // first of its 8 channels
  if (P >= static_cast<long long>(j.batch) * j.HW || c8 >= j.Cp) return;
  const long long b = P / j.HW, hw = P - b * j.HW;
  const uint16_t* src = j.x + (b * j.C + c8) * j.HW + hw;    // 8-byte aligned: HW % 4 == 0, hw % 4 == 0
  u32x2 in[8];
#pragma unroll
  for (int r = 0; r < 8; ++r)
    in[r] = c8 + r < j.C ? *reinterpret_cast<const u32x2*>(src + static_cast<long long>(r) * j.HW) : u32x2{0u, 0u};
  uint16_t* dst = j.xn + P * j.Cp + c8;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // pixel q: channel pair (2d, 2d+1) -> dword d
    u32x4 v;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t lo = in[2 * d][q >> 1], hi = in[2 * d + 1][q >> 1];
      v[d] = (q & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
    }
    *reinterpret_cast<u32x4*>(dst + static_cast<long long>(q) * j.Cp) = v;
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
  if (j.vec_load) {  // filter rows start 16-byte aligned (w aligned, n % 8 == 0): 16-byte loads
    for (int i = threadIdx.x * 8; i < n; i += kThreads * 8)
      *reinterpret_cast<u32x4*>(buf + i) = *reinterpret_cast<const u32x4*>(src + i);
  } else {
    for (int i = threadIdx.x; i < n; i += kThreads) buf[i] = src[i];
  }
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
  if (j.vec) act_vec(j, blockIdx.x);
  else if (j.small) act_small(j, blockIdx.x);
  else act_tiled(j, blockIdx.x, tile);
}

__global__ __launch_bounds__(kThreads) void repack_w_kernel(WJob j) {
  __shared__ __attribute__((aligned(16))) uint16_t buf[kWElems];
  weight_any(j, blockIdx.x, buf);
}

// Both repacks in one dispatch: blocks [0, n_act) repack activations, the rest repack weights.
__global__ __launch_bounds__(kThreads) void repack_both_kernel(ActJob a, WJob w, long long n_act) {
  __shared__ __attribute__((aligned(16))) uint16_t buf[kWElems > kTile * (kTile + 2) ? kWElems : kTile * (kTile + 2)];
  const long long blk = blockIdx.x;
  if (blk < n_act) {
    if (a.vec) act_vec(a, blk);
    else if (a.small) act_small(a, blk);
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
  j->vec = (!j->small && HW % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 7u) == 0) ? 1 : 0;
  j->vtiles_p = (static_cast<long long>(batch) * HW + kVecPx - 1) / kVecPx;
  j->vtiles_c = ceil_div_i(Cp, kVecCh);
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
  j->vec_load = (aligned16(w) && (C * RS) % 8 == 0) ? 1 : 0;
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
  if (status == GIE_HIP_ESCRATCH) return "request exceeds the library's static scratch";
  return hipGetErrorString(static_cast<hipError_t>(status));
}
