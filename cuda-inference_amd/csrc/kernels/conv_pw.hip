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
