// Split-K reduction + fused epilogue: y[i] = round(relu?(sum_z partial[z][i] + bias[c(i)])), summing the FP32
// partial slices in ascending z (the reference's order, src/kernels/tensor_core_mma.cu:254-262) so results are
// deterministic run to run. HBM-bound: reads split*4 B and writes 2 B per output. Each thread owns 4
// consecutive outputs: 16-byte partial loads (when every slice start is 16-byte aligned) and one 8-byte store
// when the destination allows it; a grid-stride loop keeps the grid bounded. Index arithmetic is 32-bit with
// magic-number divisions when every partial offset z * total + i fits an int (64-bit divisions per output cost
// more than the loads); otherwise 64-bit throughout.
#include "device_common.h"

namespace gie_hip {
namespace {

constexpr int kThreads = 256;

// n / d for 0 <= n < 2^30 with host-computed magic numbers (l = ceil(log2 d), mg = floor(2^32 (2^l - d) / d) + 1)
struct Div30 {
  unsigned mg;
  int sh;
};
__device__ __forceinline__ int div30(int n, Div30 d) { return int((__umulhi(unsigned(n), d.mg) + unsigned(n)) >> d.sh); }

// Partial offsets below 2^31 (split * total): 32-bit indices, the channel of a quad's first output by two
// magic-number divisions and the later ones by counting the plane crossings (hw_out may be below 4). NS > 0: the
// split factor is a compile-time constant, so every slice's load is in flight before the first add (a run-time trip
// count makes the compiler wait for each load in turn); NS = 0: any split, loads issued eight at a time. The bias
// values are fetched before the partials. The sum stays 0 + p0 + p1 + ... in ascending z.
template <typename E, bool kVec, int NS>
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(const float* __restrict__ partial,
                                                                 const uint16_t* __restrict__ bias,
                                                                 uint16_t* __restrict__ y, int total, int split,
                                                                 int M, int HWo, Div30 d_hw, Div30 d_m, int relu) {
  const int quads = (total + 3) / 4;
  for (int qi = int(blockIdx.x) * kThreads + int(threadIdx.x); qi < quads; qi += int(gridDim.x) * kThreads) {
    const int i0 = qi * 4;
    // the slices' loads first (all in flight for NS > 0), then the bias loads behind them
    f32x4 v[NS > 0 ? NS : 1];
    if constexpr (kVec && NS > 0) {
#pragma unroll
      for (int z = 0; z < NS; ++z) v[z] = *reinterpret_cast<const f32x4*>(partial + i0 + z * total);
    }
    const int plane = div30(i0, d_hw);
    int pix = i0 - plane * HWo, ch = plane - div30(plane, d_m) * M;
    int chs[4];
    for (int e = 0; e < 4; ++e) {
      chs[e] = ch;
      if (++pix == HWo) {
        pix = 0;
        ch = ch + 1 == M ? 0 : ch + 1;
      }
    }
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias != nullptr) {
      uint16_t bb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) bb[e] = bias[chs[e]];
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[e] = E::to_f32(bb[e]);
    }
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kVec && NS > 0) {  // total % 4 == 0: every slice is 16-byte aligned and the quad is whole
#pragma unroll
      for (int z = 0; z < NS; ++z) {
        s[0] += v[z][0];
        s[1] += v[z][1];
        s[2] += v[z][2];
        s[3] += v[z][3];
      }
    } else if constexpr (kVec) {
      const float* p = partial + i0;
      for (int z0 = 0; z0 < split; z0 += 8) {
        f32x4 w[8];
#pragma unroll
        for (int z = 0; z < 8; ++z)
          w[z] = z0 + z < split ? *reinterpret_cast<const f32x4*>(p + (z0 + z) * total) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int z = 0; z < 8; ++z) {
          if (z0 + z < split) {
            s[0] += w[z][0];
            s[1] += w[z][1];
            s[2] += w[z][2];
            s[3] += w[z][3];
          }
        }
      }
    } else {
      for (int z = 0; z < split; ++z)
        for (int e = 0; e < 4; ++e)
          if (i0 + e < total) s[e] += partial[static_cast<long long>(z) * total + i0 + e];
    }
    uint16_t h[4];
    for (int e = 0; e < 4; ++e) {
      const float v = s[e] + bv[e];
      h[e] = E::from_f32(relu ? fmaxf(v, 0.0f) : v);
    }
    uint16_t* dst = y + i0;
    if (i0 + 3 < total && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
      *reinterpret_cast<u32x2*>(dst) = u32x2{uint32_t(h[0]) | (uint32_t(h[1]) << 16), uint32_t(h[2]) | (uint32_t(h[3]) << 16)};
    } else {
      for (int e = 0; e < 4; ++e)
        if (i0 + e < total) dst[e] = h[e];
    }
  }
}

// Partial offsets of 2^31 and more: 64-bit indices and divisions.
template <typename E, bool kVec>
__global__ __launch_bounds__(kThreads) void splitk_reduce_wide_kernel(const float* __restrict__ partial,
                                                                      const uint16_t* __restrict__ bias,
                                                                      uint16_t* __restrict__ y, long long total,
                                                                      int split, int M, int HWo, int relu) {
  const long long quads = (total + 3) / 4;
  for (long long qi = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; qi < quads;
       qi += static_cast<long long>(gridDim.x) * kThreads) {
    const long long i0 = qi * 4;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if (kVec) {
      for (int z = 0; z < split; ++z) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(partial + z * total + i0);
        s[0] += v[0];
        s[1] += v[1];
        s[2] += v[2];
        s[3] += v[3];
      }
    } else {
      for (int z = 0; z < split; ++z)
        for (int e = 0; e < 4; ++e)
          if (i0 + e < total) s[e] += partial[z * total + i0 + e];
    }
    uint16_t h[4];
    for (int e = 0; e < 4; ++e) h[e] = epilogue<E>(s[e], bias, int(((i0 + e) / HWo) % M), relu);
    uint16_t* dst = y + i0;
    if (i0 + 3 < total && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
      *reinterpret_cast<u32x2*>(dst) = u32x2{uint32_t(h[0]) | (uint32_t(h[1]) << 16), uint32_t(h[2]) | (uint32_t(h[3]) << 16)};
    } else {
      for (int e = 0; e < 4; ++e)
        if (i0 + e < total) dst[e] = h[e];
    }
  }
}

// FP32 / TF32 output: the same sum and epilogue, stored as float (no rounding step)
template <bool kVec>
__global__ __launch_bounds__(kThreads) void splitk_reduce_f32_kernel(const float* __restrict__ partial,
                                                                     const float* __restrict__ bias,
                                                                     float* __restrict__ y, long long total, int split,
                                                                     int M, int HWo, int relu) {
  const long long quads = (total + 3) / 4;
  for (long long qi = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; qi < quads;
       qi += static_cast<long long>(gridDim.x) * kThreads) {
    const long long i0 = qi * 4;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int z = 0; z < split; ++z) {
      if (kVec) {
        s += *reinterpret_cast<const f32x4*>(partial + z * total + i0);
      } else {
        for (int e = 0; e < 4; ++e)
          if (i0 + e < total) s[e] += partial[z * total + i0 + e];
      }
    }
    for (int e = 0; e < 4; ++e) {
      if (i0 + e >= total) break;
      float v = s[e];
      if (bias) v += bias[((i0 + e) / HWo) % M];
      if (relu) v = fmaxf(v, 0.f);
      if (kVec) s[e] = v;
      else y[i0 + e] = v;
    }
    if (kVec) *reinterpret_cast<f32x4*>(y + i0) = s;
  }
}

void launch_f32(const float* partial, const void* bias, void* y, long long total, int split, int M, int HWo, int relu,
                hipStream_t s) {
  long long blocks = ((total + 3) / 4 + kThreads - 1) / kThreads;
  if (blocks > (1 << 20)) blocks = 1 << 20;
  const bool vec = (total % 4) == 0 && (reinterpret_cast<uintptr_t>(partial) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
  if (vec)
    hipLaunchKernelGGL((splitk_reduce_f32_kernel<true>), dim3(unsigned(blocks)), dim3(kThreads), 0, s, partial,
                       static_cast<const float*>(bias), static_cast<float*>(y), total, split, M, HWo, relu);
  else
    hipLaunchKernelGGL((splitk_reduce_f32_kernel<false>), dim3(unsigned(blocks)), dim3(kThreads), 0, s, partial,
                       static_cast<const float*>(bias), static_cast<float*>(y), total, split, M, HWo, relu);
}

Div30 div30_of(int d) {
  int l = 0;
  while ((1LL << l) < d) ++l;
  return Div30{unsigned((((1ULL << l) - unsigned(d)) << 32) / unsigned(d) + 1), l};
}

// The 32-bit kernel forms index partial[z * total + i] (i < total rounded up to a quad) and the magic-number
// divisions need n < 2^30: both hold when (total + 4) * split < 2^31 and total + 4 < 2^30.
bool narrow_indices(long long total, int split) {
  return total + 4 < (1LL << 30) && (total + 4) * static_cast<long long>(split) < (1LL << 31);
}

// The compile-time slice count of the 32-bit vectorised form (0: any split, loads issued eight at a time).
int unrolled_split(int split) { return split == 1 || split == 2 || split == 4 || split == 8 ? split : 0; }

template <typename E>
void launch(const float* partial, const void* bias, void* y, long long total, int split, int M, int HWo, int relu,
            hipStream_t s) {
  long long blocks = ((total + 3) / 4 + kThreads - 1) / kThreads;
  if (blocks > (1 << 20)) blocks = 1 << 20;
  const bool vec = (total % 4) == 0 && (reinterpret_cast<uintptr_t>(partial) & 15u) == 0;
  const auto b16 = static_cast<const uint16_t*>(bias);
  const auto y16 = static_cast<uint16_t*>(y);
  if (narrow_indices(total, split)) {
    const Div30 dh = div30_of(HWo), dm = div30_of(M);
    auto go = [&](auto fn) {
      hipLaunchKernelGGL(fn, dim3(unsigned(blocks)), dim3(kThreads), 0, s, partial, b16, y16, int(total), split, M,
                         HWo, dh, dm, relu);
    };
    switch (vec ? unrolled_split(split) : -1) {
      case -1: go(splitk_reduce_kernel<E, false, 0>); break;
      case 1: go(splitk_reduce_kernel<E, true, 1>); break;
      case 2: go(splitk_reduce_kernel<E, true, 2>); break;
      case 4: go(splitk_reduce_kernel<E, true, 4>); break;
      case 8: go(splitk_reduce_kernel<E, true, 8>); break;
      default: go(splitk_reduce_kernel<E, true, 0>); break;
    }
  } else if (vec) {
    hipLaunchKernelGGL((splitk_reduce_wide_kernel<E, true>), dim3(unsigned(blocks)), dim3(kThreads), 0, s, partial,
                       b16, y16, total, split, M, HWo, relu);
  } else {
    hipLaunchKernelGGL((splitk_reduce_wide_kernel<E, false>), dim3(unsigned(blocks)), dim3(kThreads), 0, s, partial,
                       b16, y16, total, split, M, HWo, relu);
  }
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_splitk_reduce_form(int dtype, int64_t total, int split, int vec, int* index_bits,
                                          int* slices_unrolled) {
  if (total <= 0 || split < 1 || !index_bits || !slices_unrolled) return GIE_HIP_EINVAL;
  if (dtype == GIE_HIP_FP32 || dtype == GIE_HIP_TF32) {
    *index_bits = 64;
    *slices_unrolled = 0;
    return GIE_HIP_OK;
  }
  if (dtype != GIE_HIP_FP16 && dtype != GIE_HIP_BF16) return GIE_HIP_EUNSUPPORTED;
  const bool narrow = narrow_indices(total, split);
  *index_bits = narrow ? 32 : 64;
  *slices_unrolled = narrow && vec ? unrolled_split(split) : 0;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_splitk_reduce(int dtype, const float* partial, const void* bias, void* y, int64_t total,
                                     int split, int out_channels, int hw_out, int relu, void* stream) {
  if (!partial || !y || total <= 0 || split < 1 || out_channels <= 0 || hw_out <= 0) return GIE_HIP_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GIE_HIP_FP16)
    launch<Fp16>(partial, bias, y, total, split, out_channels, hw_out, relu ? 1 : 0, s);
  else if (dtype == GIE_HIP_BF16)
    launch<Bf16>(partial, bias, y, total, split, out_channels, hw_out, relu ? 1 : 0, s);
  else if (dtype == GIE_HIP_FP32 || dtype == GIE_HIP_TF32)
    launch_f32(partial, bias, y, total, split, out_channels, hw_out, relu ? 1 : 0, s);
  else
    return GIE_HIP_EUNSUPPORTED;
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
