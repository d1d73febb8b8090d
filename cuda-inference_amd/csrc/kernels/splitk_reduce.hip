// Split-K reduction + fused epilogue: y[i] = round(relu?(sum_z partial[z][i] + bias[c(i)])), summing the FP32
// partial slices in ascending z (the reference's order, src/kernels/tensor_core_mma.cu:254-262) so results are
// deterministic run to run. HBM-bound: reads split*4 B and writes 2 B per output. Each thread owns 4
// consecutive outputs: 16-byte partial loads (when every slice start is 16-byte aligned) and one 8-byte store
// when the destination allows it; a grid-stride loop keeps the grid bounded.
#include "device_common.h"

namespace gie_hip {
namespace {

constexpr int kThreads = 256;

template <typename E, bool kVec>
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(const float* __restrict__ partial,
                                                                 const uint16_t* __restrict__ bias,
                                                                 uint16_t* __restrict__ y, long long total, int split,
                                                                 int M, int HWo, int relu) {
  const long long quads = (total + 3) / 4;
  for (long long qi = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; qi < quads;
       qi += static_cast<long long>(gridDim.x) * kThreads) {
    const long long i0 = qi * 4;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if (kVec) {  // total % 4 == 0: every slice is 16-byte aligned and the quad is whole
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

template <typename E>
void launch(const float* partial, const void* bias, void* y, long long total, int split, int M, int HWo, int relu,
            hipStream_t s) {
  long long blocks = ((total + 3) / 4 + kThreads - 1) / kThreads;
  if (blocks > (1 << 20)) blocks = 1 << 20;
  const bool vec = (total % 4) == 0 && (reinterpret_cast<uintptr_t>(partial) & 15u) == 0;
  if (vec)
    hipLaunchKernelGGL((splitk_reduce_kernel<E, true>), dim3(unsigned(blocks)), dim3(kThreads), 0, s, partial,
                       static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), total, split, M, HWo, relu);
  else
    hipLaunchKernelGGL((splitk_reduce_kernel<E, false>), dim3(unsigned(blocks)), dim3(kThreads), 0, s, partial,
                       static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y), total, split, M, HWo, relu);
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

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
