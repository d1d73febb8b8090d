// Stand-alone bias / ReLU passes over an NCHW output (the reference's src/kernels/elementwise.cu:13-56): the
// unfused side of the epilogue-fusion experiment. y[i] = round(relu?(f32(y[i]) + f32(bias[c(i)]))) in place,
// c(i) = (i / hw_out) % out_channels. Each pass reads and writes the whole tensor, which is the traffic the
// fused epilogue of the convolution kernels saves. HBM-bound: every thread owns one 16-byte chunk (8 halves or
// 4 floats) and walks its channel index incrementally, so there is one integer division per chunk.
#include "device_common.h"

namespace gie_hip {
namespace {

constexpr int kThreads = 256;

struct F32 {};  // 4-byte storage, no conversion

// storage bytes of an element tag
template <typename E>
constexpr int kBytes = 2;
template <>
constexpr int kBytes<F32> = 4;

template <typename E>
__device__ __forceinline__ float load_f(const void* p, long long i) {
  if constexpr (kBytes<E> == 4)
    return static_cast<const float*>(p)[i];
  else
    return E::to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <typename E>
__device__ __forceinline__ void store_f(void* p, long long i, float v) {
  if constexpr (kBytes<E> == 4)
    static_cast<float*>(p)[i] = v;
  else
    static_cast<uint16_t*>(p)[i] = E::from_f32(v);
}

// kVec: y 16-byte aligned and total a multiple of the chunk, so every chunk is one aligned 16-byte access
template <typename E, bool kVec>
__global__ __launch_bounds__(kThreads) void bias_act_kernel(void* __restrict__ y, const void* __restrict__ bias,
                                                            long long total, int O, int HWo, int relu) {
  constexpr int kChunk = 16 / kBytes<E>;
  const long long chunks = (total + kChunk - 1) / kChunk;
  for (long long ci = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; ci < chunks;
       ci += static_cast<long long>(gridDim.x) * kThreads) {
    const long long i0 = ci * kChunk;
    const long long plane = i0 / HWo;
    int c = int(plane % O);
    int r = int(i0 - plane * HWo);
    float v[kChunk];
    if (kVec) {
      const u32x4 raw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(y) + i0 * kBytes<E>);
      if constexpr (kBytes<E> == 4) {
        for (int e = 0; e < kChunk; ++e) v[e] = __uint_as_float(raw[e]);
      } else {
        for (int e = 0; e < kChunk; ++e) v[e] = E::to_f32(uint16_t(raw[e / 2] >> (16 * (e & 1))));
      }
    } else {
      for (int e = 0; e < kChunk; ++e) v[e] = i0 + e < total ? load_f<E>(y, i0 + e) : 0.f;
    }
    for (int e = 0; e < kChunk; ++e) {
      if (bias) v[e] += load_f<E>(bias, c);
      if (relu) v[e] = fmaxf(v[e], 0.f);
      if (++r == HWo) {
        r = 0;
        c = c + 1 == O ? 0 : c + 1;
      }
    }
    if (kVec) {
      u32x4 out;
      if constexpr (kBytes<E> == 4) {
        for (int e = 0; e < kChunk; ++e) out[e] = __float_as_uint(v[e]);
      } else {
        for (int e = 0; e < 4; ++e)
          out[e] = uint32_t(E::from_f32(v[2 * e])) | (uint32_t(E::from_f32(v[2 * e + 1])) << 16);
      }
      *reinterpret_cast<u32x4*>(static_cast<char*>(y) + i0 * kBytes<E>) = out;
    } else {
      for (int e = 0; e < kChunk; ++e)
        if (i0 + e < total) store_f<E>(y, i0 + e, v[e]);
    }
  }
}

template <typename E>
void launch(void* y, const void* bias, long long total, int O, int HWo, int relu, hipStream_t s) {
  constexpr int kChunk = 16 / kBytes<E>;
  long long blocks = ((total + kChunk - 1) / kChunk + kThreads - 1) / kThreads;
  if (blocks > (1 << 20)) blocks = 1 << 20;
  const bool vec = total % kChunk == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
  if (vec)
    hipLaunchKernelGGL((bias_act_kernel<E, true>), dim3(unsigned(blocks)), dim3(kThreads), 0, s, y, bias, total, O,
                       HWo, relu);
  else
    hipLaunchKernelGGL((bias_act_kernel<E, false>), dim3(unsigned(blocks)), dim3(kThreads), 0, s, y, bias, total, O,
                       HWo, relu);
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_bias_act(int dtype, void* y, const void* bias, int64_t total, int out_channels, int hw_out,
                                int relu, void* stream) {
  if (!y || total <= 0 || out_channels <= 0 || hw_out <= 0) return GIE_HIP_EINVAL;
  if (!bias && !relu) return GIE_HIP_OK;
  const size_t esz = dtype == GIE_HIP_FP32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(y) % esz) != 0 || (bias && reinterpret_cast<uintptr_t>(bias) % esz != 0))
    return GIE_HIP_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int r = relu ? 1 : 0;
  if (dtype == GIE_HIP_FP32)
    launch<F32>(y, bias, total, out_channels, hw_out, r, s);
  else if (dtype == GIE_HIP_FP16)
    launch<Fp16>(y, bias, total, out_channels, hw_out, r, s);
  else if (dtype == GIE_HIP_BF16)
    launch<Bf16>(y, bias, total, out_channels, hw_out, r, s);
  else
    return GIE_HIP_EUNSUPPORTED;
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
