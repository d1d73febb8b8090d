// Double-accumulation direct convolution on the GPU: the validation reference the autotuner checks every
// candidate against (as the reference's gpu_conv2d_reference, src/runtime/reference.cu:31-91). One output per
// thread in NCHW order; products and sums in double over (c, r, s) with padding taps skipped;
// scale = sqrt(sum (x*w)^2 + acc^2 + bias^2); bias, ReLU, one double -> float rounding. Not a product path.
#include "device_common.h"

namespace gie_hip {
namespace {

struct RefArgs {
  int B, C, H, W, O, KH, KW, SH, SW, PH, PW, OH, OW, relu;
};

template <int D>
__device__ __forceinline__ double load_as_double(const void* p, long long i) {
  if (D == GIE_HIP_FP32) return double(static_cast<const float*>(p)[i]);
  const uint16_t b = static_cast<const uint16_t*>(p)[i];
  return D == GIE_HIP_FP16 ? double(Fp16::to_f32(b)) : double(Bf16::to_f32(b));
}

template <int D>
__global__ __launch_bounds__(256) void reference_kernel(const void* __restrict__ x, const void* __restrict__ w,
                                                        const void* __restrict__ bias, float* __restrict__ y,
                                                        float* __restrict__ scale, RefArgs a) {
  const long long total = static_cast<long long>(a.B) * a.O * a.OH * a.OW;
  for (long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<long long>(gridDim.x) * blockDim.x) {
    const int ow = int(idx % a.OW);
    const int oh = int((idx / a.OW) % a.OH);
    const int o = int((idx / (static_cast<long long>(a.OW) * a.OH)) % a.O);
    const int b = int(idx / (static_cast<long long>(a.OW) * a.OH * a.O));
    double acc = 0.0, sumsq = 0.0;
    for (int c = 0; c < a.C; ++c) {
      for (int r = 0; r < a.KH; ++r) {
        const int ih = oh * a.SH - a.PH + r;
        if (ih < 0 || ih >= a.H) continue;
        for (int s = 0; s < a.KW; ++s) {
          const int iw = ow * a.SW - a.PW + s;
          if (iw < 0 || iw >= a.W) continue;
          const double xv = load_as_double<D>(x, ((static_cast<long long>(b) * a.C + c) * a.H + ih) * a.W + iw);
          const double wv = load_as_double<D>(w, ((static_cast<long long>(o) * a.C + c) * a.KH + r) * a.KW + s);
          const double pr = xv * wv;
          acc += pr;
          sumsq += pr * pr;
        }
      }
    }
    sumsq += acc * acc;
    if (bias != nullptr) {
      const double bv = load_as_double<D>(bias, o);
      acc += bv;
      sumsq += bv * bv;
    }
    if (a.relu && acc < 0.0) acc = 0.0;
    y[idx] = float(acc);
    scale[idx] = float(sqrt(sumsq));
  }
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_reference_conv(int dtype, const gie_conv_geom* g, const void* x, const void* w,
                                      const void* bias, float* y_ref, float* scale, void* stream) {
  if (!g || !x || !w || !y_ref || !scale) return GIE_HIP_EINVAL;
  RefArgs a{g->batch, g->in_channels, g->in_h, g->in_w, g->out_channels, g->kernel_h, g->kernel_w, g->stride_h,
            g->stride_w, g->pad_h, g->pad_w, g->out_h, g->out_w, g->relu ? 1 : 0};
  const long long total = static_cast<long long>(a.B) * a.O * a.OH * a.OW;
  if (total <= 0) return GIE_HIP_EINVAL;
  long long blocks = (total + 255) / 256;
  if (blocks > (1 << 22)) blocks = 1 << 22;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case GIE_HIP_FP32: hipLaunchKernelGGL(reference_kernel<GIE_HIP_FP32>, dim3(unsigned(blocks)), dim3(256), 0, s, x, w, bias, y_ref, scale, a); break;
    case GIE_HIP_FP16: hipLaunchKernelGGL(reference_kernel<GIE_HIP_FP16>, dim3(unsigned(blocks)), dim3(256), 0, s, x, w, bias, y_ref, scale, a); break;
    case GIE_HIP_BF16: hipLaunchKernelGGL(reference_kernel<GIE_HIP_BF16>, dim3(unsigned(blocks)), dim3(256), 0, s, x, w, bias, y_ref, scale, a); break;
    default: return GIE_HIP_EUNSUPPORTED;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
