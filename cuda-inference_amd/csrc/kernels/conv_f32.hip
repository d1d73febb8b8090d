// FP32 and TF32 convolution on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32: FP32 operands, FP32
// accumulation), straight from the caller's NCHW x and OIHW w — the strict-FP32 GPU path, the role of the
// reference's SIMT implicit GEMM (src/kernels/implicit_gemm.cu:47-189) and of its TF32 tensor-core path.
//
// GEMM view: M = output channels (A = weights), N = B*OH*OW output pixels (B = gathered activations), K walked as
// (filter tap, 16-channel chunk) so one stage reads 16 channels of one tap: the tap's row/column offset and its
// padding test are per stage, the channel step is a plain stride of H*W. A workgroup (4 waves) computes BM filters
// x 128 pixels; each wave a (BM/2) x 64 quarter as 32x32 MFMA blocks. Each stage is loaded to registers one stage
// ahead (out-of-range taps, channels, filters and pixels load as zero), written to LDS as [k][m] and [k][n] rows
// (row pitch tile + 32 floats, so the two 32-lane halves of a wave, which read rows k and k+1, hit disjoint
// banks), and consumed as 8 MFMA k-steps. The epilogue writes NCHW directly: the 32 lanes of a half-wave hold 32
// consecutive pixels of one filter, so each store instruction covers whole 128-byte runs.
//
// TF32: every operand is rounded to TF32 (10 mantissa bits, round to nearest, ties away from zero, the reference's
// round_to_tf32, src/runtime/reference.cu:143-146) as it is written to LDS. A product of two TF32 values is exact
// in FP32, so the MFMA then computes what a TF32 tensor core computes: exact products, FP32 sums.
#include "device_common.h"

namespace gie_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kBN = 128;  // output pixels per workgroup
constexpr int kBK = 16;   // channels per stage (one filter tap)
constexpr int kPad = 32;  // LDS row pitch = tile + 32 floats

struct F32Geom {
  int C, H, W, O, KW;
  int SH, SW, PH, PW, OW;
  int HW, OHW, CRS, RS;
  int N;     // B*OH*OW
  int n_cc;  // ceil(C / 16)
  int T;     // RS * n_cc stages
  int relu;
};

__device__ __forceinline__ float round_tf32(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7f800000u) != 0x7f800000u) u = (u + 0x1000u) & 0xffffe000u;  // Inf/NaN pass through
  return __uint_as_float(u);
}

template <int BM, bool TF32>
__global__ __launch_bounds__(kThreads) void f32_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       const float* __restrict__ bias, float* __restrict__ y,
                                                       float* __restrict__ partial, int split, F32Geom g) {
  constexpr int MP = BM + kPad, NP = kBN + kPad;
  constexpr int A_PER = BM * kBK / kThreads;  // weight elements per thread per stage
  constexpr int A_STEP = kThreads / BM;       // K rows between them
  constexpr int B_PER = kBN * kBK / kThreads;
  constexpr int MB = BM / 64;  // 32-row MFMA blocks per wave along M
  static_assert(A_PER * A_STEP == kBK && B_PER * 2 == kBK, "stage split");
  __shared__ float As[2][kBK][MP];
  __shared__ float Bs[2][kBK][NP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * kBN, z = blockIdx.z;
  const int t_begin = int((long long)g.T * z / split), t_end = int((long long)g.T * (z + 1) / split);

  // the gather pixel of this thread (fixed for the whole K loop) and its weight row
  const int bn = tid % kBN, bk0 = tid / kBN;
  const int ng = n0 + bn;
  const bool n_ok = ng < g.N;
  int ih0 = 0, iw0 = 0, xpix = 0;
  if (n_ok) {
    const int b = ng / g.OHW, p = ng - b * g.OHW;
    const int oh = p / g.OW, ow = p - oh * g.OW;
    ih0 = oh * g.SH - g.PH;
    iw0 = ow * g.SW - g.PW;
    xpix = b * g.C * g.HW + ih0 * g.W + iw0;  // only dereferenced with the tap's offset inside the image
  }
  const int am = tid % BM, ak0 = tid / BM;
  const bool o_ok = m0 + am < g.O;
  const int wrow = o_ok ? (m0 + am) * g.CRS : 0;

  float ra[A_PER], rb[B_PER];
  auto load = [&](int t) {
    const int tap = t / g.n_cc, cc = t - tap * g.n_cc;
    const int r = tap / g.KW, s = tap - r * g.KW;
    const int c0 = cc * kBK;
    const bool pix = n_ok && unsigned(ih0 + r) < unsigned(g.H) && unsigned(iw0 + s) < unsigned(g.W);
    const int xo = xpix + r * g.W + s;
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = c0 + bk0 + 2 * i;
      rb[i] = (pix && c < g.C) ? x[xo + c * g.HW] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int c = c0 + ak0 + A_STEP * i;
      ra[i] = (o_ok && c < g.C) ? w[wrow + c * g.RS + tap] : 0.f;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < B_PER; ++i) Bs[buf][bk0 + 2 * i][bn] = TF32 ? round_tf32(rb[i]) : rb[i];
#pragma unroll
    for (int i = 0; i < A_PER; ++i) As[buf][ak0 + A_STEP * i][am] = TF32 ? round_tf32(ra[i]) : ra[i];
  };

  f32x16 acc[MB][2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = f32x16{};

  const int half = lane >> 5, col = lane & 31;
  auto compute = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kBK / 2; ++j) {
      const int kr = 2 * j + half;  // MFMA 32x32x2: lanes 0-31 carry k = 0, lanes 32-63 k = 1
      float a[MB], b[2];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) a[mb] = As[buf][kr][wm * (BM / 2) + mb * 32 + col];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) b[nb] = Bs[buf][kr][wn * 64 + nb * 32 + col];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[mb], b[nb], acc[mb][nb], 0, 0, 0);
    }
  };

  if (t_begin < t_end) {
    load(t_begin);
    store(0);
    __syncthreads();
    for (int t = t_begin; t < t_end; ++t) {
      const int buf = (t - t_begin) & 1;
      if (t + 1 < t_end) load(t + 1);
      compute(buf);
      // the other buffer was last read in the previous iteration, before that iteration's barrier
      if (t + 1 < t_end) store(buf ^ 1);
      __syncthreads();
    }
  }

  // accumulator register r of lane l: filter row 8*(r/4) + 4*(l/32) + r%4 of the block, pixel column l%32
  const long long total = (long long)g.N * g.O;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = n0 + wn * 64 + nb * 32 + col;
    if (n >= g.N) continue;
    const int b = n / g.OHW, p = n - b * g.OHW;
    const int ybase = b * g.O * g.OHW + p;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int o = m0 + wm * (BM / 2) + mb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (o >= g.O) continue;
        float v = acc[mb][nb][r];
        const int yi = ybase + o * g.OHW;
        if (split > 1) {
          partial[(long long)z * total + yi] = v;
        } else {
          if (bias) v += bias[o];
          if (g.relu) v = fmaxf(v, 0.f);
          y[yi] = v;
        }
      }
    }
  }
}

constexpr int kTileM[] = {128, 64};
constexpr int kConfigs = 2;

bool fits_32bit(const gie_conv_geom* g) {
  const long long lim = (1LL << 31) - 1;
  const long long xs = 1LL * g->batch * g->in_channels * g->in_h * g->in_w;
  const long long ws = 1LL * g->out_channels * g->in_channels * g->kernel_h * g->kernel_w;
  const long long ys = 1LL * g->batch * g->out_channels * g->out_h * g->out_w;
  return xs <= lim && ws <= lim && ys <= lim;
}

F32Geom make_geom(const gie_conv_geom* g) {
  F32Geom f;
  f.C = g->in_channels;
  f.H = g->in_h;
  f.W = g->in_w;
  f.O = g->out_channels;
  f.KW = g->kernel_w;
  f.SH = g->stride_h;
  f.SW = g->stride_w;
  f.PH = g->pad_h;
  f.PW = g->pad_w;
  f.OW = g->out_w;
  f.HW = g->in_h * g->in_w;
  f.OHW = g->out_h * g->out_w;
  f.RS = g->kernel_h * g->kernel_w;
  f.CRS = f.C * f.RS;
  f.N = g->batch * f.OHW;
  f.n_cc = (f.C + kBK - 1) / kBK;
  f.T = f.RS * f.n_cc;
  f.relu = g->relu ? 1 : 0;
  return f;
}

template <int BM, bool TF32>
void launch(const F32Geom& f, const float* x, const float* w, const float* bias, float* y, float* partial,
            int split, hipStream_t s) {
  const dim3 grid(unsigned((f.N + kBN - 1) / kBN), unsigned((f.O + BM - 1) / BM), unsigned(split));
  hipLaunchKernelGGL((f32_kernel<BM, TF32>), grid, dim3(kThreads), 0, s, x, w, bias, y, partial, split, f);
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_f32_config_count(void) { return kConfigs; }

extern "C" int gie_hip_f32_config_tile_m(int config) {
  return config >= 0 && config < kConfigs ? kTileM[config] : GIE_HIP_EINVAL;
}

extern "C" int gie_hip_f32_check(int config, const gie_conv_geom* g, int* stages) {
  if (!g || config < 0 || config >= kConfigs) return GIE_HIP_EINVAL;
  if (g->batch <= 0 || g->in_channels <= 0 || g->in_h <= 0 || g->in_w <= 0 || g->out_channels <= 0 ||
      g->kernel_h <= 0 || g->kernel_w <= 0 || g->stride_h <= 0 || g->stride_w <= 0 || g->pad_h < 0 || g->pad_w < 0 ||
      g->out_h <= 0 || g->out_w <= 0)
    return GIE_HIP_EINVAL;
  if (!fits_32bit(g)) return GIE_HIP_EUNSUPPORTED;
  const long long n = 1LL * g->batch * g->out_h * g->out_w;
  if ((n + kBN - 1) / kBN > 0x7fffffffLL || (g->out_channels + kTileM[config] - 1) / kTileM[config] > 65535)
    return GIE_HIP_EUNSUPPORTED;
  if (stages) *stages = make_geom(g).T;
  return GIE_HIP_OK;
}

extern "C" int gie_hip_conv_f32(int config, int dtype, const gie_conv_geom* g, const void* x, const void* w,
                                const void* bias, void* y, float* partial, int split, void* stream) {
  const int rc = gie_hip_f32_check(config, g, nullptr);
  if (rc != GIE_HIP_OK) return rc;
  if (dtype != GIE_HIP_FP32 && dtype != GIE_HIP_TF32) return GIE_HIP_EUNSUPPORTED;
  if (!x || !w || !y) return GIE_HIP_EINVAL;
  auto a4 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; };
  if (!a4(x) || !a4(w) || !a4(y) || (bias && !a4(bias))) return GIE_HIP_EINVAL;
  const F32Geom f = make_geom(g);
  if (split < 1 || split > f.T) return GIE_HIP_EINVAL;
  if (split > 1 && (!partial || !a4(partial))) return GIE_HIP_EINVAL;
  const float *xf = static_cast<const float*>(x), *wf = static_cast<const float*>(w);
  const float* bf = static_cast<const float*>(bias);
  float* yf = static_cast<float*>(y);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool tf32 = dtype == GIE_HIP_TF32;
  if (config == 0)
    tf32 ? launch<128, true>(f, xf, wf, bf, yf, partial, split, s) : launch<128, false>(f, xf, wf, bf, yf, partial, split, s);
  else
    tf32 ? launch<64, true>(f, xf, wf, bf, yf, partial, split, s) : launch<64, false>(f, xf, wf, bf, yf, partial, split, s);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}
