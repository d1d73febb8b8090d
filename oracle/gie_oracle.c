/* TEST INFRASTRUCTURE ONLY — CPU oracle for the fused Conv2D hot path (see gie_oracle.h).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this code.
 * Compiled with plain gcc (-O2, no fast-math) so float arithmetic stays IEEE single precision. */
#include "gie_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static float u2f(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

/* conv2d.h:55-56 */
int gie_oracle_out_h(const gie_oracle_params* p) {
  return (p->in_h + 2 * p->pad_h - p->dilation_h * (p->kernel_h - 1) - 1) / p->stride_h + 1;
}
int gie_oracle_out_w(const gie_oracle_params* p) {
  return (p->in_w + 2 * p->pad_w - p->dilation_w * (p->kernel_w - 1) - 1) / p->stride_w + 1;
}

/* conv2d.cpp:83-109: same checks, same order, same status classes. */
int gie_oracle_validate(const gie_oracle_params* p) {
  const int64_t lim = 2147483647LL;
  if (p->batch <= 0 || p->in_channels <= 0 || p->in_h <= 0 || p->in_w <= 0 || p->out_channels <= 0 ||
      p->kernel_h <= 0 || p->kernel_w <= 0)
    return GIE_ORACLE_INVALID;
  if (p->stride_h <= 0 || p->stride_w <= 0) return GIE_ORACLE_INVALID;
  if (p->pad_h < 0 || p->pad_w < 0) return GIE_ORACLE_INVALID;
  if (p->dilation_h != 1 || p->dilation_w != 1) return GIE_ORACLE_UNSUPPORTED;
  if (p->groups != 1) return GIE_ORACLE_UNSUPPORTED;
  {
    const int64_t eff_h = (int64_t)p->dilation_h * (p->kernel_h - 1) + 1;
    const int64_t eff_w = (int64_t)p->dilation_w * (p->kernel_w - 1) + 1;
    if ((int64_t)p->in_h + 2 * (int64_t)p->pad_h < eff_h || (int64_t)p->in_w + 2 * (int64_t)p->pad_w < eff_w)
      return GIE_ORACLE_INVALID;
  }
  {
    const int oh = gie_oracle_out_h(p), ow = gie_oracle_out_w(p);
    if (oh <= 0 || ow <= 0) return GIE_ORACLE_INVALID;
    const int64_t gn = (int64_t)p->batch * oh * ow;
    const int64_t gk = (int64_t)p->in_channels * p->kernel_h * p->kernel_w;
    if (gn > lim || gk > lim || (int64_t)p->out_channels > lim) return GIE_ORACLE_INVALID;
    if ((int64_t)p->in_channels * p->in_h * p->in_w > lim) return GIE_ORACLE_INVALID;
    if ((int64_t)p->out_channels * oh * ow > lim) return GIE_ORACLE_INVALID;
  }
  return GIE_ORACLE_OK;
}

/* cpu_reference.cpp:13-56: one output at a time in NCHW order, double accumulation over (c, r, s) with
   padding taps skipped, scale = sqrt(sum (x*w)^2 + acc^2 + bias^2), bias, ReLU, one double->float round. */
static void conv_one(const gie_oracle_params* p, int has_bias, int relu, const float* x, const float* w,
                     const float* bias, int OH, int OW, int64_t idx, float* yo, float* so);

int gie_oracle_conv2d(const gie_oracle_params* p, int has_bias, int relu, const float* x, const float* w,
                      const float* bias, float* y, float* scale, int threads) {
  const int rc = gie_oracle_validate(p);
  if (rc != GIE_ORACLE_OK) return rc;
  const int OH = gie_oracle_out_h(p), OW = gie_oracle_out_w(p);
  const int64_t total = (int64_t)p->batch * p->out_channels * OH * OW;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
#else
  (void)threads;
#endif
  for (int64_t idx = 0; idx < total; ++idx) conv_one(p, has_bias, relu, x, w, bias, OH, OW, idx, &y[idx], &scale[idx]);
  return GIE_ORACLE_OK;
}

int gie_oracle_conv2d_points(const gie_oracle_params* p, int has_bias, int relu, const float* x, const float* w,
                             const float* bias, const int64_t* idx, int64_t n, float* y, float* scale, int threads) {
  const int rc = gie_oracle_validate(p);
  if (rc != GIE_ORACLE_OK) return rc;
  const int OH = gie_oracle_out_h(p), OW = gie_oracle_out_w(p);
  const int64_t total = (int64_t)p->batch * p->out_channels * OH * OW;
  for (int64_t i = 0; i < n; ++i)
    if (idx[i] < 0 || idx[i] >= total) return GIE_ORACLE_INVALID;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
#else
  (void)threads;
#endif
  for (int64_t i = 0; i < n; ++i) conv_one(p, has_bias, relu, x, w, bias, OH, OW, idx[i], &y[i], &scale[i]);
  return GIE_ORACLE_OK;
}

static void conv_one(const gie_oracle_params* p, int has_bias, int relu, const float* x, const float* w,
                     const float* bias, int OH, int OW, int64_t idx, float* yo, float* so) {
  {
    const int ow = (int)(idx % OW);
    const int oh = (int)((idx / OW) % OH);
    const int o = (int)((idx / ((int64_t)OW * OH)) % p->out_channels);
    const int b = (int)(idx / ((int64_t)OW * OH * p->out_channels));
    double acc = 0.0, sumsq = 0.0;
    for (int c = 0; c < p->in_channels; ++c) {
      for (int r = 0; r < p->kernel_h; ++r) {
        const int ih = oh * p->stride_h - p->pad_h + r * p->dilation_h;
        if (ih < 0 || ih >= p->in_h) continue;
        for (int s = 0; s < p->kernel_w; ++s) {
          const int iw = ow * p->stride_w - p->pad_w + s * p->dilation_w;
          if (iw < 0 || iw >= p->in_w) continue;
          const double xv = x[(((int64_t)b * p->in_channels + c) * p->in_h + ih) * p->in_w + iw];
          const double wv = w[(((int64_t)o * p->in_channels + c) * p->kernel_h + r) * p->kernel_w + s];
          acc += xv * wv;
          sumsq += xv * xv * wv * wv;
        }
      }
    }
    sumsq += acc * acc;
    if (has_bias && bias != NULL) {
      acc += (double)bias[o];
      sumsq += (double)bias[o] * (double)bias[o];
    }
    if (relu && acc < 0.0) acc = 0.0;
    *yo = (float)acc;
    *so = (float)sqrt(sumsq);
  }
}

/* ---- IEEE-754 binary16 / bfloat16 round-to-nearest-even, written from the format definitions ---- */
uint16_t gie_oracle_f32_to_f16(float v) {
  const uint32_t x = f2u(v);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  const uint32_t mant = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | (mant ? 0x7e00u : 0x7c00u));
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e >= 1) {
    uint32_t h = mant >> 13;
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign + (((uint32_t)e << 10) + h)); /* mantissa carry rolls into the exponent */
  }
  /* binary16 subnormal: value = m * 2^-24 */
  {
    const uint32_t full = exp ? (mant | 0x800000u) : mant;
    const int shift = 126 - (int)exp;
    if (shift > 24 || full == 0) return (uint16_t)sign;
    uint32_t m = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (m & 1u))) ++m;
    return (uint16_t)(sign | m);
  }
}

float gie_oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t mant = (uint32_t)h & 0x3ffu;
  if (exp == 0x1fu) return u2f(sign | 0x7f800000u | (mant << 13));
  if (exp == 0) {
    if (mant == 0) return u2f(sign);
    /* subnormal: exact as m * 2^-24 */
    const float mag = (float)mant * 5.9604644775390625e-08f;
    return sign ? -mag : mag;
  }
  return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

uint16_t gie_oracle_f32_to_bf16(float v) {
  const uint32_t x = f2u(v);
  if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu)) return (uint16_t)((x >> 16) | 0x0040u);
  const uint32_t lsb = (x >> 16) & 1u;
  return (uint16_t)((x + 0x7fffu + lsb) >> 16);
}

float gie_oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* reference.cu:95-104: round to nearest, ties away, 10 mantissa bits */
float gie_oracle_round_tf32(float v) {
  uint32_t bits = f2u(v);
  if ((bits & 0x7f800000u) == 0x7f800000u) return v;
  bits += 0x1000u;
  bits &= 0xffffe000u;
  return u2f(bits);
}

float gie_oracle_quantize(int precision, float v) {
  switch (precision) {
    case GIE_ORACLE_FP16: return gie_oracle_f16_to_f32(gie_oracle_f32_to_f16(v));
    case GIE_ORACLE_BF16: return gie_oracle_bf16_to_f32(gie_oracle_f32_to_bf16(v));
    case GIE_ORACLE_TF32: return gie_oracle_round_tf32(v);
    default: return v;
  }
}

void gie_oracle_quantize_array(int precision, const float* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = gie_oracle_quantize(precision, in[i]);
}

void gie_oracle_to_bits(int precision, const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = precision == GIE_ORACLE_BF16 ? gie_oracle_f32_to_bf16(in[i]) : gie_oracle_f32_to_f16(in[i]);
}

void gie_oracle_from_bits(int precision, const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = precision == GIE_ORACLE_BF16 ? gie_oracle_bf16_to_f32(in[i]) : gie_oracle_f16_to_f32(in[i]);
}

/* ---- testing.cu:12-24 SplitMix64 and its derived draws ---- */
uint64_t gie_oracle_splitmix64(uint64_t* s) {
  uint64_t z = (*s += 0x9e3779b97f4a7c15ULL);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

double gie_oracle_uniform01(uint64_t* s) { return (double)(gie_oracle_splitmix64(s) >> 11) * (1.0 / 9007199254740992.0); }

static float uniform_lohi(uint64_t* s, float lo, float hi) { return lo + (float)gie_oracle_uniform01(s) * (hi - lo); }

static float draw(uint64_t* s, int dist) {
  switch (dist) {
    case GIE_DIST_NORMAL: {
      double acc = 0;
      for (int i = 0; i < 12; ++i) acc += gie_oracle_uniform01(s);
      return (float)(acc - 6.0);
    }
    case GIE_DIST_SPARSE: return gie_oracle_uniform01(s) < 0.7 ? 0.f : uniform_lohi(s, -2.f, 2.f);
    case GIE_DIST_POSITIVE: return uniform_lohi(s, 0.f, 1.f);
    default: return uniform_lohi(s, -1.f, 1.f);
  }
}

/* testing.cu:75-105 draw order x (NCHW), w (OIHW), bias (O); then quantize to the storage type. */
int gie_oracle_make_data(const gie_oracle_params* p, int precision, uint64_t seed, int dist, int scaling,
                         float* x, float* w, float* bias) {
  const int rc = gie_oracle_validate(p);
  if (rc != GIE_ORACLE_OK) return rc;
  uint64_t s = seed;
  const int64_t nx = (int64_t)p->batch * p->in_channels * p->in_h * p->in_w;
  const int64_t nw = (int64_t)p->out_channels * p->in_channels * p->kernel_h * p->kernel_w;
  const int64_t k = (int64_t)p->in_channels * p->kernel_h * p->kernel_w;
  const float wscale = scaling == GIE_SCALING_BENCH ? 1.0f / sqrtf((float)k) : sqrtf(3.0f / (float)k);
  const float blim = scaling == GIE_SCALING_BENCH ? 0.1f : 1.0f;
  for (int64_t i = 0; i < nx; ++i) x[i] = draw(&s, dist);
  for (int64_t i = 0; i < nw; ++i) w[i] = draw(&s, dist) * wscale;
  for (int i = 0; i < p->out_channels; ++i) bias[i] = uniform_lohi(&s, -blim, blim);
  const int half = precision == GIE_ORACLE_FP16 || precision == GIE_ORACLE_BF16;
  for (int64_t i = 0; i < nx; ++i) x[i] = gie_oracle_quantize(precision, x[i]);
  for (int64_t i = 0; i < nw; ++i) w[i] = gie_oracle_quantize(precision, w[i]);
  if (half)
    for (int i = 0; i < p->out_channels; ++i) bias[i] = gie_oracle_quantize(precision, bias[i]);
  return GIE_ORACLE_OK;
}

/* ---- reference.cu:139-200 tolerance model and metrics ---- */
static double u_out_of(int precision) {
  switch (precision) {
    case GIE_ORACLE_FP16: return 4.8828125e-04;
    case GIE_ORACLE_BF16: return 3.90625e-03;
    default: return 5.9604644775390625e-08;
  }
}

double gie_oracle_tol(int precision, int64_t k, int intermediate_rounding, double ref, double scale) {
  const double c_acc = 8.0, c_out = 1.0, u_acc = 5.9604644775390625e-08, u_in = 0.00048828125;
  const double u_out = u_out_of(precision);
  const double c_inter = intermediate_rounding ? 1.0 : 0.0;
  const double c_in = precision == GIE_ORACLE_TF32 ? 8.0 : 0.0;
  const double floor_ = precision == GIE_ORACLE_FP16 ? 3.0e-8 : 1e-30;
  return c_acc * u_acc * sqrt((double)k) * scale + c_out * u_out * fabs(ref) + c_inter * u_out * scale +
         c_in * u_in * scale + floor_;
}

void gie_oracle_compare(const float* test, const float* ref, const float* scale, int64_t n, int precision,
                        int64_t k, int intermediate_rounding, gie_oracle_metrics* m) {
  memset(m, 0, sizeof(*m));
  m->n = n;
  double sum_abs = 0, sum_sq = 0, ref_sq = 0;
  for (int64_t i = 0; i < n; ++i) ref_sq += (double)ref[i] * (double)ref[i];
  double rel_floor = 1e-3 * sqrt(ref_sq / (double)(n > 1 ? n : 1));
  if (rel_floor < 1e-30) rel_floor = 1e-30;
  for (int64_t i = 0; i < n; ++i) {
    const double t = test[i];
    if (isnan(t)) { ++m->nan_count; continue; }
    if (isinf(t)) { ++m->inf_count; continue; }
    const double err = fabs(t - (double)ref[i]);
    sum_abs += err;
    sum_sq += err * err;
    if (err > m->max_abs) m->max_abs = err;
    {
      const double d = fabs((double)ref[i]) > rel_floor ? fabs((double)ref[i]) : rel_floor;
      if (err / d > m->max_rel) m->max_rel = err / d;
    }
    const double ti = gie_oracle_tol(precision, k, intermediate_rounding, ref[i], scale[i]);
    if (err / ti > m->worst_tol_ratio) m->worst_tol_ratio = err / ti;
    if (err > ti) ++m->over_tol;
  }
  m->mean_abs = n ? sum_abs / (double)n : 0;
  m->rms = n ? sqrt(sum_sq / (double)n) : 0;
  m->frac_over_tol = n ? (double)m->over_tol / (double)n : 0;
  m->rel_l2 = ref_sq > 0 ? sqrt(sum_sq / ref_sq) : sqrt(sum_sq);
}

/* ---- tensor_core_mma.cu:61-82 layout permutation (plus zero channel padding) ---- */
void gie_oracle_repack_c_hw(const uint16_t* src, uint16_t* dst, int batch, int C, int HW, int C_pad) {
  for (int b = 0; b < batch; ++b) {
    const uint16_t* s = src + (int64_t)b * C * HW;
    uint16_t* d = dst + (int64_t)b * C_pad * HW;
    for (int hw = 0; hw < HW; ++hw)
      for (int c = 0; c < C_pad; ++c) d[(int64_t)hw * C_pad + c] = c < C ? s[(int64_t)c * HW + hw] : 0;
  }
}

/* conv_common.cu:22-37: one entry per k, k = c * KH * KW + r * KW + s (the unchunked gather table) */
int64_t gie_oracle_lut(const gie_oracle_params* p, int32_t* out4) {
  const int khw = p->kernel_h * p->kernel_w;
  const int64_t n = (int64_t)p->in_channels * khw;
  if (out4 == NULL) return n;
  for (int64_t k = 0; k < n; ++k) {
    const int c = (int)(k / khw), rs = (int)(k % khw);
    out4[4 * k + 0] = (int32_t)((int64_t)c * p->in_h * p->in_w);
    out4[4 * k + 1] = (rs / p->kernel_w) * p->dilation_h;
    out4[4 * k + 2] = (rs % p->kernel_w) * p->dilation_w;
    out4[4 * k + 3] = 0;
  }
  return n;
}

/* conv_common.cu:39-50 with the channel count generalised to the padded count C_pad = in_channels here */
int64_t gie_oracle_lut_chunked(const gie_oracle_params* p, int32_t* out4) {
  if (p->in_channels % 8 != 0) return -1;
  const int cv = p->in_channels / 8;
  const int64_t chunks = (int64_t)p->in_channels * p->kernel_h * p->kernel_w / 8;
  if (out4 == NULL) return chunks;
  for (int64_t q = 0; q < chunks; ++q) {
    const int rs = (int)(q / cv);
    const int r = rs / p->kernel_w, s = rs % p->kernel_w;
    out4[4 * q + 0] = (int32_t)(8 * (q % cv));
    out4[4 * q + 1] = r * p->dilation_h;
    out4[4 * q + 2] = s * p->dilation_w;
    out4[4 * q + 3] = 0;
  }
  return chunks;
}

/* tensor_core_mma.cu:112-115 */
void gie_oracle_splitk_range(int ktiles, int z, int split, int* begin, int* end) {
  *begin = (int)(((int64_t)ktiles * z) / split);
  *end = (int)(((int64_t)ktiles * (z + 1)) / split);
}

/* tensor_core_mma.cu:254-262 with fused_epilogue.cuh:11-16: FP32 sum in ascending z, + bias, ReLU, one round */
void gie_oracle_splitk_reduce(const float* partial, const float* bias, float* y, int64_t total, int split, int M,
                              int HWo, int relu, int precision) {
  for (int64_t i = 0; i < total; ++i) {
    float s = 0.f;
    for (int z = 0; z < split; ++z) s += partial[(int64_t)z * total + i];
    if (bias) s += bias[(i / HWo) % M];
    if (relu) s = fmaxf(s, 0.0f);
    y[i] = gie_oracle_quantize(precision, s);
  }
}
