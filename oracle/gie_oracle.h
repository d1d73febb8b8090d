/* TEST INFRASTRUCTURE ONLY — CPU oracle for the fused Conv2D hot path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only
 * as the checker / CPU baseline. The product library (cuda-inference_amd/) never links or calls it.
 *
 * Plain-C restatement of the reference's CPU-side algorithms (paths relative to the reference checkout):
 *   conv + scale          src/cpu/cpu_reference.cpp:13-56
 *   validate_problem      src/runtime/conv2d.cpp:83-109
 *   output size / flops   include/gpu_inference/conv2d.h:55-64
 *   quantize_to           src/runtime/reference.cu:106-114 (IEEE-754 RNE written from the standard)
 *   TolerancePolicy       src/runtime/reference.cu:139-167
 *   compare_outputs       src/runtime/reference.cu:176-200
 *   Rng (SplitMix64)      src/runtime/testing.cu:12-24
 *   make_conv_data        src/runtime/testing.cu:63-105 (draw order x, w, bias)
 *   transpose_c_hw        src/kernels/tensor_core_mma.cu:61-82,309-310 (activation / weight repack)
 *   build_conv_lut       src/kernels/conv_common.cu:22-37
 *   build_conv_lut_chunked src/kernels/conv_common.cu:39-50
 *   split-K partition     src/kernels/tensor_core_mma.cu:112-115
 *   splitk_reduce         src/kernels/tensor_core_mma.cu:254-262
 *
 * How each function is pinned (not by retyping its formula): see tests/test_oracle.py — the reference's
 * known-answer tests (tests/test_cpu_reference.cpp), brute force on tiny inputs through an independent
 * formulation, numpy's IEEE float16 for FP16 rounding, exhaustive bf16 rounding against an integer
 * restatement, SplitMix64 against its published first outputs, and permutation invariants.
 */
#ifndef GIE_ORACLE_H_
#define GIE_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gie_oracle_params {
  int batch, in_channels, in_h, in_w, out_channels, kernel_h, kernel_w;
  int stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups;
} gie_oracle_params;

enum { GIE_ORACLE_FP32 = 0, GIE_ORACLE_FP16 = 1, GIE_ORACLE_BF16 = 2, GIE_ORACLE_TF32 = 3 };
enum { GIE_ORACLE_OK = 0, GIE_ORACLE_INVALID = 1, GIE_ORACLE_UNSUPPORTED = 2 };
enum { GIE_DIST_UNIFORM = 0, GIE_DIST_NORMAL = 1, GIE_DIST_SPARSE = 2, GIE_DIST_POSITIVE = 3 };
/* scaling of the drawn values: the reference's make_conv_data (w * sqrt(3/K), bias U(-1,1)) or the
   benchmark spec (w * 1/sqrt(K), bias U(-0.1,0.1)). */
enum { GIE_SCALING_REFERENCE = 0, GIE_SCALING_BENCH = 1 };

int gie_oracle_out_h(const gie_oracle_params* p);
int gie_oracle_out_w(const gie_oracle_params* p);
int gie_oracle_validate(const gie_oracle_params* p);

/* y, scale: float[B*O*OH*OW] NCHW. Returns the validate code (nothing is written unless 0). */
int gie_oracle_conv2d(const gie_oracle_params* p, int has_bias, int relu, const float* x, const float* w,
                      const float* bias, float* y, float* scale, int threads);

/* the same computation for a list of NCHW output indices only (y, scale: float[n]) */
int gie_oracle_conv2d_points(const gie_oracle_params* p, int has_bias, int relu, const float* x, const float* w,
                             const float* bias, const int64_t* idx, int64_t n, float* y, float* scale, int threads);

uint16_t gie_oracle_f32_to_f16(float v);
float gie_oracle_f16_to_f32(uint16_t h);
uint16_t gie_oracle_f32_to_bf16(float v);
float gie_oracle_bf16_to_f32(uint16_t h);
float gie_oracle_round_tf32(float v);
float gie_oracle_quantize(int precision, float v);
void gie_oracle_quantize_array(int precision, const float* in, float* out, int64_t n);
/* storage bits of a quantized array (fp16 / bf16 only) */
void gie_oracle_to_bits(int precision, const float* in, uint16_t* out, int64_t n);
void gie_oracle_from_bits(int precision, const uint16_t* in, float* out, int64_t n);

uint64_t gie_oracle_splitmix64(uint64_t* state);
double gie_oracle_uniform01(uint64_t* state);
/* Draws x (NCHW), then w (OIHW), then bias (O) from one SplitMix64 stream and quantizes them to
   `precision` (values already rounded; TF32 leaves storage raw and rounds the multiplier view). */
int gie_oracle_make_data(const gie_oracle_params* p, int precision, uint64_t seed, int dist, int scaling,
                         float* x, float* w, float* bias);

typedef struct gie_oracle_metrics {
  int64_t n, over_tol, nan_count, inf_count;
  double max_abs, mean_abs, rms, max_rel, frac_over_tol, worst_tol_ratio;
  double rel_l2; /* ||test-ref||_2 / ||ref||_2 (benchmark gate, not part of the reference's metrics) */
} gie_oracle_metrics;

double gie_oracle_tol(int precision, int64_t k, int intermediate_rounding, double ref, double scale);
void gie_oracle_compare(const float* test, const float* ref, const float* scale, int64_t n, int precision,
                        int64_t k, int intermediate_rounding, gie_oracle_metrics* m);

/* 16-bit permutation dst[b][hw][c] = src[b][c][hw]; channels c in [C, C_pad) are zero in dst. */
void gie_oracle_repack_c_hw(const uint16_t* src, uint16_t* dst, int batch, int C, int HW, int C_pad);

/* one entry per k (c-major): {c * H * W, r * dilation_h, s * dilation_w, 0}; out4 NULL: the count only */
int64_t gie_oracle_lut(const gie_oracle_params* p, int32_t* out4);

/* one entry per 8 consecutive k for (r,s,c) ordering: {c_off, r_off, s_off, 0} */
int64_t gie_oracle_lut_chunked(const gie_oracle_params* p, int32_t* out4);

void gie_oracle_splitk_range(int ktiles, int z, int split, int* begin, int* end);
/* y[i] = round(epilogue(sum_{z ascending} partial[z*total+i])) ; bias indexed by (i / HWo) % M */
void gie_oracle_splitk_reduce(const float* partial, const float* bias, float* y, int64_t total, int split, int M,
                              int HWo, int relu, int precision);

#ifdef __cplusplus
}
#endif
#endif
