/* C-ABI of the MI355X (gfx950) Conv2D kernels — the drop-in boundary under the gie:: C++ plan API.
 *
 * The C++ runtime (KernelDesc::launch implementations) calls only these functions. Every entry point takes
 * plain device pointers, sizes and a hipStream_t passed as `void*`; none allocates, frees or synchronizes,
 * so a sequence of calls can be captured into a hipGraph. Exceptions never cross this boundary: each call
 * returns 0 on success, a negative GIE_HIP_E* code for a rejected argument, or a positive hipError_t from
 * the launch (the host wrapper turns both into gie::Error).
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   gie_hip_repack_act_nchw_to_nhwc  launch_transpose(x, xn, B, C, H*W)    src/kernels/tensor_core_mma.cu:78-82,309
 *   gie_hip_repack_w_oihw_to_orsc    launch_transpose(w, wk, O, C, KH*KW)  src/kernels/tensor_core_mma.cu:78-82,310
 *   gie_hip_conv_igemm               tcmma_kernel<<<>>> launch             src/kernels/tensor_core_mma.cu:99-251,311-316
 *   gie_hip_splitk_reduce            splitk_reduce<<<>>> launch            src/kernels/tensor_core_mma.cu:254-262,317-323
 *   gie_hip_igemm_config_*           the registered tile table             src/kernels/tensor_core_mma.cu:370-388
 *   gie_hip_igemm_occupancy          cudaOccupancyMaxActiveBlocksPerMultiprocessor in src/runtime/perf_model.cpp:75-102
 *   gie_hip_repack_blocked           both launch_transpose calls, one launch src/kernels/tensor_core_mma.cu:78-82,309-310
 *   gie_hip_conv_halo                tcmma_kernel<<<>>> launch (halo-tiled)  src/kernels/tensor_core_mma.cu:99-251,311-316
 *   gie_hip_halo_config_*, _check    the registered tile table / supports  src/kernels/tensor_core_mma.cu:280-295,370-388
 *   gie_hip_repack_w_blocked         launch_transpose(w, wk, O, C, KH*KW)  src/kernels/tensor_core_mma.cu:78-82,310
 *   gie_hip_conv_band                transpose_c_hw of x + tcmma_kernel, fused (no activation repack)
 *                                                                         src/kernels/tensor_core_mma.cu:61-82,99-251,309
 *   gie_hip_band_config_*, _check    the registered tile table / supports  src/kernels/tensor_core_mma.cu:280-295,370-388
 *   gie_hip_conv_pw, gie_hip_pw_check both transposes + tcmma_kernel for 1x1 filters, fused (no repack)
 *                                                                         src/kernels/tensor_core_mma.cu:61-82,99-251,309-316
 *   gie_hip_conv_pws, _pws_check     the same, weight-stationary streaming form for in_channels <= 256
 *   gie_hip_conv_stem, _stem_check   transposes + tcmma_kernel for the 7x7 stride-2 stem (in_channels <= 4), fused
 *   gie_hip_conv_narrow, _narrow_check transposes + tcmma_kernel (+ split-K reduce) for 3x3 layers with few pixels
 *                                                                         src/kernels/tensor_core_mma.cu:61-82,99-251,309-316
 *   gie_hip_conv_slab, _slab_check   both transposes + tcmma_kernel (split-K partials included) for 3x3 stride-1
 *                                    layers, fused: one launch straight from NCHW x / OIHW w
 *                                                                         src/kernels/tensor_core_mma.cu:61-82,99-251,297-324
 *   gie_hip_slab_config_*            the registered tile table             src/kernels/tensor_core_mma.cu:370-388
 *   gie_hip_conv_deep, _deep_check   both transposes + tcmma_kernel + splitk_reduce for 3x3 stride-1 layers over
 *                                    small images with long reductions, fused into one launch without split-K
 *   gie_hip_conv_stack, _stack_check both transposes + tcmma_kernel (split-K partials included) for 3x3 stride-1
 *                                    layers with small images and a long reduction, fused: one launch straight from
 *                                    NCHW x / OIHW w, images of a group stacked in one plane
 *                                                                         src/kernels/tensor_core_mma.cu:61-82,99-251,297-324
 *   gie_hip_stack_config_*           the registered tile table             src/kernels/tensor_core_mma.cu:370-388
 *   gie_hip_conv_f32, _f32_check     implicit_gemm_kernel<<<>>> launch (FP32) and the TF32 path
 *                                                                         src/kernels/implicit_gemm.cu:47-189,204-214
 *   gie_hip_f32_config_*             the registered FP32 tile table        src/kernels/implicit_gemm.cu:218-268
 *   gie_hip_bias_act                 launch_bias_act / _bias_add / _relu   src/kernels/elementwise.cu:13-56
 *   gie_hip_reference_conv           gpu_conv2d_reference                  src/runtime/reference.cu:31-91
 *   gie_hip_ceiling_*                ceilings microbenchmarks              src/profiling/ceilings.cu:21-58
 */
#ifndef GIE_HIP_H_
#define GIE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes (0 = ok, > 0 = hipError_t) */
#define GIE_HIP_OK 0
#define GIE_HIP_EINVAL (-1)      /* null pointer, bad size, shape the kernel's grid cannot cover */
#define GIE_HIP_EUNSUPPORTED (-2) /* valid request this kernel configuration cannot run */
#define GIE_HIP_ESCRATCH (-3)     /* request needs more than the library's static scratch */

/* element types; numbering follows gie::Precision (kFp32 = 0, kFp16 = 1, kBf16 = 2, kTf32 = 3). TF32 is FP32
   storage whose multiplier inputs are rounded to TF32 inside the kernel. */
#define GIE_HIP_FP32 0
#define GIE_HIP_FP16 1
#define GIE_HIP_BF16 2
#define GIE_HIP_TF32 3

/* Convolution geometry as the kernels see it (dilation and groups are 1, enforced by the host). */
typedef struct gie_conv_geom {
  int batch, in_channels, in_h, in_w;
  int out_channels, kernel_h, kernel_w;
  int stride_h, stride_w, pad_h, pad_w;
  int out_h, out_w;
  int c_pad; /* channel count of the repacked activation / weight buffers: multiple of 8, >= in_channels */
  int relu;  /* 1: ReLU after bias */
} gie_conv_geom;

/* One registered implicit-GEMM tile configuration. GEMM view as the reference names it:
   M = out_channels (tile_m), N = batch*out_h*out_w pixels (tile_n), K = kernel_h*kernel_w*c_pad (tile_k). */
typedef struct gie_igemm_config {
  int tile_m, tile_n, tile_k;
  int waves_m, waves_n; /* wave64 grid inside a workgroup */
  int threads;          /* waves_m * waves_n * 64 */
  int lds_bytes;        /* LDS per workgroup (two stages of the A and B tiles) */
  int stages;           /* K slices in flight in registers ahead of the LDS stage being multiplied */
  int version;          /* bumps when the kernel's code changes behaviour or speed */
} gie_igemm_config;

const char* gie_hip_status_string(int status);

/* x: [batch][channels][hw] 16-bit elements (any 2-byte alignment); xn: [batch][hw][c_pad], 16-byte aligned.
   xn[b][p][c] = x[b][c][p] for c < channels, 0 for channels <= c < c_pad. Bit-exact permutation. */
int gie_hip_repack_act_nchw_to_nhwc(const void* x, void* xn, int batch, int channels, int hw, int c_pad,
                                    void* stream);

/* w: [out_channels][channels][rs] (OIHW) -> wk: [out_channels][rs][c_pad], zero channel padding. */
int gie_hip_repack_w_oihw_to_orsc(const void* w, void* wk, int out_channels, int channels, int rs, int c_pad,
                                  void* stream);

/* The two repacks above in one launch (same results; one dispatch instead of two). */
int gie_hip_repack_act_and_w(const void* x, void* xn, const void* w, void* wk, const gie_conv_geom* g,
                             void* stream);

int gie_hip_igemm_config_count(void);
int gie_hip_igemm_config_get(int index, gie_igemm_config* out);
/* resident workgroups per CU for that configuration and element type */
int gie_hip_igemm_occupancy(int index, int dtype, int* blocks_per_cu);

/* Implicit-GEMM convolution on MFMA (FP16/BF16 storage, FP32 accumulation) over the repacked buffers.
   split == 1: y (NCHW, dtype, any 2-byte alignment) = round(relu?(acc + bias)) — one rounding.
   split  > 1: partial[z][NCHW index] = FP32 sum over the z-th slice of the K tiles
               [floor(kt*z/split), floor(kt*(z+1)/split)); y and bias are not touched (reduce below).
   bias may be null. partial must be 16-byte aligned and hold split*batch*out_channels*out_h*out_w floats. */
int gie_hip_conv_igemm(int config, int dtype, const gie_conv_geom* g, const void* xn, const void* wk,
                       const void* bias, void* y, float* partial, int split, void* stream);

/* One registered halo-tiled configuration: tile_m output channels x tile_n output pixels, channel slices of
   tile_k, filter kernel_h x kernel_w. */
typedef struct gie_halo_config {
  int tile_m, tile_n, tile_k;
  int kernel_h, kernel_w;
  int threads;
  int stages; /* LDS stages of the load pipeline */
  int version;
} gie_halo_config;

int gie_hip_halo_config_count(void);
int gie_hip_halo_config_get(int index, gie_halo_config* out);
/* 0 when configuration `config` runs geometry g, with the LDS bytes per workgroup in *lds_bytes;
   GIE_HIP_EUNSUPPORTED otherwise (other filter size, tile's input rows too large for the LDS stage, offsets
   beyond 32 bits). */
int gie_hip_halo_check(int config, const gie_conv_geom* g, int* lds_bytes);

/* Channel-blocked repack for the halo-tiled kernel, both tensors in one launch (S = ceil(in_channels / 32)):
   xb[b][s][h*w][32] = x[b][32s + l][h*w] and wb[o][s][kh*kw][32] = w[o][32s + l][kh*kw] for channel 32s + l
   < in_channels, 0 past it. x, w: caller tensors (any 2-byte alignment); xb, wb: 16-byte aligned. */
int gie_hip_repack_blocked(const void* x, void* xb, const void* w, void* wb, const gie_conv_geom* g, void* stream);

/* Halo-tiled implicit GEMM on MFMA 32x32x16 (FP32 accumulation) over the buffers of gie_hip_repack_blocked
   (xb, wb 16-byte aligned; g->c_pad is ignored): each input pixel is staged once per 32-channel slice and read by
   every tap from LDS. split == 1: y (NCHW, any 2-byte alignment) = round(relu?(acc + bias)), one rounding.
   split > 1: partial[z][NCHW index] = FP32 sum over the z-th range of channel slices [floor(S*z/split),
   floor(S*(z+1)/split)); reduce with gie_hip_splitk_reduce. split <= S. */
int gie_hip_conv_halo(int config, int dtype, const gie_conv_geom* g, const void* xb, const void* wb,
                      const void* bias, void* y, float* partial, int split, void* stream);

/* Weights only of gie_hip_repack_blocked: wb[o][s][kh*kw][32] = w[o][32s + l][kh*kw], zero past in_channels
   (w any 2-byte alignment, wb 16-byte aligned). Feeds gie_hip_conv_band, which reads activations as NCHW. */
int gie_hip_repack_w_blocked(const void* w, void* wb, const gie_conv_geom* g, void* stream);

/* One registered band configuration: tile_m (32) output channels x tile_n padded output pixels (one band of
   rows of one image), channel slices of tile_k, filter kernel_h x kernel_w. */
typedef struct gie_band_config {
  int tile_m, tile_n, tile_k;
  int kernel_h, kernel_w;
  int threads;
  int stages; /* LDS stages of the weight pipeline */
  int version;
} gie_band_config;

int gie_hip_band_config_count(void);
int gie_hip_band_config_get(int index, gie_band_config* out);
/* 0 when configuration `config` runs geometry g, with the LDS bytes per workgroup in *lds_bytes;
   GIE_HIP_EUNSUPPORTED otherwise (other filter size, band rows too wide for the LDS stage, offsets beyond
   32 bits). */
int gie_hip_band_check(int config, const gie_conv_geom* g, int* lds_bytes);

/* Band convolution on MFMA 32x32x16 (FP32 accumulation) reading x as NCHW directly (any 2-byte alignment;
   8-byte loads when x is 8-byte aligned and every band's rows start on a 4-pixel boundary) and the weights from
   gie_hip_repack_w_blocked (wb 16-byte aligned; g->c_pad is ignored). split == 1: y (NCHW, any 2-byte alignment)
   = round(relu?(acc + bias)), one rounding. split > 1: partial[z][NCHW index] = FP32 sum over channel slices
   [floor(S*z/split), floor(S*(z+1)/split)); reduce with gie_hip_splitk_reduce. split <= S. */
int gie_hip_conv_band(int config, int dtype, const gie_conv_geom* g, const void* x, const void* wb,
                      const void* bias, void* y, float* partial, int split, void* stream);

/* 0 when the pointwise kernel runs geometry g (1x1 filter, stride 1, no padding, in_channels % 8 == 0,
   in_h*in_w % 8 == 0, offsets within 32 bits), with its LDS bytes per workgroup in *lds_bytes. */
int gie_hip_pw_check(const gie_conv_geom* g, int* lds_bytes);

/* Pointwise convolution on MFMA 32x32x16 (FP32 accumulation) straight from the caller's tensors: x NCHW,
   w [out_channels][in_channels], y NCHW, all 16-byte aligned (GIE_HIP_EUNSUPPORTED otherwise), bias any 2-byte
   alignment or NULL. y = round(relu?(acc + bias)), one rounding. One launch, no workspace. */
int gie_hip_conv_pw(int dtype, const gie_conv_geom* g, const void* x, const void* w, const void* bias, void* y,
                    void* stream);

/* FP32 / TF32 convolution on MFMA 32x32x2 f32 (FP32 products and sums) straight from the caller's NCHW x and OIHW
   w (float, 4-byte aligned; no workspace). TF32 rounds every multiplier input to TF32 (round to nearest, ties away
   from zero) first. Configuration c computes tile_m(c) output channels x 128 pixels per workgroup.
   split == 1: y = relu?(acc + bias), NCHW float. split > 1: partial[z][NCHW index] = sum over the z-th range of
   the (tap, 16-channel chunk) stages [floor(T*z/split), floor(T*(z+1)/split)), T = kh*kw*ceil(C/16) (1 <= split
   <= T); reduce with gie_hip_splitk_reduce (dtype GIE_HIP_FP32). */
int gie_hip_f32_config_count(void);
int gie_hip_f32_config_tile_m(int config);
/* 0 when configuration `config` runs geometry g (offsets within 32 bits, grid limits), with T in *stages. */
int gie_hip_f32_check(int config, const gie_conv_geom* g, int* stages);
int gie_hip_conv_f32(int config, int dtype, const gie_conv_geom* g, const void* x, const void* w, const void* bias,
                     void* y, float* partial, int split, void* stream);

/* Weight-stationary streaming form of gie_hip_conv_pw for in_channels <= 256 (same operands and result; x and w
   16-byte aligned, y 8-byte aligned, GIE_HIP_EUNSUPPORTED otherwise): each workgroup holds 256 filters x C in
   registers and streams a contiguous range of 32-pixel blocks of the flattened batch*h*w axis. One launch, no
   workspace. *_check: 0 when the geometry qualifies, LDS bytes per workgroup in *lds_bytes. */
int gie_hip_pws_check(const gie_conv_geom* g, int* lds_bytes);
int gie_hip_conv_pws(int dtype, const gie_conv_geom* g, const void* x, const void* w, const void* bias, void* y,
                     void* stream);

/* Stem convolution straight from NCHW x / OIHW w: 7x7 filter, stride 2, padding 3, 1 <= in_channels <= 4,
   in_w % 16 == 0, fused bias + ReLU, dtype GIE_HIP_FP16 / _BF16 (x, w and y 16-byte aligned, bias 2-byte
   aligned; GIE_HIP_EUNSUPPORTED for other alignments or geometries). One launch, no workspace.
   *_check: 0 when the geometry qualifies, LDS bytes per workgroup in *lds_bytes. */
int gie_hip_stem_check(const gie_conv_geom* g, int* lds_bytes);
int gie_hip_conv_stem(int dtype, const gie_conv_geom* g, const void* x, const void* w, const void* bias, void* y,
                      void* stream);

/* Narrow convolution straight from NCHW x / OIHW w for 3x3, stride 1, padding 1 layers with in_channels % 128 == 0
   whose 32-pixel blocks touch few enough images to stage them in LDS (the whole reduction in one workgroup, no
   partials): fused bias + ReLU, dtype GIE_HIP_FP16 / _BF16 (x and w 16-byte aligned, y and bias 2-byte aligned;
   GIE_HIP_EUNSUPPORTED for other alignments or geometries). One launch, no workspace. *_check: 0 when the
   geometry qualifies, LDS bytes per workgroup in *lds_bytes. */
int gie_hip_narrow_check(const gie_conv_geom* g, int* lds_bytes);
int gie_hip_conv_narrow(int dtype, const gie_conv_geom* g, const void* x, const void* w, const void* bias, void* y,
                        void* stream);

/* One registered slab configuration: tile_m (32) output channels x a slab of `rows` output rows of one image laid
   out `pitch` positions per row (in_w + 1 <= pitch), channel slices of tile_k, `stages` LDS load stages,
   `workgroups_per_cu` resident workgroups per compute unit. */
typedef struct gie_slab_config {
  int tile_m, rows, pitch, tile_k;
  int stages;
  int workgroups_per_cu; /* resident workgroups per CU: 2 for the lean form with at most 80 KiB LDS */
  int form;              /* 0: double-buffered fragments; 1: lean (single fragment set, at most 256 VGPR+AGPR);
                            2: pipelined (double-buffered fragments, one MFMA per issue slot carrying the side work;
                            in_channels a multiple of 32); 3: split (the pipelined layout with a second wave per
                            SIMD that issues all loads, 512 threads; in_channels a multiple of 32) */
  int threads;
  int lds_bytes;
  int version;
} gie_slab_config;

int gie_hip_slab_config_count(void);
int gie_hip_slab_config_get(int index, gie_slab_config* out);
/* 0 when configuration `config` runs geometry g (3x3 filter, stride 1, padding 1, in_channels % 8 == 0,
   in_w + 1 <= pitch, sizes within 32-bit offsets), with the LDS bytes per workgroup in *lds_bytes. */
int gie_hip_slab_check(int config, const gie_conv_geom* g, int* lds_bytes);

/* Slab convolution on MFMA 16x16x32 (FP32 accumulation) straight from the caller's NCHW x and OIHW w: no repack,
   no workspace at split 1. x: any 2-byte alignment (16-byte register loads when the slab is the whole image and x
   is 16-byte aligned, 4-byte direct-to-LDS loads for even rows on a 4-byte aligned x, 2-byte loads otherwise;
   GIE_HIP_EUNSUPPORTED when the configuration lacks the form needed). w: 16-byte aligned, GIE_HIP_EUNSUPPORTED
   otherwise. split == 1: y (NCHW, any 2-byte alignment) = round(relu?(acc + bias)), one rounding. split > 1:
   partial[z][NCHW index] = FP32 sum over the channel slices [floor(S*z/split), floor(S*(z+1)/split)),
   S = ceil(in_channels / tile_k); reduce with gie_hip_splitk_reduce. 1 <= split <= S. */
int gie_hip_conv_slab(int config, int dtype, const gie_conv_geom* g, const void* x, const void* w,
                      const void* bias, void* y, float* partial, int split, void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph capture,
   tight serving loops, harnesses that forbid hipMalloc): gie_hip_conv_slab followed, for split > 1, by
   gie_hip_splitk_reduce, with the FP32 partials in the library's static per-device scratch of
   gie_hip_slab_scratch_floats() floats (32 MiB) instead of a caller buffer. Allocates nothing; the first call on a
   device sets that device up. split * batch * out_channels * in_h * in_w above the scratch size: GIE_HIP_ESCRATCH.
   Every call on one GPU shares that GPU's scratch: calls that overlap on one GPU (other streams, other threads)
   race. */
int gie_hip_conv_slab_noalloc(int config, int dtype, const gie_conv_geom* g, const void* x, const void* w,
                              const void* bias, void* y, int split, void* stream);
long long gie_hip_slab_scratch_floats(void);

/* One registered stack configuration: tile_m (32) output channels x `rows` stack rows (a group of images of in_h
   rows each plus one zero separator row per image, laid out `pitch` positions per row, in_w + 1 <= pitch), channel
   slices of tile_k; `halves` groups of 4 waves per workgroup each take part of the workgroup's slices (their
   accumulators are added in LDS before the epilogue). */
typedef struct gie_stack_config {
  int tile_m, rows, pitch, tile_k;
  int threads;
  int lds_bytes;
  int halves;
  int version;
} gie_stack_config;

int gie_hip_stack_config_count(void);
int gie_hip_stack_config_get(int index, gie_stack_config* out);
/* 0 when configuration `config` runs geometry g (3x3 filter, stride 1, padding 1, in_channels % 32 == 0,
   in_w + 1 <= pitch, in_h + 1 <= rows, sizes within 32-bit offsets): LDS bytes per workgroup in *lds_bytes, images
   stacked per workgroup in *images_per_unit (either may be NULL). */
int gie_hip_stack_check(int config, const gie_conv_geom* g, int* lds_bytes, int* images_per_unit);

/* Stacked-image convolution on MFMA 16x16x32 (FP32 accumulation) straight from the caller's NCHW x and OIHW w, for
   3x3 layers with small images and a long reduction: each workgroup owns 32 output channels x a group of images
   stacked into one tall zero-separated plane x one range of channel slices. x 4-byte aligned and w 16-byte aligned
   (GIE_HIP_EUNSUPPORTED otherwise); y and bias 2-byte aligned. split == 1: y (NCHW) = round(relu?(acc + bias)), one
   rounding. split > 1: partial[z][NCHW index] = FP32 sum over the channel slices [floor(S*z/split),
   floor(S*(z+1)/split)), S = in_channels / 32; reduce with gie_hip_splitk_reduce. 1 <= split <= S. */
int gie_hip_conv_stack(int config, int dtype, const gie_conv_geom* g, const void* x, const void* w,
                       const void* bias, void* y, float* partial, int split, void* stream);

/* Deep-reduction convolution on MFMA 16x16x32 (FP32 accumulation) straight from the caller's NCHW x and OIHW w, for
   3x3 stride-1 padding-1 layers over small images (in_h <= 8, in_w <= 7) with in_channels % 128 == 0: one workgroup
   per (16-filter block, image) sums the whole reduction (four waves over interleaved channel slices, partial tiles
   added in LDS in a fixed order), so there is no split-K and no workspace. y (NCHW) = round(relu?(acc + bias)), one
   rounding. x 4-byte aligned and w 16-byte aligned (GIE_HIP_EUNSUPPORTED otherwise); y and bias 2-byte aligned.
   Replaces, for these shapes, the tcmma launch sequence of src/kernels/tensor_core_mma.cu:297-324 (two transposes,
   tcmma_kernel, splitk_reduce). *_check: 0 when the geometry runs, with the LDS bytes per workgroup. */
int gie_hip_deep_check(const gie_conv_geom* g, int* lds_bytes);
int gie_hip_conv_deep(int dtype, const gie_conv_geom* g, const void* x, const void* w, const void* bias, void* y,
                      void* stream);

/* y[i] = round(relu?(sum_{z=0..split-1, ascending} partial[z*total+i] + bias[(i / hw_out) % out_channels]));
   dtype GIE_HIP_FP32 / _TF32: y and bias are float and there is no rounding step. */
int gie_hip_splitk_reduce(int dtype, const float* partial, const void* bias, void* y, int64_t total, int split,
                          int out_channels, int hw_out, int relu, void* stream);

/* The kernel form gie_hip_splitk_reduce selects for (dtype, total, split), without launching anything: index_bits =
   32 when every partial offset z * total + i fits an int (else 64), slices_unrolled = the compile-time slice count
   of the 32-bit form (1, 2, 4 or 8; 0 = any split). vec != 0 states that total % 4 == 0 and partial is 16-byte
   aligned. Host-side query for tests and tools; no reference counterpart. */
int gie_hip_splitk_reduce_form(int dtype, int64_t total, int split, int vec, int* index_bits, int* slices_unrolled);

/* Stand-alone epilogue pass over an NCHW output, in place (the unfused side of the fusion experiment):
   y[i] = round(relu?(f32(y[i]) + f32(bias[(i / hw_out) % out_channels]))); bias may be NULL (ReLU only). dtype
   GIE_HIP_FP32, _FP16 or _BF16; y and bias aligned to their element size. No-op when bias is NULL and relu 0. */
int gie_hip_bias_act(int dtype, void* y, const void* bias, int64_t total, int out_channels, int hw_out, int relu,
                     void* stream);

/* Double-accumulation direct convolution (validation reference for the autotuner and tests):
   y_ref, scale: float[batch*out_channels*out_h*out_w]. dtype may be GIE_HIP_FP32 here. */
int gie_hip_reference_conv(int dtype, const gie_conv_geom* g, const void* x, const void* w, const void* bias,
                           float* y_ref, float* scale, void* stream);

/* Ceiling microbenchmarks (one launch each; the caller times them with events).
   mfma: `blocks` workgroups of 256 threads issuing `iters` dependent-free 16x16x32 f16 MFMAs per wave
   (flops = blocks * 4 waves * iters * 4 chains * 16384); copy: dst = src, `bytes` multiple of 16;
   empty: one 64-thread workgroup that does nothing. `sink` receives a value so nothing is optimized out. */
int gie_hip_ceiling_mfma(int blocks, int iters, float* sink, void* stream);
int gie_hip_ceiling_copy(const void* src, void* dst, size_t bytes, void* stream);
int gie_hip_ceiling_empty(void* stream);
/* The empty kernel with an argument block of arg_bytes (8: one pointer; 128; 1024): what a launch costs the host as a
   function of its kernel arguments (HIP copies a non-empty block to device memory by default). GIE_HIP_EINVAL for
   other sizes. No counterpart in the reference: a measurement of this build's launch path. */
int gie_hip_ceiling_empty_args(int arg_bytes, void* stream);
/* HBM streaming probe: `workgroups` workgroups of 512 threads, workgroup b reading its own contiguous read_bytes /
   workgroups of src and writing its own write_bytes / workgroups of dst in 16-byte lane accesses (reads spread evenly
   over the writes); store_policy 0 write-back, 1 device scope (written through the L2), 2 non-temporal. Both sizes
   multiples of 16 * workgroups; dst is required (with write_bytes 0 it only receives a never-taken sink store). No
   counterpart in the reference: the write and read/write ceilings the stem and pointwise kernels are measured
   against. */
int gie_hip_ceiling_stream(const void* src, size_t read_bytes, void* dst, size_t write_bytes, int store_policy,
                           int workgroups, void* stream);

/* dst[i] = value for i < n (16-bit elements, any 2-byte alignment). A graph-safe fill (no memset node). */
int gie_hip_fill_u16(void* dst, int64_t n, uint16_t value, void* stream);

#ifdef __cplusplus
}
#endif
#endif
