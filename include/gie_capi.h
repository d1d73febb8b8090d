/* C-ABI over the gie:: C++ plan API (libgie.so), for hosts that bind C rather than C++ (ctypes, cgo, JNI).
 *
 * The reference exposes this path only as C++ (the gpu_inference headers); each function below is a flat
 * wrapper over one of those calls and cites it (paths relative to the reference checkout). Exceptions never
 * cross this boundary: every function returns 0 or a gie::StatusCode value
 * (1 InvalidArgument, 2 Unsupported, 3 WorkspaceTooSmall, 4 HipError, 5 Internal, 6 Io) and leaves the
 * message in gie_last_error() (thread-local). Streams/events/plans/graphs are opaque `void*` handles.
 */
#ifndef GIE_CAPI_H_
#define GIE_CAPI_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ConvProblem (include/gpu_inference/conv2d.h:47-85). precision: 0 fp32, 1 fp16, 2 bf16, 3 tf32 */
typedef struct gie_problem {
  int batch, in_channels, in_h, in_w, out_channels, kernel_h, kernel_w;
  int stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, groups;
  int precision, has_bias, relu;
} gie_problem;

/* Conv2DOptions (conv2d.h:90-96). backend: 0 auto, 1 cpu_reference, 2 direct, 3 im2col_gemm, 4 simt_tiled,
   5 implicit_gemm, 6 tensor_core. kernel / cache_path may be null. */
typedef struct gie_options {
  int backend;
  const char* kernel;
  int autotune, force_retune;
  const char* cache_path;
} gie_options;

/* A tensor view (ConstTensorRef / TensorRef, tensor.h:45-66). dtype: 0 float32, 1 float16, 2 bfloat16 */
typedef struct gie_tensor {
  const void* data;
  int dtype;
  int64_t n, c, h, w;
} gie_tensor;

const char* gie_last_error(void);
const char* gie_status_string(int status);

/* ---- problem ---- */
int gie_validate_problem(const gie_problem* p);                              /* conv2d.cpp:83-109 */
int gie_problem_key(const gie_problem* p, char* buf, size_t n);              /* conv2d.cpp:77-81 */

/* ---- Conv2D (conv2d.h:98-112) ---- */
int gie_conv2d_forward(const gie_problem* p, const gie_tensor* x, const gie_tensor* w, const gie_tensor* bias,
                       const gie_tensor* y, void* workspace, size_t workspace_bytes, void* stream,
                       const gie_options* opt);
/* `count` back-to-back Conv2D::forward calls on one stream (plan lookup + argument validation + launch each
   time): the benchmark's timed step without a host-language loop in the way */
int gie_conv2d_forward_n(const gie_problem* p, const gie_tensor* x, const gie_tensor* w, const gie_tensor* bias,
                         const gie_tensor* y, void* workspace, size_t workspace_bytes, void* stream,
                         const gie_options* opt, int count);
/* gie_conv2d_forward_n bracketed by two events (hipEvent_t) recorded on `stream` right before the first call and
   right after the last, so no host-language work sits inside the timed interval; only enqueues (the caller
   synchronizes). No counterpart in the reference, whose harness records its events from C++ around the loop
   (benchmarks/benchmark_main.cpp:55-56). */
int gie_conv2d_forward_n_timed(const gie_problem* p, const gie_tensor* x, const gie_tensor* w,
                               const gie_tensor* bias, const gie_tensor* y, void* workspace, size_t workspace_bytes,
                               void* stream, const gie_options* opt, int count, void* ev_start, void* ev_end);
/* time_stream_work (timing.h:36-38, the reference's timing.cpp:42-83 protocol) around Conv2D::forward itself:
   `warmup` calls, then `samples` samples of back-to-back forward calls lasting at least min_sample_ms each;
   stats = {median, mean, min, max, p10, p90, stddev} in microseconds per call, *inner = calls per sample. The
   reference's benchmark harness reports the median of this protocol (benchmarks/benchmark_main.cpp:55-56). */
int gie_conv2d_time_forward(const gie_problem* p, const gie_tensor* x, const gie_tensor* w, const gie_tensor* bias,
                            const gie_tensor* y, void* workspace, size_t workspace_bytes, void* stream,
                            const gie_options* opt, int warmup, int samples, double min_sample_ms, double* stats7,
                            int* inner);
/* Host cost of the plan API, no counterpart in the reference: median host wall time to enqueue one
   gie_conv2d_forward call on problem p (zero-filled tensors, plan already cached) and one bare empty-kernel launch,
   each over batches of `batch` back-to-back calls; out3 = {host us per forward, host us per bare launch,
   device us per forward}. */
int gie_measure_host_cost(const gie_problem* p, const gie_options* opt, int batch, double* out3);
int gie_conv2d_workspace_size(const gie_problem* p, const gie_options* opt, size_t* bytes);
int gie_conv2d_clear_plan_cache(void);

/* ---- ExecutionPlan (execution_plan.h:14-51) ---- */
int gie_plan_create(const gie_problem* p, const char* kernel_name, int device, void** plan);
int gie_plan_destroy(void* plan);
int gie_plan_workspace_bytes(void* plan, size_t* bytes);
int gie_plan_kernel_name(void* plan, char* buf, size_t n);
/* execute_unchecked with stage events (execution_plan.cpp:122-136, im2col.cu:88-114): a family with a repack stage
   records events3[0] before it, events3[1] after it and events3[2] after the convolution; others record none */
int gie_plan_execute_staged(void* plan, const void* x, const void* w, const void* bias, void* y, void* workspace,
                            size_t workspace_bytes, void* stream, void* const* events3);
/* bytes of the plan's device gather table (execution_plan.cpp:69-73; 0 unless the kernel sets needs_lut) */
int gie_plan_lut_bytes(void* plan, size_t* bytes);
/* build_conv_lut / build_conv_lut_chunked (kernel_registry.h:86-96, conv_common.cu:22-50): *count entries of four
   int32 (c_off, r_off, s_off, 0); out4 == NULL asks for the count only, cap is out4's capacity in entries */
int gie_build_conv_lut(const gie_problem* p, int chunked, int32_t* out4, int64_t cap, int64_t* count);
int gie_plan_execute(void* plan, const gie_tensor* x, const gie_tensor* w, const gie_tensor* bias,
                     const gie_tensor* y, void* workspace, size_t workspace_bytes, void* stream);
int gie_plan_execute_unchecked(void* plan, const void* x, const void* w, const void* bias, void* y, void* workspace,
                               size_t workspace_bytes, void* stream);
/* time_stream_work (timing.h:36-38) around execute_unchecked; stats = {median, mean, min, max, p10, p90, stddev}
   in microseconds per call, *inner = launches per sample */
int gie_plan_time(void* plan, const void* x, const void* w, const void* bias, void* y, void* workspace,
                  size_t workspace_bytes, void* stream, int warmup, int samples, double min_sample_ms,
                  double* stats7, int* inner);
/* per-stage device time: after one full call, each stage alone runs `iters` times back to back between two
   events; us3 = average duration of {repack, implicit GEMM, split-K reduce (~0 when split == 1)} */
int gie_plan_time_stages(void* plan, const void* x, const void* w, const void* bias, void* y, void* workspace,
                         size_t workspace_bytes, void* stream, int iters, double* us3);

/* ---- registry / dispatcher (kernel_registry.h:76-82, dispatcher.h:34-53) ---- */
int gie_registry_count(void);
int gie_registry_name(int index, char* buf, size_t n);
/* params as "key=value,key=value" and flags */
int gie_kernel_describe(const char* name, char* buf, size_t n);
int gie_kernel_supports(const char* name, const gie_problem* p, int* ok, char* why, size_t why_n);
/* source: 0 forced_kernel, 1 forced_backend, 2 tuning_cache, 3 tuned, 4 cost_model */
int gie_dispatch_select(const gie_problem* p, const gie_options* opt, char* kernel, size_t n, int* source,
                        double* predicted_us);
/* cost-model ranking of all compatible kernels: names joined by '\n' into buf, predicted us into us[max] */
int gie_rank_by_model(const gie_problem* p, char* buf, size_t n, double* us, int max, int* count);

/* ---- autotuner / tune cache (autotuner.h:21-93) ---- */
typedef struct gie_tune_options {
  int warmup, samples;
  double min_sample_ms;
  uint64_t seed;
  int validate, model_keep, max_candidates, use_cache, force_retune, verbose;
  const char* cache_path;
} gie_tune_options;
void gie_tune_options_default(gie_tune_options* o);
/* best kernel name into best; counts: {candidates_total, candidates_measured, from_cache, n_rejected,
   n_failed_validation, n_error} */
int gie_autotune(const gie_problem* p, const gie_tune_options* o, char* best, size_t n, double* best_us,
                 double* search_seconds, int* counts6);
int gie_tune_cache_key(const gie_problem* p, int scope_backend, char* buf, size_t n);
int gie_tune_cache_size(const char* path, size_t* size);
int gie_tune_cache_clear(const char* path);

/* ---- cost model (perf_model.h) ---- */
/* out6 = {time_us, compute_us, memory_us, launch_us, tile_efficiency, wave_efficiency}; bound: 0/1/2 */
int gie_estimate_kernel(const char* name, const gie_problem* p, double* out6, int* bound);
/* out3 = {fp16_mfma_tflops, bw_gbs, launch_overhead_us} */
int gie_measure_ceilings(int device, int use_cache, double* out3, int* measured);
int gie_theoretical_ceilings(int device, double* out3);
/* The cost model on a described device instead of the current GPU (no GPU needed): a gfx950 part with `cus`
   compute units, the given ceilings and LDS opt-in limit. No counterpart in the reference; it lets hosts and tests
   see which kernel the model would pick for a machine without one. */
typedef struct gie_device_model {
  int cus;
  double mfma_tflops, fp32_tflops, hbm_gbs, launch_us;
  size_t lds_per_workgroup;
} gie_device_model;
int gie_model_estimate(const char* name, const gie_problem* p, const gie_device_model* d, double* out6, int* bound);
/* capable kernels, best first, newline-separated in buf; estimated us in us[0..max) */
int gie_model_rank(const gie_problem* p, const gie_device_model* d, char* buf, size_t n, double* us, int max,
                   int* count);

/* ---- reference and device description ---- */
/* GPU double reference (reference.h:36-39): y, scale float device buffers */
int gie_gpu_reference(const gie_problem* p, const void* x, const void* w, const void* bias, float* y, float* scale,
                      void* stream);
/* CPU reference of the library (reference.h:31-34) on host float arrays */
int gie_cpu_reference(const gie_problem* p, const float* x, const float* w, const float* bias, float* y,
                      float* scale);
/* make_conv_data's host half (testing.h): seeded draws x, w, bias quantized to the storage type.
   dist: 0 uniform, 1 normal, 2 sparse_signed, 3 positive; scaling: 0 reference, 1 benchmark */
int gie_make_host_data(const gie_problem* p, uint64_t seed, int dist, int scaling, float* x, float* w, float* bias);
int gie_device_describe(int device, char* buf, size_t n);
int gie_device_arch(int device, char* buf, size_t n);
int gie_device_cu_count(int device, int* cus);
int gie_build_fingerprint(char* buf, size_t n);

/* TESTING ONLY (kernel_registry_for_testing, kernel_registry.h:78-80): appends a deliberately faulty tensor_core
   kernel to the registry so tests can prove the autotuner never selects it. kind 0: fast but wrong (fills y with
   a constant), kind 1: its launch throws. Names: "test_garbage_<p>" / "test_throwing_<p>" per precision. */
int gie_testing_add_faulty_kernels(int kind);
/* TESTING ONLY: appends needs_lut probe kernels "test_lut_probe_<p>" and "test_lut_chunked_probe_<p>" that run only
   2x3 filters over 24 input channels and copy the plan's device gather table into y, so a test can read back what
   ExecutionPlan::create uploaded (execution_plan.cpp:69-73, :133). */
int gie_testing_add_lut_probe_kernels(void);

/* ---- HipGraphExecutor (cuda_graph.h:14-46) over a chain of plan executions ---- */
int gie_graph_create(void** graph);
int gie_graph_destroy(void* graph);
/* captures plans[i]->execute_unchecked(xs[i], ws[i], biases[i], ys[i], wss[i], ws_bytes[i]) for i = 0..n-1 */
int gie_graph_capture_chain(void* graph, int n, void* const* plans, const void* const* xs, const void* const* ws,
                            const void* const* biases, void* const* ys, void* const* wss, const size_t* ws_bytes);
int gie_graph_recapture_chain(void* graph, int n, void* const* plans, const void* const* xs, const void* const* ws,
                              const void* const* biases, void* const* ys, void* const* wss, const size_t* ws_bytes,
                              int* updated_in_place);
int gie_graph_launch(void* graph, void* stream);
int gie_graph_node_count(void* graph, size_t* nodes);

/* ---- device memory / streams / events for bindings without their own HIP runtime ---- */
int gie_dev_malloc(size_t bytes, void** ptr);
int gie_dev_free(void* ptr);
int gie_memcpy_h2d(void* dst, const void* src, size_t bytes);
int gie_memcpy_d2h(void* dst, const void* src, size_t bytes);
int gie_memcpy_d2d_async(void* dst, const void* src, size_t bytes, void* stream);
int gie_memset(void* ptr, int value, size_t bytes);
int gie_device_synchronize(void);
int gie_get_device_count(int* n);
int gie_set_device(int device);
int gie_stream_create(void** stream);
int gie_stream_destroy(void* stream);
int gie_stream_synchronize(void* stream);
int gie_event_create(void** ev);
int gie_event_destroy(void* ev);
int gie_event_record(void* ev, void* stream);
int gie_event_synchronize(void* ev);
int gie_event_elapsed_ms(void* start, void* stop, float* ms);

#ifdef __cplusplus
}
#endif
#endif
