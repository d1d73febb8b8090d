// Flat C-ABI over the gie:: C++ API (include/gie_capi.h). Each function catches every exception and turns it
// into a status code plus a thread-local message.
#include "gie_capi.h"
#include "gie_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <functional>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gpu_inference/autotuner.h"
#include "gpu_inference/build_info.h"
#include "gpu_inference/conv2d.h"
#include "gpu_inference/dispatcher.h"
#include "gpu_inference/execution_plan.h"
#include "gpu_inference/hip_graph.h"
#include "gpu_inference/perf_model.h"
#include "gpu_inference/reference.h"
#include "gpu_inference/testing.h"
#include "gpu_inference/timing.h"

using namespace gie;

namespace {

thread_local std::string g_last_error;

template <typename F>
int guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return 0;
  } catch (const Error& e) {
    g_last_error = e.what();
    return int(e.code());
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return int(StatusCode::kInternal);
  } catch (...) {
    g_last_error = "unknown exception";
    return int(StatusCode::kInternal);
  }
}

void copy_str(const std::string& s, char* buf, size_t n) {
  if (!buf || n == 0) return;
  const size_t k = std::min(n - 1, s.size());
  std::memcpy(buf, s.data(), k);
  buf[k] = '\0';
}

ConvProblem to_problem(const gie_problem* p) {
  GIE_REQUIRE(p != nullptr, StatusCode::kInvalidArgument, "null problem");
  ConvProblem pr;
  pr.p.batch = p->batch;
  pr.p.in_channels = p->in_channels;
  pr.p.in_h = p->in_h;
  pr.p.in_w = p->in_w;
  pr.p.out_channels = p->out_channels;
  pr.p.kernel_h = p->kernel_h;
  pr.p.kernel_w = p->kernel_w;
  pr.p.stride_h = p->stride_h;
  pr.p.stride_w = p->stride_w;
  pr.p.pad_h = p->pad_h;
  pr.p.pad_w = p->pad_w;
  pr.p.dilation_h = p->dilation_h;
  pr.p.dilation_w = p->dilation_w;
  pr.p.groups = p->groups;
  GIE_REQUIRE(p->precision >= 0 && p->precision <= 3, StatusCode::kInvalidArgument, "bad precision");
  pr.precision = static_cast<Precision>(p->precision);
  pr.has_bias = p->has_bias != 0;
  pr.activation = p->relu ? Activation::kReLU : Activation::kNone;
  return pr;
}

Conv2DOptions to_options(const gie_options* o) {
  Conv2DOptions opt;
  if (!o) return opt;
  GIE_REQUIRE(o->backend >= 0 && o->backend <= 6, StatusCode::kInvalidArgument, "bad backend");
  opt.backend = static_cast<Backend>(o->backend);
  if (o->kernel) opt.kernel = o->kernel;
  opt.autotune = o->autotune != 0;
  opt.force_retune = o->force_retune != 0;
  if (o->cache_path) opt.cache_path = o->cache_path;
  return opt;
}

ConstTensorRef to_cref(const gie_tensor* t) {
  GIE_REQUIRE(t != nullptr, StatusCode::kInvalidArgument, "null tensor descriptor");
  GIE_REQUIRE(t->dtype >= 0 && t->dtype <= 2, StatusCode::kInvalidArgument, "bad dtype");
  return {t->data, static_cast<DataType>(t->dtype), {t->n, t->c, t->h, t->w}};
}

TensorRef to_ref(const gie_tensor* t) {
  const ConstTensorRef c = to_cref(t);
  return {const_cast<void*>(c.data), c.dtype, c.shape};
}

struct PlanHandle {
  std::shared_ptr<ExecutionPlan> plan;
};

ExecutionPlan& plan_of(void* h) {
  GIE_REQUIRE(h != nullptr, StatusCode::kInvalidArgument, "null plan handle");
  return *static_cast<PlanHandle*>(h)->plan;
}

const KernelDesc& kernel_named(const char* name) {
  GIE_REQUIRE(name != nullptr, StatusCode::kInvalidArgument, "null kernel name");
  const KernelDesc* k = find_kernel(name);
  GIE_REQUIRE(k != nullptr, StatusCode::kInvalidArgument, std::string("unknown kernel '") + name + "'");
  return *k;
}

DeviceInfo modelled_device(const gie_device_model& d) {
  GIE_REQUIRE(d.cus > 0 && d.mfma_tflops > 0 && d.fp32_tflops > 0 && d.hbm_gbs > 0 && d.launch_us >= 0,
              StatusCode::kInvalidArgument, "device model needs positive CU count and ceilings");
  DeviceInfo dev;
  dev.device = -1;
  dev.name = "modelled gfx950 device";
  dev.gcn_arch = "gfx950:sramecc+:xnack-";
  dev.cc_major = 9;
  dev.cc_minor = 5;
  dev.sm_count = d.cus;
  dev.global_mem_bytes = size_t(288) << 30;
  dev.l2_bytes = size_t(4) << 20;
  dev.smem_per_block_default = 64 * 1024;
  dev.smem_per_block_optin = d.lds_per_workgroup;
  dev.smem_per_sm = 160 * 1024;
  dev.regs_per_sm = 4 * 512 * 64;
  dev.max_threads_per_sm = 2048;
  dev.max_threads_per_block = 1024;
  dev.max_blocks_per_sm = 32;
  dev.warp_size = 64;
  dev.max_sm_clock_khz = 2400000;
  return dev;
}

DeviceCeilings modelled_ceilings(const gie_device_model& d) {
  DeviceCeilings c;
  c.fp16_tc_tflops = d.mfma_tflops;
  c.fp32_tflops = d.fp32_tflops;
  c.bw_gbs = d.hbm_gbs;
  c.launch_overhead_us = d.launch_us;
  c.measured = false;
  c.source = "caller-described device";
  return c;
}

HipGraphExecutor::Enqueue chain_enqueue(int n, void* const* plans, const void* const* xs, const void* const* ws,
                                        const void* const* biases, void* const* ys, void* const* wss,
                                        const size_t* ws_bytes) {
  GIE_REQUIRE(n > 0 && plans && xs && ws && ys, StatusCode::kInvalidArgument, "bad chain description");
  std::vector<std::shared_ptr<ExecutionPlan>> ps;
  for (int i = 0; i < n; ++i) {
    GIE_REQUIRE(plans[i] != nullptr, StatusCode::kInvalidArgument, "null plan in chain");
    ps.push_back(static_cast<PlanHandle*>(plans[i])->plan);
  }
  std::vector<const void*> vx(xs, xs + n), vw(ws, ws + n), vb(n, nullptr);
  std::vector<void*> vy(ys, ys + n), vws(n, nullptr);
  std::vector<size_t> vwb(n, 0);
  for (int i = 0; i < n; ++i) {
    if (biases) vb[i] = biases[i];
    if (wss) vws[i] = wss[i];
    if (ws_bytes) vwb[i] = ws_bytes[i];
  }
  return [=](hipStream_t s) {
    for (int i = 0; i < n; ++i) ps[size_t(i)]->execute_unchecked(vx[i], vw[i], vb[i], vy[i], vws[i], vwb[i], s);
  };
}

}  // namespace

extern "C" {

const char* gie_last_error(void) { return g_last_error.c_str(); }
const char* gie_status_string(int status) { return to_string(static_cast<StatusCode>(status)); }

int gie_validate_problem(const gie_problem* p) {
  return guarded([&] { validate_problem(to_problem(p)); });
}

int gie_problem_key(const gie_problem* p, char* buf, size_t n) {
  return guarded([&] { copy_str(to_problem(p).key(), buf, n); });
}

int gie_conv2d_forward(const gie_problem* p, const gie_tensor* x, const gie_tensor* w, const gie_tensor* bias,
                       const gie_tensor* y, void* workspace, size_t workspace_bytes, void* stream,
                       const gie_options* opt) {
  return guarded([&] {
    const ConstTensorRef b = bias ? to_cref(bias) : ConstTensorRef{};
    Conv2D::forward(to_cref(x), to_cref(w), bias ? &b : nullptr, to_problem(p), to_ref(y), workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream), to_options(opt));
  });
}

int gie_conv2d_forward_n(const gie_problem* p, const gie_tensor* x, const gie_tensor* w, const gie_tensor* bias,
                         const gie_tensor* y, void* workspace, size_t workspace_bytes, void* stream,
                         const gie_options* opt, int count) {
  return guarded([&] {
    const ConstTensorRef b = bias ? to_cref(bias) : ConstTensorRef{};
    const ConstTensorRef xr = to_cref(x), wr = to_cref(w);
    const TensorRef yr = to_ref(y);
    const ConvProblem pr = to_problem(p);
    const Conv2DOptions o = to_options(opt);
    for (int i = 0; i < count; ++i)
      Conv2D::forward(xr, wr, bias ? &b : nullptr, pr, yr, workspace, workspace_bytes,
                      static_cast<hipStream_t>(stream), o);
  });
}

int gie_conv2d_forward_n_timed(const gie_problem* p, const gie_tensor* x, const gie_tensor* w,
                               const gie_tensor* bias, const gie_tensor* y, void* workspace, size_t workspace_bytes,
                               void* stream, const gie_options* opt, int count, void* ev_start, void* ev_end) {
  return guarded([&] {
    GIE_REQUIRE(ev_start != nullptr && ev_end != nullptr, StatusCode::kInvalidArgument, "null event");
    const ConstTensorRef b = bias ? to_cref(bias) : ConstTensorRef{};
    const ConstTensorRef xr = to_cref(x), wr = to_cref(w);
    const TensorRef yr = to_ref(y);
    const ConvProblem pr = to_problem(p);
    const Conv2DOptions o = to_options(opt);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    GIE_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(ev_start), s));
    for (int i = 0; i < count; ++i) Conv2D::forward(xr, wr, bias ? &b : nullptr, pr, yr, workspace, workspace_bytes, s, o);
    GIE_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(ev_end), s));
  });
}

int gie_conv2d_time_forward(const gie_problem* p, const gie_tensor* x, const gie_tensor* w, const gie_tensor* bias,
                            const gie_tensor* y, void* workspace, size_t workspace_bytes, void* stream,
                            const gie_options* opt, int warmup, int samples, double min_sample_ms, double* stats7,
                            int* inner) {
  return guarded([&] {
    const ConstTensorRef b = bias ? to_cref(bias) : ConstTensorRef{};
    const ConstTensorRef xr = to_cref(x), wr = to_cref(w);
    const TensorRef yr = to_ref(y);
    const ConvProblem pr = to_problem(p);
    const Conv2DOptions o = to_options(opt);
    TimingOptions to;
    to.warmup_iters = warmup;
    to.samples = samples;
    to.min_sample_ms = min_sample_ms;
    const TimingStats t = time_stream_work(
        [&](hipStream_t s) { Conv2D::forward(xr, wr, bias ? &b : nullptr, pr, yr, workspace, workspace_bytes, s, o); },
        static_cast<hipStream_t>(stream), to);
    const double v[7] = {t.median_us, t.mean_us, t.min_us, t.max_us, t.p10_us, t.p90_us, t.stddev_us};
    if (stats7) std::memcpy(stats7, v, sizeof(v));
    if (inner) *inner = t.inner_iters;
  });
}

int gie_measure_host_cost(const gie_problem* p, const gie_options* opt, int batch, double* out3) {
  return guarded([&] {
    GIE_REQUIRE(p != nullptr && out3 != nullptr && batch > 0, StatusCode::kInvalidArgument,
                "host cost: null problem/output or batch <= 0");
    const ConvProblem pr = to_problem(p);
    const Conv2DOptions o = to_options(opt);
    const Conv2DParams& q = pr.p;
    const DataType dt = pr.dtype();
    const size_t es = dtype_size(dt);
    DeviceBuffer x(size_t(q.input_shape().numel()) * es), w(size_t(q.weight_shape().numel()) * es),
        b(size_t(q.out_channels) * es), y(size_t(q.output_shape().numel()) * es);
    GIE_HIP_CHECK(hipMemset(x.data(), 0, x.size()));
    GIE_HIP_CHECK(hipMemset(w.data(), 0, w.size()));
    GIE_HIP_CHECK(hipMemset(b.data(), 0, b.size()));
    const size_t wsb = Conv2D::workspace_size(pr, o);
    DeviceBuffer ws(wsb);
    hipStream_t s = nullptr;
    GIE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    struct Done {
      hipStream_t s;
      ~Done() { (void)hipStreamDestroy(s); }
    } done{s};
    const ConstTensorRef xr{x.data(), dt, q.input_shape()}, wr{w.data(), dt, q.weight_shape()},
        br{b.data(), dt, q.bias_shape()};
    const TensorRef yr{y.data(), dt, q.output_shape()};
    auto forward = [&] { Conv2D::forward(xr, wr, pr.has_bias ? &br : nullptr, pr, yr, ws.data(), wsb, s, o); };
    auto empty = [&] { check_kernel_status(gie_hip_ceiling_empty(s), "empty kernel"); };
    // host wall time to enqueue `batch` calls (a batch well below the queue depth never waits for the GPU),
    // median of 9 batches; the GPU time of the same batch from events on the stream
    auto measure = [&](const std::function<void()>& call, double* host_us, double* dev_us) {
      for (int i = 0; i < 32; ++i) call();
      GIE_HIP_CHECK(hipStreamSynchronize(s));
      std::vector<double> h, d;
      hipEvent_t e0, e1;
      GIE_HIP_CHECK(hipEventCreate(&e0));
      GIE_HIP_CHECK(hipEventCreate(&e1));
      for (int rep = 0; rep < 9; ++rep) {
        GIE_HIP_CHECK(hipEventRecord(e0, s));
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < batch; ++i) call();
        const auto t1 = std::chrono::steady_clock::now();
        GIE_HIP_CHECK(hipEventRecord(e1, s));
        GIE_HIP_CHECK(hipEventSynchronize(e1));
        float ms = 0;
        GIE_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        h.push_back(std::chrono::duration<double, std::micro>(t1 - t0).count() / batch);
        d.push_back(1000.0 * ms / batch);
      }
      (void)hipEventDestroy(e0);
      (void)hipEventDestroy(e1);
      std::sort(h.begin(), h.end());
      std::sort(d.begin(), d.end());
      *host_us = h[h.size() / 2];
      if (dev_us) *dev_us = d[d.size() / 2];
    };
    measure(forward, &out3[0], &out3[2]);
    measure(empty, &out3[1], nullptr);
  });
}

int gie_conv2d_workspace_size(const gie_problem* p, const gie_options* opt, size_t* bytes) {
  return guarded([&] { *bytes = Conv2D::workspace_size(to_problem(p), to_options(opt)); });
}

int gie_conv2d_clear_plan_cache(void) {
  return guarded([&] { Conv2D::clear_plan_cache(); });
}

int gie_plan_create(const gie_problem* p, const char* kernel_name, int device, void** plan) {
  return guarded([&] {
    GIE_REQUIRE(plan != nullptr, StatusCode::kInvalidArgument, "null output handle");
    auto h = std::make_unique<PlanHandle>();
    h->plan = ExecutionPlan::create(to_problem(p), kernel_named(kernel_name), device);
    *plan = h.release();
  });
}

int gie_plan_destroy(void* plan) {
  return guarded([&] { delete static_cast<PlanHandle*>(plan); });
}

int gie_plan_workspace_bytes(void* plan, size_t* bytes) {
  return guarded([&] { *bytes = plan_of(plan).workspace_bytes(); });
}

int gie_plan_execute_staged(void* plan, const void* x, const void* w, const void* bias, void* y, void* workspace,
                            size_t workspace_bytes, void* stream, void* const* events3) {
  return guarded([&] {
    GIE_REQUIRE(events3 != nullptr, StatusCode::kInvalidArgument, "null stage events");
    hipEvent_t ev[3] = {static_cast<hipEvent_t>(events3[0]), static_cast<hipEvent_t>(events3[1]),
                        static_cast<hipEvent_t>(events3[2])};
    plan_of(plan).execute_unchecked(x, w, bias, y, workspace, workspace_bytes, static_cast<hipStream_t>(stream), ev);
  });
}

int gie_plan_lut_bytes(void* plan, size_t* bytes) {
  return guarded([&] { *bytes = plan_of(plan).lut_bytes(); });
}

int gie_build_conv_lut(const gie_problem* p, int chunked, int32_t* out4, int64_t cap, int64_t* count) {
  return guarded([&] {
    GIE_REQUIRE(count != nullptr, StatusCode::kInvalidArgument, "null count");
    const ConvProblem pr = to_problem(p);
    const std::vector<LutEntry> t = chunked ? build_conv_lut_chunked(pr.p) : build_conv_lut(pr.p);
    *count = int64_t(t.size());
    if (out4 == nullptr) return;
    GIE_REQUIRE(cap >= int64_t(t.size()), StatusCode::kInvalidArgument, "gather-table buffer too small");
    for (size_t i = 0; i < t.size(); ++i) {
      out4[4 * i + 0] = t[i].c_off;
      out4[4 * i + 1] = t[i].r_off;
      out4[4 * i + 2] = t[i].s_off;
      out4[4 * i + 3] = t[i].pad_;
    }
  });
}

int gie_plan_kernel_name(void* plan, char* buf, size_t n) {
  return guarded([&] { copy_str(plan_of(plan).kernel().name, buf, n); });
}

int gie_plan_execute(void* plan, const gie_tensor* x, const gie_tensor* w, const gie_tensor* bias,
                     const gie_tensor* y, void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    const ConstTensorRef b = bias ? to_cref(bias) : ConstTensorRef{};
    plan_of(plan).execute(to_cref(x), to_cref(w), bias ? &b : nullptr, to_ref(y), workspace, workspace_bytes,
                          static_cast<hipStream_t>(stream));
  });
}

int gie_plan_execute_unchecked(void* plan, const void* x, const void* w, const void* bias, void* y, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return guarded([&] {
    plan_of(plan).execute_unchecked(x, w, bias, y, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  });
}

int gie_plan_time(void* plan, const void* x, const void* w, const void* bias, void* y, void* workspace,
                  size_t workspace_bytes, void* stream, int warmup, int samples, double min_sample_ms,
                  double* stats7, int* inner) {
  return guarded([&] {
    ExecutionPlan& pl = plan_of(plan);
    TimingOptions to;
    to.warmup_iters = warmup;
    to.samples = samples;
    to.min_sample_ms = min_sample_ms;
    const TimingStats t = time_stream_work(
        [&](hipStream_t s) { pl.execute_unchecked(x, w, bias, y, workspace, workspace_bytes, s); },
        static_cast<hipStream_t>(stream), to);
    const double v[7] = {t.median_us, t.mean_us, t.min_us, t.max_us, t.p10_us, t.p90_us, t.stddev_us};
    if (stats7) std::memcpy(stats7, v, sizeof(v));
    if (inner) *inner = t.inner_iters;
  });
}

int gie_plan_time_stages(void* plan, const void* x, const void* w, const void* bias, void* y, void* workspace,
                         size_t workspace_bytes, void* stream, int iters, double* us3) {
  return guarded([&] {
    ExecutionPlan& pl = plan_of(plan);
    GIE_REQUIRE(iters > 0 && us3, StatusCode::kInvalidArgument, "bad iteration count");
    hipStream_t s = static_cast<hipStream_t>(stream);
    // One full call fills the workspace; then each stage alone runs `iters` times back to back between two
    // events (every stage is idempotent on a filled workspace), so us3[k] is that kernel's average duration
    // inside a steady stream of its own launches. A stage the kernel does not have reads as ~0.
    hipEvent_t e0 = nullptr, e1 = nullptr;
    struct G {
      hipEvent_t& a;
      hipEvent_t& b;
      ~G() {
        if (a) (void)hipEventDestroy(a);
        if (b) (void)hipEventDestroy(b);
      }
    } guard{e0, e1};
    GIE_HIP_CHECK(hipEventCreate(&e0));
    GIE_HIP_CHECK(hipEventCreate(&e1));
    pl.execute_unchecked(x, w, bias, y, workspace, workspace_bytes, s);
    for (int k = 0; k < 3; ++k) {
      pl.execute_unchecked(x, w, bias, y, workspace, workspace_bytes, s, nullptr, k);  // warm this stage
      GIE_HIP_CHECK(hipEventRecord(e0, s));
      for (int it = 0; it < iters; ++it) pl.execute_unchecked(x, w, bias, y, workspace, workspace_bytes, s, nullptr, k);
      GIE_HIP_CHECK(hipEventRecord(e1, s));
      GIE_HIP_CHECK(hipEventSynchronize(e1));
      float ms = 0;
      GIE_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
      us3[k] = ms * 1e3 / iters;
    }
    pl.execute_unchecked(x, w, bias, y, workspace, workspace_bytes, s);  // leave y as one full call made it
    GIE_HIP_CHECK(hipStreamSynchronize(s));
  });
}

int gie_registry_count(void) {
  int n = 0;
  guarded([&] { n = int(kernel_registry().size()); });
  return n;
}

int gie_registry_name(int index, char* buf, size_t n) {
  return guarded([&] {
    GIE_REQUIRE(index >= 0 && size_t(index) < kernel_registry().size(), StatusCode::kInvalidArgument, "bad index");
    copy_str(kernel_registry()[size_t(index)].name, buf, n);
  });
}

int gie_kernel_describe(const char* name, char* buf, size_t n) {
  return guarded([&] {
    const KernelDesc& k = kernel_named(name);
    std::string s = "backend=" + std::string(to_string(k.backend)) + ",version=" + std::to_string(k.version) +
                    ",threads=" + std::to_string(k.threads_per_block) + ",tile_m=" + std::to_string(k.tile_m) +
                    ",tile_n=" + std::to_string(k.tile_n) + ",tile_k=" + std::to_string(k.tile_k) +
                    ",launches=" + std::to_string(k.launches);
    for (const auto& kv : k.params) s += "," + kv.first + "=" + std::to_string(kv.second);
    copy_str(s, buf, n);
  });
}

int gie_kernel_supports(const char* name, const gie_problem* p, int* ok, char* why, size_t why_n) {
  return guarded([&] {
    const KernelDesc& k = kernel_named(name);
    std::string reason;
    *ok = k.supports(to_problem(p), DeviceInfo::current(), &reason) ? 1 : 0;
    copy_str(reason, why, why_n);
  });
}

int gie_dispatch_select(const gie_problem* p, const gie_options* opt, char* kernel, size_t n, int* source,
                        double* predicted_us) {
  return guarded([&] {
    const Selection sel = Dispatcher::select(to_problem(p), DeviceInfo::current(), to_options(opt));
    copy_str(sel.kernel->name, kernel, n);
    if (source) *source = int(sel.source);
    if (predicted_us) *predicted_us = sel.predicted_us;
  });
}

int gie_rank_by_model(const gie_problem* p, char* buf, size_t n, double* us, int max, int* count) {
  return guarded([&] {
    const ConvProblem pr = to_problem(p);
    const DeviceInfo& dev = DeviceInfo::current();
    const auto ranked = Dispatcher::rank_by_model(pr, dev, Dispatcher::compatible_kernels(pr, dev));
    std::string names;
    int i = 0;
    for (const auto& r : ranked) {
      if (i < max && us) us[i] = r.second;
      if (!names.empty()) names += "\n";
      names += r.first->name;
      ++i;
    }
    copy_str(names, buf, n);
    if (count) *count = int(ranked.size());
  });
}

void gie_tune_options_default(gie_tune_options* o) {
  if (!o) return;
  const TuneOptions d;
  o->warmup = d.timing.warmup_iters;
  o->samples = d.timing.samples;
  o->min_sample_ms = d.timing.min_sample_ms;
  o->seed = d.seed;
  o->validate = d.validate ? 1 : 0;
  o->model_keep = d.model_keep;
  o->max_candidates = d.max_candidates;
  o->use_cache = d.use_cache ? 1 : 0;
  o->force_retune = d.force_retune ? 1 : 0;
  o->verbose = d.verbose ? 1 : 0;
  o->cache_path = nullptr;
}

int gie_autotune(const gie_problem* p, const gie_tune_options* o, char* best, size_t n, double* best_us,
                 double* search_seconds, int* counts6) {
  return guarded([&] {
    TuneOptions to;
    if (o) {
      to.timing.warmup_iters = o->warmup;
      to.timing.samples = o->samples;
      to.timing.min_sample_ms = o->min_sample_ms;
      to.seed = o->seed;
      to.validate = o->validate != 0;
      to.model_keep = o->model_keep;
      to.max_candidates = o->max_candidates;
      to.use_cache = o->use_cache != 0;
      to.force_retune = o->force_retune != 0;
      to.verbose = o->verbose != 0;
      if (o->cache_path) to.cache_path = o->cache_path;
    }
    const TuneResult r = Autotuner::tune(to_problem(p), DeviceInfo::current(), to);
    copy_str(r.best_kernel, best, n);
    if (best_us) *best_us = r.best_us;
    if (search_seconds) *search_seconds = r.search_seconds;
    if (counts6) {
      int rej = 0, fail = 0, err = 0;
      for (const auto& c : r.candidates) {
        if (c.status.rfind("rejected", 0) == 0) ++rej;
        else if (c.status.rfind("failed validation", 0) == 0) ++fail;
        else if (c.status.rfind("error", 0) == 0) ++err;
      }
      const int v[6] = {r.candidates_total, r.candidates_measured, r.from_cache ? 1 : 0, rej, fail, err};
      std::memcpy(counts6, v, sizeof(v));
    }
  });
}

int gie_tune_cache_key(const gie_problem* p, int scope_backend, char* buf, size_t n) {
  return guarded([&] {
    copy_str(TuneCache::make_key(to_problem(p), DeviceInfo::current(), static_cast<Backend>(scope_backend)), buf, n);
  });
}

int gie_tune_cache_size(const char* path, size_t* size) {
  return guarded([&] { *size = TuneCache(path ? path : "").size(); });
}

int gie_tune_cache_clear(const char* path) {
  return guarded([&] { TuneCache(path ? path : "").clear(); });
}

int gie_estimate_kernel(const char* name, const gie_problem* p, double* out6, int* bound) {
  return guarded([&] {
    const DeviceInfo& dev = DeviceInfo::current();
    DeviceCeilings c;
    if (!load_cached_ceilings(dev.device, &c)) c = theoretical_ceilings(dev);
    const Estimate e = estimate_kernel(to_problem(p), kernel_named(name), dev, c);
    const double v[6] = {e.time_us, e.compute_us, e.memory_us, e.launch_us, e.tile_efficiency, e.wave_efficiency};
    std::memcpy(out6, v, sizeof(v));
    if (bound) *bound = int(e.bound);
  });
}

int gie_model_estimate(const char* name, const gie_problem* p, const gie_device_model* d, double* out6, int* bound) {
  return guarded([&] {
    GIE_REQUIRE(d != nullptr && out6 != nullptr, StatusCode::kInvalidArgument, "null device model or output");
    const DeviceInfo dev = modelled_device(*d);
    const Estimate e = estimate_kernel(to_problem(p), kernel_named(name), dev, modelled_ceilings(*d));
    const double v[6] = {e.time_us, e.compute_us, e.memory_us, e.launch_us, e.tile_efficiency, e.wave_efficiency};
    std::memcpy(out6, v, sizeof(v));
    if (bound) *bound = int(e.bound);
  });
}

int gie_model_rank(const gie_problem* p, const gie_device_model* d, char* buf, size_t n, double* us, int max,
                   int* count) {
  return guarded([&] {
    GIE_REQUIRE(d != nullptr, StatusCode::kInvalidArgument, "null device model");
    const ConvProblem pr = to_problem(p);
    validate_problem(pr);
    const DeviceInfo dev = modelled_device(*d);
    const DeviceCeilings c = modelled_ceilings(*d);
    std::vector<std::pair<std::string, double>> order;
    for (const KernelDesc* k : Dispatcher::compatible_kernels(pr, dev))
      order.emplace_back(k->name, estimate_kernel(pr, *k, dev, c).time_us);
    std::stable_sort(order.begin(), order.end(), [](const auto& a, const auto& b) { return a.second < b.second; });
    std::string names;
    for (size_t i = 0; i < order.size(); ++i) {
      if (int(i) < max && us) us[i] = order[i].second;
      if (i) names += "\n";
      names += order[i].first;
    }
    copy_str(names, buf, n);
    if (count) *count = int(order.size());
  });
}

int gie_measure_ceilings(int device, int use_cache, double* out3, int* measured) {
  return guarded([&] {
    const DeviceCeilings c = measure_ceilings(device, use_cache != 0);
    out3[0] = c.fp16_tc_tflops;
    out3[1] = c.bw_gbs;
    out3[2] = c.launch_overhead_us;
    if (measured) *measured = c.measured ? 1 : 0;
  });
}

int gie_theoretical_ceilings(int device, double* out3) {
  return guarded([&] {
    const DeviceCeilings c = theoretical_ceilings(DeviceInfo::get(device));
    out3[0] = c.fp16_tc_tflops;
    out3[1] = c.bw_gbs;
    out3[2] = c.launch_overhead_us;
  });
}

int gie_gpu_reference(const gie_problem* p, const void* x, const void* w, const void* bias, float* y, float* scale,
                      void* stream) {
  return guarded([&] { gpu_conv2d_reference(to_problem(p), x, w, bias, y, scale, static_cast<hipStream_t>(stream)); });
}

int gie_cpu_reference(const gie_problem* p, const float* x, const float* w, const float* bias, float* y,
                      float* scale) {
  return guarded([&] {
    ReferenceOutput out;
    const ConvProblem pr = to_problem(p);
    cpu_conv2d_reference(pr, x, w, bias, &out);
    std::memcpy(y, out.y.data(), out.y.size() * 4);
    std::memcpy(scale, out.scale.data(), out.scale.size() * 4);
  });
}

int gie_make_host_data(const gie_problem* p, uint64_t seed, int dist, int scaling, float* x, float* w, float* bias) {
  return guarded([&] {
    GIE_REQUIRE(dist >= 0 && dist <= 3 && (scaling == 0 || scaling == 1), StatusCode::kInvalidArgument,
                "bad distribution or scaling");
    const ConvProblem pr = to_problem(p);
    validate_problem(pr);
    const Conv2DParams& q = pr.p;
    Rng rng(seed);
    const int64_t nx = q.input_shape().numel(), nw = q.weight_shape().numel();
    auto draw = [&]() -> float {
      switch (dist) {
        case 1: return rng.normal();
        case 2: return rng.uniform() < 0.7 ? 0.f : rng.uniform(-2.f, 2.f);
        case 3: return rng.uniform(0.f, 1.f);
        default: return rng.uniform(-1.f, 1.f);
      }
    };
    const float k = float(q.gemm_k());
    const float wscale = scaling == 1 ? 1.0f / std::sqrt(k) : std::sqrt(3.0f / k);
    const float blim = scaling == 1 ? 0.1f : 1.0f;
    for (int64_t i = 0; i < nx; ++i) x[i] = quantize_to(pr.precision, draw());
    for (int64_t i = 0; i < nw; ++i) w[i] = quantize_to(pr.precision, draw() * wscale);
    const bool half = pr.dtype() != DataType::kFloat32;
    for (int i = 0; i < q.out_channels; ++i) {
      const float v = rng.uniform(-blim, blim);
      bias[i] = half ? quantize_to(pr.precision, v) : v;
    }
  });
}

int gie_device_describe(int device, char* buf, size_t n) {
  return guarded([&] { copy_str(DeviceInfo::get(device).describe(), buf, n); });
}

int gie_device_arch(int device, char* buf, size_t n) {
  return guarded([&] { copy_str(DeviceInfo::get(device).gcn_arch, buf, n); });
}

int gie_device_cu_count(int device, int* cus) {
  return guarded([&] { *cus = DeviceInfo::get(device).sm_count; });
}

int gie_build_fingerprint(char* buf, size_t n) {
  return guarded([&] { copy_str(build_info().source_fingerprint, buf, n); });
}

int gie_graph_create(void** graph) {
  return guarded([&] { *graph = new HipGraphExecutor(); });
}

int gie_graph_destroy(void* graph) {
  return guarded([&] { delete static_cast<HipGraphExecutor*>(graph); });
}

int gie_graph_capture_chain(void* graph, int n, void* const* plans, const void* const* xs, const void* const* ws,
                            const void* const* biases, void* const* ys, void* const* wss, const size_t* ws_bytes) {
  return guarded([&] {
    GIE_REQUIRE(graph != nullptr, StatusCode::kInvalidArgument, "null graph");
    static_cast<HipGraphExecutor*>(graph)->capture(chain_enqueue(n, plans, xs, ws, biases, ys, wss, ws_bytes));
  });
}

int gie_graph_recapture_chain(void* graph, int n, void* const* plans, const void* const* xs, const void* const* ws,
                              const void* const* biases, void* const* ys, void* const* wss, const size_t* ws_bytes,
                              int* updated_in_place) {
  return guarded([&] {
    GIE_REQUIRE(graph != nullptr, StatusCode::kInvalidArgument, "null graph");
    const bool up =
        static_cast<HipGraphExecutor*>(graph)->recapture_update(chain_enqueue(n, plans, xs, ws, biases, ys, wss, ws_bytes));
    if (updated_in_place) *updated_in_place = up ? 1 : 0;
  });
}

int gie_graph_launch(void* graph, void* stream) {
  return guarded([&] {
    GIE_REQUIRE(graph != nullptr, StatusCode::kInvalidArgument, "null graph");
    static_cast<HipGraphExecutor*>(graph)->launch(static_cast<hipStream_t>(stream));
  });
}

int gie_graph_node_count(void* graph, size_t* nodes) {
  return guarded([&] {
    GIE_REQUIRE(graph != nullptr, StatusCode::kInvalidArgument, "null graph");
    *nodes = static_cast<HipGraphExecutor*>(graph)->node_count();
  });
}

int gie_dev_malloc(size_t bytes, void** ptr) {
  return guarded([&] { GIE_HIP_CHECK(hipMalloc(ptr, bytes)); });
}
int gie_dev_free(void* ptr) {
  return guarded([&] { GIE_HIP_CHECK(hipFree(ptr)); });
}
int gie_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return guarded([&] { GIE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)); });
}
int gie_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return guarded([&] { GIE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost)); });
}
int gie_memcpy_d2d_async(void* dst, const void* src, size_t bytes, void* stream) {
  return guarded([&] {
    GIE_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)));
  });
}
int gie_memset(void* ptr, int value, size_t bytes) {
  return guarded([&] {
    GIE_HIP_CHECK(hipMemset(ptr, value, bytes));
    GIE_HIP_CHECK(hipDeviceSynchronize());
  });
}
int gie_device_synchronize(void) {
  return guarded([&] { GIE_HIP_CHECK(hipDeviceSynchronize()); });
}
int gie_get_device_count(int* n) {
  return guarded([&] { GIE_HIP_CHECK(hipGetDeviceCount(n)); });
}
int gie_set_device(int device) {
  return guarded([&] { GIE_HIP_CHECK(hipSetDevice(device)); });
}
int gie_stream_create(void** stream) {
  return guarded([&] {
    hipStream_t s;
    GIE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
  });
}
int gie_stream_destroy(void* stream) {
  return guarded([&] { GIE_HIP_CHECK(hipStreamDestroy(static_cast<hipStream_t>(stream))); });
}
int gie_stream_synchronize(void* stream) {
  return guarded([&] { GIE_HIP_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream))); });
}
int gie_event_create(void** ev) {
  return guarded([&] {
    hipEvent_t e;
    GIE_HIP_CHECK(hipEventCreate(&e));
    *ev = e;
  });
}
int gie_event_destroy(void* ev) {
  return guarded([&] { GIE_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(ev))); });
}
int gie_event_record(void* ev, void* stream) {
  return guarded([&] { GIE_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(stream))); });
}
int gie_event_synchronize(void* ev) {
  return guarded([&] { GIE_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(ev))); });
}
int gie_event_elapsed_ms(void* start, void* stop, float* ms) {
  return guarded([&] {
    GIE_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  });
}

}  // extern "C"

// ---- testing hook: faulty registry entries (kernel_registry_for_testing) ----
namespace {
bool faulty_supports_fp16(const ConvProblem& p, const DeviceInfo&, std::string* why) {
  if (p.precision == Precision::kFp16) return true;
  if (why) *why = "test kernel is fp16 only";
  return false;
}
bool faulty_supports_bf16(const ConvProblem& p, const DeviceInfo&, std::string* why) {
  if (p.precision == Precision::kBf16) return true;
  if (why) *why = "test kernel is bf16 only";
  return false;
}
size_t no_workspace(const ConvProblem&) { return 0; }
void garbage_launch(const LaunchArgs& la) {
  check_kernel_status(gie_hip_fill_u16(la.y, la.problem->p.output_shape().numel(), 0x3c00, la.stream),
                      "garbage fill");
}
void throwing_launch(const LaunchArgs&) { throw Error(StatusCode::kInternal, "deliberately failing test kernel"); }

// gather-table probe: runs only 2x3 filters over 24 input channels (a shape no benchmark or parity case uses), so
// the dispatcher never meets it elsewhere; its "convolution" copies the plan's device table into y
bool lut_probe_shape(const ConvProblem& p, Precision want, std::string* why) {
  if (p.precision == want && p.p.kernel_h == 2 && p.p.kernel_w == 3 && p.p.in_channels == 24) return true;
  if (why) *why = "gather-table probe runs only 2x3 filters over 24 channels";
  return false;
}
bool lut_probe_fp16(const ConvProblem& p, const DeviceInfo&, std::string* why) {
  return lut_probe_shape(p, Precision::kFp16, why);
}
bool lut_probe_bf16(const ConvProblem& p, const DeviceInfo&, std::string* why) {
  return lut_probe_shape(p, Precision::kBf16, why);
}
template <bool CHUNKED>
void lut_probe_launch(const LaunchArgs& la) {
  GIE_REQUIRE(la.plan_data != nullptr, StatusCode::kInternal, "needs_lut kernel launched without a gather table");
  const int64_t k = la.problem->p.gemm_k();
  const size_t table = size_t(CHUNKED ? k / 8 : k) * sizeof(LutEntry);
  const size_t ybytes = size_t(la.problem->p.output_shape().numel()) * dtype_size(la.problem->dtype());
  GIE_HIP_CHECK(hipMemcpyAsync(la.y, la.plan_data, table < ybytes ? table : ybytes, hipMemcpyDeviceToDevice,
                               la.stream));
}
}  // namespace

extern "C" int gie_testing_add_lut_probe_kernels(void) {
  return guarded([&] {
    std::vector<KernelDesc>& reg = kernel_registry_for_testing();
    for (Precision p : {Precision::kFp16, Precision::kBf16}) {
      for (bool chunked : {false, true}) {
        const std::string name = std::string(chunked ? "test_lut_chunked_probe_" : "test_lut_probe_") + to_string(p);
        if (find_kernel(name)) continue;
        GIE_REQUIRE(reg.size() < reg.capacity(), StatusCode::kInternal, "registry capacity exhausted");
        KernelDesc k;
        k.name = name;
        k.backend = Backend::kDirect;
        k.threads_per_block = 64;
        k.needs_lut = true;
        k.lut_chunked = chunked;
        k.efficiency_prior = 1e-6;
        k.supports = p == Precision::kFp16 ? &lut_probe_fp16 : &lut_probe_bf16;
        k.workspace_bytes = &no_workspace;
        k.launch = chunked ? &lut_probe_launch<true> : &lut_probe_launch<false>;
        reg.push_back(std::move(k));
      }
    }
  });
}

extern "C" int gie_testing_add_faulty_kernels(int kind) {
  return guarded([&] {
    GIE_REQUIRE(kind == 0 || kind == 1, StatusCode::kInvalidArgument, "kind must be 0 (garbage) or 1 (throwing)");
    std::vector<KernelDesc>& reg = kernel_registry_for_testing();
    for (Precision p : {Precision::kFp16, Precision::kBf16}) {
      const std::string name = std::string(kind == 0 ? "test_garbage_" : "test_throwing_") + to_string(p);
      if (find_kernel(name)) continue;
      GIE_REQUIRE(reg.size() < reg.capacity(), StatusCode::kInternal, "registry capacity exhausted");
      KernelDesc k;
      k.name = name;
      k.backend = Backend::kTensorCore;
      k.threads_per_block = 256;
      k.tile_m = k.tile_n = k.tile_k = 1024;  // a huge tile: the cost model must not be what rejects it
      k.uses_tensor_cores = true;
      k.efficiency_prior = 1.0;
      k.supports = p == Precision::kFp16 ? &faulty_supports_fp16 : &faulty_supports_bf16;
      k.workspace_bytes = &no_workspace;
      k.launch = kind == 0 ? &garbage_launch : &throwing_launch;
      reg.push_back(std::move(k));
    }
  });
}
