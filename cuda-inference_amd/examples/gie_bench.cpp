// gie_bench for MI355X: the reference's measurement harness (benchmarks/benchmark_main.cpp) rebuilt on the gie::
// plan API, with the same command line, the same workload-file schema and the same result columns, so workload
// sets and analysis scripts written for the reference apply unchanged.
//
// For every (workload, precision, fusion, backend) the harness
//   * draws the seeded tensors (testing.h) and computes the double-accumulation GPU reference once;
//   * picks the kernel: the autotuner's winner and/or the backend's fixed configuration, a kernel named on the
//     command line, or the dispatcher's own choice;
//   * checks the output against the reference under the tolerance policy before timing anything;
//   * times steady-state launches with HIP events (time_stream_work) and derives TFLOP/s and images/s;
//   * appends one JSON line to results.jsonl and one row to results.csv. Unsupported combinations, failed
//     validations and errors are rows too, with a status and a reason: nothing is dropped.
// Backends: tensor_core (the FP16/BF16/TF32 MFMA families), implicit_gemm (the FP32 MFMA family), dispatcher,
// cpu_reference. The reference's other backend names (direct, im2col_gemm, simt_tiled, cudnn, cudnn_gemm,
// cutlass) are accepted and produce "unsupported" rows that say why. With only cpu_reference requested the
// harness runs without a GPU.
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <functional>
#include <iostream>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "gie_hip.h"
#include "gpu_inference/autotuner.h"
#include "gpu_inference/build_info.h"
#include "gpu_inference/conv2d.h"
#include "gpu_inference/device_info.h"
#include "gpu_inference/dispatcher.h"
#include "gpu_inference/execution_plan.h"
#include "gpu_inference/fused_ops.h"
#include "gpu_inference/json_lite.h"
#include "gpu_inference/kernel_registry.h"
#include "gpu_inference/perf_model.h"
#include "gpu_inference/reference.h"
#include "gpu_inference/testing.h"
#include "gpu_inference/timing.h"

using namespace gie;
using json::Value;

namespace {

// ---------------------------------------------------------------------------------------------------------
// command line (benchmarks/benchmark_main.cpp:80-146: same flags and defaults, plus --scaling)

struct Options {
  std::string workloads = "examples/workloads.json";
  std::string split_label;
  std::vector<std::string> backends = {"tensor_core", "implicit_gemm", "dispatcher"};
  std::vector<std::string> kernels;
  std::vector<Precision> precisions = {Precision::kFp32, Precision::kFp16};
  std::string mode = "tuned";
  std::string fusion = "fused";
  int warmup = 5, samples = 30, tune_samples = 7, model_keep = 0, device = 0, max_workloads = 0;
  double min_sample_ms = 1.0, cpu_max_gflop = 0.3;
  bool flush_l2 = false, validate = true, e2e = false, skip_transfers = false, retune = false, list = false;
  std::string cache_path, filter, category, out_dir = "results/raw/run", tag = "run";
  uint64_t seed = 0x1234ABCDULL;
  Scaling scaling = Scaling::kReference;
};

std::vector<std::string> split_list(const std::string& s) {
  std::vector<std::string> out;
  size_t b = 0;
  while (b <= s.size()) {
    const size_t e = std::min(s.find(',', b), s.size());
    if (e > b) out.push_back(s.substr(b, e - b));
    b = e + 1;
  }
  return out;
}

const char* kUsage =
    "gie_bench [options]\n"
    "  --workloads FILE        workload JSON {\"workloads\": [{\"name\", \"category\", B, C, H, W, O, K|Kh,Kw,\n"
    "                          S|Sh,Sw, P|Ph,Pw, bias, relu}], \"split\"} (default examples/workloads.json)\n"
    "  --split LABEL           split label recorded in every row (default: the file's \"split\")\n"
    "  --backends LIST         tensor_core,implicit_gemm,dispatcher,cpu_reference (default tensor_core,\n"
    "                          implicit_gemm,dispatcher); the reference's direct,im2col_gemm,simt_tiled,cudnn,\n"
    "                          cudnn_gemm,cutlass give 'unsupported' rows\n"
    "  --kernels LIST          also time these registered kernels by name (backend column 'kernel')\n"
    "  --precisions LIST       fp32,fp16,bf16,tf32 (default fp32,fp16)\n"
    "  --mode tuned|fixed|both configuration policy of tensor_core and implicit_gemm\n"
    "  --fusion fused|unfused|both   unfused = conv without epilogue + separate bias and ReLU passes\n"
    "  --warmup N --samples N --min-sample-ms X   timing protocol (defaults 5, 30, 1.0)\n"
    "  --flush-l2              evict L2 before every timed launch (cold-cache protocol)\n"
    "  --no-validate           skip correctness checking\n"
    "  --e2e                   also measure host-synchronous latency and H2D/D2H copies (pinned memory)\n"
    "  --skip-transfers        with --e2e: no H2D/D2H rows\n"
    "  --retune                ignore cached tuning results\n"
    "  --tune-samples N        timing samples per candidate during tuning (default 7)\n"
    "  --model-keep N          tune only the N best candidates of the cost model\n"
    "  --cache FILE            tuning cache path (default $GIE_TUNE_CACHE)\n"
    "  --filter SUBSTR --category NAME --max-workloads N\n"
    "  --out DIR --tag NAME --device N --seed N\n"
    "  --scaling reference|benchmark   data scaling (weights sqrt(3/K), bias U(-1,1) | 1/sqrt(K), U(-0.1,0.1))\n"
    "  --cpu-max-gflop X       run the CPU reference only below X GFLOP (default 0.3)\n"
    "  --list                  print the selected workloads and exit\n";

Options parse_options(int argc, char** argv) {
  Options o;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto value = [&]() -> std::string {
      if (i + 1 >= argc) throw Error(StatusCode::kInvalidArgument, "missing value for " + a);
      return argv[++i];
    };
    auto as_int = [&]() { return std::stoi(value()); };
    if (a == "--workloads") o.workloads = value();
    else if (a == "--split") o.split_label = value();
    else if (a == "--backends") o.backends = split_list(value());
    else if (a == "--kernels") o.kernels = split_list(value());
    else if (a == "--precisions") {
      o.precisions.clear();
      for (const std::string& s : split_list(value())) o.precisions.push_back(precision_from_string(s));
    } else if (a == "--mode") o.mode = value();
    else if (a == "--fusion") o.fusion = value();
    else if (a == "--warmup") o.warmup = as_int();
    else if (a == "--samples") o.samples = as_int();
    else if (a == "--min-sample-ms") o.min_sample_ms = std::stod(value());
    else if (a == "--flush-l2") o.flush_l2 = true;
    else if (a == "--no-validate") o.validate = false;
    else if (a == "--e2e") o.e2e = true;
    else if (a == "--skip-transfers") o.skip_transfers = true;
    else if (a == "--retune") o.retune = true;
    else if (a == "--tune-samples") o.tune_samples = as_int();
    else if (a == "--model-keep") o.model_keep = as_int();
    else if (a == "--cache") o.cache_path = value();
    else if (a == "--filter") o.filter = value();
    else if (a == "--category") o.category = value();
    else if (a == "--max-workloads") o.max_workloads = as_int();
    else if (a == "--out") o.out_dir = value();
    else if (a == "--tag") o.tag = value();
    else if (a == "--device") o.device = as_int();
    else if (a == "--seed") o.seed = std::stoull(value(), nullptr, 0);
    else if (a == "--cpu-max-gflop") o.cpu_max_gflop = std::stod(value());
    else if (a == "--cudnn-ws-mb") value();  // accepted for command-line compatibility; no library baseline here
    else if (a == "--scaling") {
      const std::string s = value();
      if (s == "reference") o.scaling = Scaling::kReference;
      else if (s == "benchmark") o.scaling = Scaling::kBenchmark;
      else throw Error(StatusCode::kInvalidArgument, "--scaling must be reference|benchmark");
    } else if (a == "--list") o.list = true;
    else if (a == "--help" || a == "-h") {
      std::cout << kUsage;
      std::exit(0);
    } else throw Error(StatusCode::kInvalidArgument, "unknown option " + a);
  }
  if (o.mode != "tuned" && o.mode != "fixed" && o.mode != "both")
    throw Error(StatusCode::kInvalidArgument, "--mode must be tuned|fixed|both");
  if (o.fusion != "fused" && o.fusion != "unfused" && o.fusion != "both")
    throw Error(StatusCode::kInvalidArgument, "--fusion must be fused|unfused|both");
  if (o.samples < 1 || o.warmup < 0) throw Error(StatusCode::kInvalidArgument, "--samples >= 1, --warmup >= 0");
  return o;
}

// ---------------------------------------------------------------------------------------------------------
// workloads (benchmark_main.cpp:148-181): W defaults to H, O to C; Kh/Kw to K (3), Sh/Sw to S (1), Ph/Pw to
// P (0); bias and relu default to true.

struct Workload {
  std::string name, category, split;
  Conv2DParams p;
  bool bias = true, relu = true;
};

std::vector<Workload> load_workloads(const Options& o) {
  const Value root = json::parse_file(o.workloads);
  const Value* list = root.find("workloads");
  if (!list || !list->is_array()) throw Error(StatusCode::kIo, o.workloads + ": no 'workloads' array");
  const Value* fs = root.find("split");
  const std::string file_split = fs && fs->is_string() ? fs->as_string() : "unspecified";
  std::vector<Workload> out;
  for (const Value& e : list->elements()) {
    auto num = [&](const char* key, int def) {
      const Value* v = e.find(key);
      return v && v->is_number() ? int(v->as_int()) : def;
    };
    auto str = [&](const char* key, const char* def) {
      const Value* v = e.find(key);
      return v && v->is_string() ? v->as_string() : std::string(def);
    };
    auto flag = [&](const char* key) {
      const Value* v = e.find(key);
      return v ? v->as_bool(true) : true;
    };
    Workload w;
    w.name = str("name", "unnamed");
    w.category = str("category", "uncategorized");
    w.split = o.split_label.empty() ? file_split : o.split_label;
    w.p.batch = num("B", 1);
    w.p.in_channels = num("C", 1);
    w.p.in_h = num("H", 1);
    w.p.in_w = num("W", w.p.in_h);
    w.p.out_channels = num("O", w.p.in_channels);
    const int k = num("K", 3), s = num("S", 1), pad = num("P", 0);
    w.p.kernel_h = num("Kh", k);
    w.p.kernel_w = num("Kw", k);
    w.p.stride_h = num("Sh", s);
    w.p.stride_w = num("Sw", s);
    w.p.pad_h = num("Ph", pad);
    w.p.pad_w = num("Pw", pad);
    w.bias = flag("bias");
    w.relu = flag("relu");
    if (!o.filter.empty() && w.name.find(o.filter) == std::string::npos) continue;
    if (!o.category.empty() && w.category != o.category) continue;
    out.push_back(std::move(w));
    if (o.max_workloads > 0 && int(out.size()) >= o.max_workloads) break;
  }
  return out;
}

// ---------------------------------------------------------------------------------------------------------
// result files (benchmark_main.cpp:183-229): JSON lines with every field, CSV with this fixed column list;
// booleans as 1/0, absent or null fields empty, RFC 4180 quoting.

const std::vector<std::string> kColumns = {
    "tag", "gpu", "cc", "workload", "category", "split", "B", "C", "H", "W", "O", "Kh", "Kw", "Sh", "Sw", "Ph", "Pw",
    "precision", "bias", "relu", "fusion", "backend", "mode", "kernel", "status", "reason", "median_us", "mean_us",
    "min_us", "p10_us", "p90_us", "p99_us", "stddev_us", "samples", "inner_iters", "images_per_s", "tflops",
    "workspace_bytes", "persistent_bytes", "tuning_seconds", "tuning_cache_hit", "setup_seconds", "max_abs_err",
    "frac_over_tol", "worst_tol_ratio", "flops", "compulsory_bytes", "arithmetic_intensity", "model_pred_us",
    "roofline_bound", "conv_only_us", "layout_inclusive_us", "src_fp", "warmup", "layout", "stage_im2col_us",
    "stage_gemm_us", "host_sync_latency_us", "flush_l2", "config"};

std::string csv_cell(const Value* v) {
  if (!v || v->is_null()) return "";
  std::string s;
  if (v->type() == Value::Type::kBool) s = v->as_bool() ? "1" : "0";
  else if (v->is_string()) s = v->as_string();
  else s = v->dump();
  if (s.find_first_of(",\"\n\r") == std::string::npos) return s;
  std::string q = "\"";
  for (char ch : s) {
    if (ch == '"') q += '"';
    q += ch;
  }
  return q + "\"";
}

class ResultFiles {
 public:
  explicit ResultFiles(const std::string& dir) {
    if (std::system(("mkdir -p '" + dir + "'").c_str()) != 0) throw Error(StatusCode::kIo, "cannot create " + dir);
    const std::string csv_path = dir + "/results.csv";
    const bool new_csv = !std::ifstream(csv_path).good();
    jsonl_.open(dir + "/results.jsonl", std::ios::app);
    csv_.open(csv_path, std::ios::app);
    if (!jsonl_ || !csv_) throw Error(StatusCode::kIo, "cannot open the result files in " + dir);
    if (new_csv) {
      for (size_t i = 0; i < kColumns.size(); ++i) csv_ << (i ? "," : "") << kColumns[i];
      csv_ << "\n";
    }
  }
  void append(const Value& r) {
    jsonl_ << r.dump() << "\n";
    jsonl_.flush();
    for (size_t i = 0; i < kColumns.size(); ++i) csv_ << (i ? "," : "") << csv_cell(r.find(kColumns[i]));
    csv_ << "\n";
    csv_.flush();
    ++rows_;
  }
  int rows() const { return rows_; }

 private:
  std::ofstream jsonl_, csv_;
  int rows_ = 0;
};

// ---------------------------------------------------------------------------------------------------------
// run state

struct Bench {
  Options opt;
  bool gpu = false;                  // false: cpu_reference rows only, no device touched
  const DeviceInfo* dev = nullptr;
  DeviceCeilings ceilings;
  hipStream_t stream = nullptr;
  DeviceBuffer flush;
  ResultFiles* out = nullptr;
};

// seeded tensors of one (workload, precision) and the GPU reference output, shared by its backends
struct Inputs {
  ConvData dev;         // device tensors (GPU runs)
  HostConvData host;    // host values (CPU-only runs)
  std::vector<float> ref, scale;
  bool have_ref = false;
  const std::vector<float>& hx() const { return dev.hx.empty() ? host.hx : dev.hx; }
  const std::vector<float>& hw() const { return dev.hw.empty() ? host.hw : dev.hw; }
  const std::vector<float>& hb() const { return dev.hb.empty() ? host.hb : dev.hb; }
};

Inputs make_inputs(const Bench& b, const ConvProblem& prob) {
  Inputs in;
  if (!b.gpu) {
    in.host = make_host_conv_data(prob, b.opt.seed, Distribution::kUniform, b.opt.scaling);
    return in;
  }
  in.dev = make_conv_data(prob, b.opt.seed, Distribution::kUniform, b.opt.scaling);
  if (b.opt.validate) {
    const int64_t n = prob.p.output_shape().numel();
    DeviceBuffer dref(size_t(n) * 4), dscale(size_t(n) * 4);
    gpu_conv2d_reference(prob, in.dev.dx.data(), in.dev.dw.data(), prob.has_bias ? in.dev.db.data() : nullptr,
                         static_cast<float*>(dref.data()), static_cast<float*>(dscale.data()), b.stream);
    GIE_HIP_CHECK(hipStreamSynchronize(b.stream));
    in.ref.resize(size_t(n));
    in.scale.resize(size_t(n));
    GIE_HIP_CHECK(hipMemcpy(in.ref.data(), dref.data(), size_t(n) * 4, hipMemcpyDeviceToHost));
    GIE_HIP_CHECK(hipMemcpy(in.scale.data(), dscale.data(), size_t(n) * 4, hipMemcpyDeviceToHost));
    in.have_ref = true;
  }
  return in;
}

TimingOptions timing_of(const Bench& b) {
  TimingOptions t;
  t.warmup_iters = b.opt.warmup;
  t.samples = b.opt.samples;
  t.min_sample_ms = b.opt.min_sample_ms;
  if (b.opt.flush_l2) {
    t.flush_buffer = b.flush.data();
    t.flush_bytes = b.flush.size();
  }
  return t;
}

Value new_row(const Bench& b, const Workload& wl, const ConvProblem& prob, const std::string& fusion,
              const std::string& backend, const std::string& mode) {
  Value r = Value::object();
  r["tag"] = b.opt.tag;
  r["gpu"] = b.gpu ? b.dev->name : std::string("none");
  r["cc"] = b.gpu ? Value(b.dev->cc()) : Value(nullptr);
  r["arch"] = b.gpu ? b.dev->gcn_arch : std::string("none");
  r["workload"] = wl.name;
  r["category"] = wl.category;
  r["split"] = wl.split;
  const Conv2DParams& p = prob.p;
  r["B"] = p.batch;
  r["C"] = p.in_channels;
  r["H"] = p.in_h;
  r["W"] = p.in_w;
  r["O"] = p.out_channels;
  r["Kh"] = p.kernel_h;
  r["Kw"] = p.kernel_w;
  r["Sh"] = p.stride_h;
  r["Sw"] = p.stride_w;
  r["Ph"] = p.pad_h;
  r["Pw"] = p.pad_w;
  r["precision"] = to_string(prob.precision);
  r["bias"] = prob.has_bias;
  r["relu"] = prob.activation == Activation::kReLU;
  r["fusion"] = fusion;
  r["backend"] = backend;
  r["mode"] = mode;
  r["status"] = "ok";
  r["flops"] = double(p.flops());
  const ProblemModel m = analyze_problem(prob);
  r["compulsory_bytes"] = m.compulsory_bytes;
  r["arithmetic_intensity"] = m.arithmetic_intensity;
  if (b.gpu) {
    const bool mfma = prob.precision == Precision::kFp16 || prob.precision == Precision::kBf16;
    r["roofline_bound"] = to_string(roofline_estimate(prob, b.ceilings, mfma).bound);
  }
  r["flush_l2"] = b.opt.flush_l2;
  r["seed"] = double(b.opt.seed);
  r["src_fp"] = build_info().source_fingerprint;
  r["warmup"] = b.opt.warmup;
  r["layout"] = "NCHW/OIHW";
  return r;
}

void mark_failed(Value& r, const std::string& status, const std::string& reason) {
  r["status"] = status;
  r["reason"] = reason;
}

std::string status_of(const Error& e) {
  if (e.code() == StatusCode::kUnsupported) return "unsupported";
  if (std::string(e.what()).find("out of memory") != std::string::npos) return "oom";
  return "error";
}

void put_timing(Value& r, const TimingStats& t, const ConvProblem& prob) {
  r["median_us"] = t.median_us;
  r["mean_us"] = t.mean_us;
  r["min_us"] = t.min_us;
  r["p10_us"] = t.p10_us;
  r["p90_us"] = t.p90_us;
  r["p99_us"] = t.p99_us;
  r["stddev_us"] = t.stddev_us;
  r["samples"] = t.samples;
  r["inner_iters"] = t.inner_iters;
  if (t.median_us > 0) {
    r["images_per_s"] = double(prob.p.batch) / (t.median_us * 1e-6);
    r["tflops"] = double(prob.p.flops()) / (t.median_us * 1e-6) / 1e12;
  }
}

// Compares a device output with the reference (benchmark_main.cpp:340-355). two_roundings: the output went
// through a separate rounding before the epilogue (unfused passes), which the tolerance allows for.
void check_output(Value& r, const Inputs& in, const ConvProblem& prob, const void* y, bool two_roundings) {
  if (!in.have_ref) {
    r["validated"] = false;
    return;
  }
  const int64_t n = prob.p.output_shape().numel();
  const std::vector<float> got = download_as_float(y, prob.dtype(), n);
  const ErrorMetrics m = compare_outputs(got.data(), in.ref.data(), in.scale.data(), n,
                                         TolerancePolicy::for_problem(prob, two_roundings));
  r["validated"] = true;
  r["max_abs_err"] = m.max_abs;
  r["mean_abs_err"] = m.mean_abs;
  r["rms_err"] = m.rms;
  r["max_rel_err"] = m.max_rel;
  r["rel_l2_err"] = m.rel_l2;
  r["frac_over_tol"] = m.frac_over_tol;
  r["worst_tol_ratio"] = m.worst_tol_ratio;
  r["nan_count"] = double(m.nan_count);
  r["inf_count"] = double(m.inf_count);
  if (!m.passed()) mark_failed(r, "failed_validation", m.summary());
}

// Median of n host-clock measurements of f() followed by a stream sync, after `warm` untimed ones.
double host_sync_us(Bench& b, const std::function<void()>& f, int warm, int n) {
  std::vector<double> us;
  for (int i = 0; i < warm + n; ++i) {
    const auto t0 = std::chrono::steady_clock::now();
    f();
    GIE_HIP_CHECK(hipStreamSynchronize(b.stream));
    if (i >= warm) us.push_back(std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count());
  }
  return summarize(us, 1).median_us;
}

// Validate, then time one kernel (benchmark_main.cpp:359-425). fused: the kernel's own epilogue; unfused: the
// kernel on the problem without bias and ReLU, followed by the stand-alone bias and ReLU passes.
void measure(Bench& b, const ConvProblem& prob, Inputs& in, const KernelDesc& k, const std::string& fusion,
             Value& r) {
  const bool unfused = fusion == "unfused";
  ConvProblem conv = prob;
  if (unfused) {
    conv.has_bias = false;
    conv.activation = Activation::kNone;
  }
  const auto plan = ExecutionPlan::create(conv, k, b.dev->device);
  DeviceBuffer ws(plan->workspace_bytes());
  r["kernel"] = unfused ? k.name + "+bias+relu(unfused)" : k.name;
  r["workspace_bytes"] = double(plan->workspace_bytes());
  r["persistent_bytes"] = double(plan->persistent_bytes());
  r["model_pred_us"] = estimate_kernel(prob, k, *b.dev, b.ceilings).time_us;
  const void* bias = prob.has_bias ? in.dev.db.data() : nullptr;
  void* y = in.dev.dy.data();
  auto run = [&](hipStream_t s, int only_stage) {
    plan->execute_unchecked(in.dev.dx.data(), in.dev.dw.data(), unfused ? nullptr : bias, y, ws.data(), ws.size(), s,
                            nullptr, only_stage);
    if (unfused && only_stage < 0) {
      if (prob.has_bias) launch_bias_add(prob.p, prob.precision, bias, y, s);
      if (prob.activation == Activation::kReLU) launch_relu(prob.p, prob.precision, y, s);
    }
  };

  // no timing for a kernel whose output is wrong
  GIE_HIP_CHECK(hipMemsetAsync(y, 0xFF, in.dev.dy.size(), b.stream));
  run(b.stream, -1);
  GIE_HIP_CHECK(hipStreamSynchronize(b.stream));
  const bool two_roundings =
      prob.precision != Precision::kFp32 && unfused && (prob.has_bias || prob.activation != Activation::kNone);
  check_output(r, in, prob, y, two_roundings);
  if (r.find("status")->as_string() != "ok") return;

  const TimingOptions topt = timing_of(b);
  const TimingStats t = time_stream_work([&](hipStream_t s) { run(s, -1); }, b.stream, topt);
  GIE_HIP_CHECK(hipGetLastError());
  put_timing(r, t, prob);

  // multi-launch kernels: each stage alone, launched back to back on the workspace the full call filled
  // (0 = weight/activation repack where the family has one, 1 = convolution, 2 = split-K reduction)
  if (!unfused && k.launches > 1) {
    int split = 1;
    for (const auto& kv : k.params)
      if (kv.first == "split_k") split = kv.second;
    const bool repack = k.launches - (split > 1 ? 1 : 0) >= 2;
    auto stage_us = [&](int st) {
      return time_stream_work([&](hipStream_t s) { run(s, st); }, b.stream, topt).median_us;
    };
    if (repack) r["stage_repack_us"] = stage_us(0);
    r["stage_conv_us"] = stage_us(1);
    if (split > 1) r["stage_reduce_us"] = stage_us(2);
    run(b.stream, -1);
    GIE_HIP_CHECK(hipStreamSynchronize(b.stream));
  }
  if (b.opt.e2e) r["host_sync_latency_us"] = host_sync_us(b, [&] { run(b.stream, -1); }, 10, 40);
}

// The reference's fixed configuration per backend (benchmark_main.cpp:427-435), mapped to the MI355X registry.
std::string fixed_kernel(const std::string& backend, Precision p) {
  if (backend == "tensor_core" && (p == Precision::kFp16 || p == Precision::kBf16))
    return std::string("mfma_") + to_string(p) + "_128x128x64_w4x2_s3_sk1";
  if (backend == "tensor_core" && p == Precision::kTf32) return "mfma_tf32_128x128x16_sk1";
  if (backend == "implicit_gemm" && p == Precision::kFp32) return "implicit_gemm_fp32_128x128x16_mfma_sk1";
  return "";
}

bool reference_only_backend(const std::string& be, std::string* why) {
  if (be == "direct" || be == "im2col_gemm" || be == "simt_tiled") {
    *why = be + ": no such kernel family on gfx950; every registered kernel is an MFMA implicit GEMM "
                "(backends tensor_core and implicit_gemm)";
    return true;
  }
  if (be == "cudnn" || be == "cudnn_gemm" || be == "cutlass") {
    *why = be + ": vendor-library baselines are not part of this build";
    return true;
  }
  return false;
}

// tensor_core / implicit_gemm rows: the backend's fixed configuration and/or its autotuned winner
// (benchmark_main.cpp:437-482)
void run_custom_backend(Bench& b, const Workload& wl, const ConvProblem& prob, Inputs& in, const std::string& backend,
                        const std::string& fusion) {
  std::vector<std::string> modes;
  if (b.opt.mode == "both") modes = {"fixed", "tuned"};
  else modes = {b.opt.mode};
  ConvProblem conv = prob;
  if (fusion == "unfused") {
    conv.has_bias = false;
    conv.activation = Activation::kNone;
  }
  for (const std::string& mode : modes) {
    Value r = new_row(b, wl, prob, fusion, backend, mode);
    try {
      const KernelDesc* k = nullptr;
      if (mode == "fixed") {
        k = find_kernel(fixed_kernel(backend, prob.precision));
        if (!k)
          throw Error(StatusCode::kUnsupported, "no fixed " + backend + " kernel for " + to_string(prob.precision));
        std::string why;
        if (!k->supports(conv, *b.dev, &why)) throw Error(StatusCode::kUnsupported, k->name + ": " + why);
      } else {
        TuneOptions to;
        to.only_backend = backend_from_string(backend);
        to.cache_path = b.opt.cache_path;
        to.force_retune = b.opt.retune;
        to.model_keep = b.opt.model_keep;
        to.timing.samples = b.opt.tune_samples;
        to.timing.warmup_iters = 3;
        to.timing.min_sample_ms = 0.5;
        const TuneResult tr = Autotuner::tune(conv, *b.dev, to);
        k = find_kernel(tr.best_kernel);
        if (!k) throw Error(StatusCode::kInternal, "autotuner returned an unknown kernel " + tr.best_kernel);
        r["tuning_seconds"] = tr.search_seconds;
        r["tuning_cache_hit"] = tr.from_cache;
        if (!tr.from_cache) {
          r["tune_candidates"] = tr.candidates_measured;
          r["tune_best_us"] = tr.best_us;
        }
      }
      measure(b, prob, in, *k, fusion, r);
    } catch (const Error& e) {
      mark_failed(r, status_of(e), e.what());
    }
    b.out->append(r);
  }
}

void run_named(Bench& b, const Workload& wl, const ConvProblem& prob, Inputs& in, const std::string& name,
               const std::string& fusion) {
  Value r = new_row(b, wl, prob, fusion, "kernel", "named");
  try {
    const KernelDesc* k = find_kernel(name);
    if (!k) throw Error(StatusCode::kUnsupported, "unknown kernel " + name);
    ConvProblem conv = prob;
    if (fusion == "unfused") {
      conv.has_bias = false;
      conv.activation = Activation::kNone;
    }
    std::string why;
    if (!k->supports(conv, *b.dev, &why)) throw Error(StatusCode::kUnsupported, name + ": " + why);
    measure(b, prob, in, *k, fusion, r);
  } catch (const Error& e) {
    mark_failed(r, status_of(e), e.what());
  }
  b.out->append(r);
}

// The dispatcher's autotuned choice, then the host cost of Conv2D::forward against a raw plan launch
// (benchmark_main.cpp:499-548).
void run_dispatcher(Bench& b, const Workload& wl, const ConvProblem& prob, Inputs& in, const std::string& fusion) {
  Value r = new_row(b, wl, prob, fusion, "dispatcher", "auto");
  try {
    if (fusion == "unfused") throw Error(StatusCode::kUnsupported, "the dispatcher is measured fused only");
    Conv2DOptions opt;
    opt.autotune = true;
    opt.force_retune = b.opt.retune;
    opt.cache_path = b.opt.cache_path;
    const auto t0 = std::chrono::steady_clock::now();
    const Selection sel = Dispatcher::select(prob, *b.dev, opt);
    r["tuning_seconds"] = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    r["selection_source"] = to_string(sel.source);
    measure(b, prob, in, *sel.kernel, "fused", r);
    r["config"] = "selected " + sel.kernel->name + " via " + to_string(sel.source);
    if (r.find("status")->as_string() == "ok") {
      Conv2DOptions fo;
      fo.kernel = sel.kernel->name;
      DeviceBuffer ws(Conv2D::workspace_size(prob, fo));
      const ConstTensorRef bias = in.dev.b_ref();
      const auto plan = ExecutionPlan::create(prob, *sel.kernel, b.dev->device);
      // host time per call over 200 enqueues, median of 9 repetitions, after 50 warm calls
      auto per_call_us = [&](const std::function<void()>& f) {
        for (int i = 0; i < 50; ++i) f();
        GIE_HIP_CHECK(hipStreamSynchronize(b.stream));
        std::vector<double> v;
        for (int rep = 0; rep < 9; ++rep) {
          const auto s0 = std::chrono::steady_clock::now();
          for (int i = 0; i < 200; ++i) f();
          v.push_back(std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - s0).count() / 200);
          GIE_HIP_CHECK(hipStreamSynchronize(b.stream));
        }
        return summarize(v, 1).median_us;
      };
      const double api = per_call_us([&] {
        Conv2D::forward(in.dev.x_ref(), in.dev.w_ref(), prob.has_bias ? &bias : nullptr, prob, in.dev.y_ref(),
                        ws.data(), ws.size(), b.stream, fo);
      });
      const double raw = per_call_us([&] {
        plan->execute_unchecked(in.dev.dx.data(), in.dev.dw.data(), prob.has_bias ? in.dev.db.data() : nullptr,
                                in.dev.dy.data(), ws.data(), ws.size(), b.stream);
      });
      r["dispatch_api_host_us"] = api;
      r["raw_launch_host_us"] = raw;
      r["warm_dispatch_overhead_us"] = api - raw;
    }
  } catch (const Error& e) {
    mark_failed(r, status_of(e), e.what());
  }
  b.out->append(r);
}

// The double-accumulation CPU reference timed once (benchmark_main.cpp:603-626); below --cpu-max-gflop only.
void run_cpu_reference(Bench& b, const Workload& wl, const ConvProblem& prob, Inputs& in, const std::string& fusion) {
  Value r = new_row(b, wl, prob, fusion, "cpu_reference", "host");
  try {
    const double gflop = double(prob.p.flops()) / 1e9;
    if (gflop > b.opt.cpu_max_gflop)
      throw Error(StatusCode::kUnsupported,
                  "skipped: " + std::to_string(gflop) + " GFLOP exceeds --cpu-max-gflop");
    ReferenceOutput out;
    const auto t0 = std::chrono::steady_clock::now();
    cpu_conv2d_reference(prob, in.hx().data(), in.hw().data(), prob.has_bias ? in.hb().data() : nullptr, &out);
    const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    r["kernel"] = "cpu_reference(double accum, OpenMP)";
    r["median_us"] = us;
    r["samples"] = 1;
    r["images_per_s"] = double(prob.p.batch) / (us * 1e-6);
    r["tflops"] = double(prob.p.flops()) / (us * 1e-6) / 1e12;
    if (in.have_ref) {
      const ErrorMetrics m = compare_outputs(out.y.data(), in.ref.data(), in.scale.data(), int64_t(out.y.size()),
                                             TolerancePolicy::for_problem(prob));
      r["max_abs_err"] = m.max_abs;
      if (!m.passed()) mark_failed(r, "failed_validation", m.summary());
    }
  } catch (const Error& e) {
    mark_failed(r, status_of(e), e.what());
  }
  b.out->append(r);
}

// Host<->device copies of the inputs and the output through pinned memory (benchmark_main.cpp:628-658).
void run_transfers(Bench& b, const Workload& wl, const ConvProblem& prob) {
  Value r = new_row(b, wl, prob, "n/a", "memcpy", "pinned");
  void *h_in = nullptr, *h_out = nullptr;
  try {
    const size_t esz = dtype_size(prob.dtype());
    const size_t in_bytes = size_t(prob.p.input_shape().numel() + prob.p.weight_shape().numel()) * esz;
    const size_t out_bytes = size_t(prob.p.output_shape().numel()) * esz;
    GIE_HIP_CHECK(hipHostMalloc(&h_in, in_bytes, hipHostMallocDefault));
    GIE_HIP_CHECK(hipHostMalloc(&h_out, out_bytes, hipHostMallocDefault));
    DeviceBuffer d_in(in_bytes), d_out(out_bytes);
    TimingOptions t = timing_of(b);
    t.flush_bytes = 0;
    t.flush_buffer = nullptr;
    t.inner = 1;
    const TimingStats h2d = time_stream_work(
        [&](hipStream_t s) { (void)hipMemcpyAsync(d_in.data(), h_in, in_bytes, hipMemcpyHostToDevice, s); }, b.stream, t);
    const TimingStats d2h = time_stream_work(
        [&](hipStream_t s) { (void)hipMemcpyAsync(h_out, d_out.data(), out_bytes, hipMemcpyDeviceToHost, s); }, b.stream,
        t);
    GIE_HIP_CHECK(hipGetLastError());
    r["kernel"] = "hipMemcpyAsync";
    r["h2d_us"] = h2d.median_us;
    r["d2h_us"] = d2h.median_us;
    r["h2d_bytes"] = double(in_bytes);
    r["d2h_bytes"] = double(out_bytes);
    r["median_us"] = h2d.median_us + d2h.median_us;
  } catch (const Error& e) {
    mark_failed(r, status_of(e), e.what());
  }
  if (h_in) (void)hipHostFree(h_in);
  if (h_out) (void)hipHostFree(h_out);
  b.out->append(r);
}

Value run_meta(const Bench& b, int argc, char** argv) {
  Value m = Value::object();
  m["tag"] = b.opt.tag;
  if (b.gpu) {
    const DeviceInfo& d = *b.dev;
    m["gpu"] = d.name;
    m["arch"] = d.gcn_arch;
    m["compute_capability"] = d.cc();
    m["cu_count"] = d.sm_count;
    m["gpu_memory_bytes"] = double(d.global_mem_bytes);
    m["l2_bytes"] = double(d.l2_bytes);
    m["hip_runtime"] = d.runtime_version;
    m["hip_driver"] = d.driver_version;
    m["est_peak_fp32_tflops"] = d.est_peak_fp32_tflops();
    m["est_peak_fp16_mfma_tflops"] = d.est_peak_fp16_tc_tflops();
    m["est_peak_bw_gbs"] = d.est_peak_bw_gbs();
    m["measured_fp32_tflops"] = b.ceilings.fp32_tflops;
    m["measured_fp16_mfma_tflops"] = b.ceilings.fp16_tc_tflops;
    m["measured_bw_gbs"] = b.ceilings.bw_gbs;
    m["measured_launch_overhead_us"] = b.ceilings.launch_overhead_us;
    m["ceilings_source"] = b.ceilings.source;
  } else {
    m["gpu"] = "none";
  }
  m["library_version"] = kLibraryVersion;
  char host[256] = {0};
  gethostname(host, sizeof(host) - 1);
  m["hostname"] = host;
  const BuildInfo& bi = build_info();
  m["source_fingerprint"] = bi.source_fingerprint;
  m["build_type"] = bi.build_type;
  m["offload_archs"] = bi.offload_archs;
  m["hipcc_version"] = bi.hipcc_version;
  m["cxx_compiler"] = bi.cxx_compiler;
  m["hip_flags"] = bi.hip_flags;
  m["roctx"] = bi.has_roctx;
  m["input_layout"] = "NCHW activations / OIHW weights";
  m["timing_mode"] = b.opt.flush_l2 ? "cold_l2_single_launch_events" : "warm_back_to_back_batched_events";
  m["data_scaling"] = b.opt.scaling == Scaling::kBenchmark ? "benchmark" : "reference";
  m["seed"] = double(b.opt.seed);
  m["warmup"] = b.opt.warmup;
  m["samples"] = b.opt.samples;
  m["min_sample_ms"] = b.opt.min_sample_ms;
  m["flush_l2"] = b.opt.flush_l2;
  Value precs = Value::array();
  for (Precision p : b.opt.precisions) precs.push_back(to_string(p));
  m["precisions"] = precs;
  Value bes = Value::array();
  for (const std::string& s : b.opt.backends) bes.push_back(s);
  m["backends"] = bes;
  std::string cmd;
  for (int i = 0; i < argc; ++i) cmd += std::string(i ? " " : "") + argv[i];
  m["command"] = cmd;
  m["tolerance_policy"] = "tol_i = c_acc*u_acc*sqrt(K)*scale_i + c_out*u_out*|ref_i| + floor (reference.h)";
  return m;
}

// A device fault poisons every later HIP call of the process: stop with the rows written so far instead of
// turning the rest into misleading error rows (benchmark_main.cpp:720-727).
void stop_if_device_lost(const std::string& where) {
  const hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) return;
  std::cerr << "[gie_bench] FATAL: the HIP context is unusable after " << where << ": " << hipGetErrorString(e)
            << ". The rows written so far are valid; run the rest in a fresh process.\n";
  std::exit(4);
}

}  // namespace

int main(int argc, char** argv) {
  try {
    Bench b;
    b.opt = parse_options(argc, argv);
    const std::vector<Workload> workloads = load_workloads(b.opt);
    if (b.opt.list) {
      for (const Workload& w : workloads) std::cout << w.name << "\t" << w.category << "\t" << w.p.to_string() << "\n";
      return 0;
    }
    b.gpu = !b.opt.kernels.empty() ||
            std::any_of(b.opt.backends.begin(), b.opt.backends.end(), [](const std::string& s) {
              std::string why;
              return s != "cpu_reference" && !reference_only_backend(s, &why);
            });
    if (b.gpu) {
      GIE_HIP_CHECK(hipSetDevice(b.opt.device));
      b.dev = &DeviceInfo::get(b.opt.device);
      b.ceilings = measure_ceilings(b.opt.device, true);
      GIE_HIP_CHECK(hipStreamCreateWithFlags(&b.stream, hipStreamNonBlocking));
      if (b.opt.flush_l2) b.flush = DeviceBuffer(std::max<size_t>(2 * b.dev->l2_bytes, size_t(128) << 20));
    } else {
      b.opt.validate = false;  // the GPU reference is the oracle; without a GPU the CPU rows carry no error
    }
    ResultFiles files(b.opt.out_dir);
    b.out = &files;
    json::write_file(b.opt.out_dir + "/meta.json", run_meta(b, argc, argv));
    std::cerr << "[gie_bench] " << (b.gpu ? b.dev->describe() : std::string("no GPU (cpu_reference rows only)"))
              << "\n[gie_bench] " << workloads.size() << " workloads -> " << b.opt.out_dir << "\n";

    int idx = 0;
    for (const Workload& wl : workloads) {
      ++idx;
      for (Precision prec : b.opt.precisions) {
        ConvProblem prob;
        prob.p = wl.p;
        prob.precision = prec;
        prob.has_bias = wl.bias;
        prob.activation = wl.relu ? Activation::kReLU : Activation::kNone;
        std::cerr << "[" << idx << "/" << workloads.size() << "] " << wl.name << " " << to_string(prec) << " "
                  << prob.p.to_string() << std::endl;
        try {
          validate_problem(prob);
          if (b.gpu) {
            // x, w, y, the FP32 reference and its scales, and an equal margin for workspaces
            const ProblemModel pm = analyze_problem(prob);
            const double need = double(prob.p.output_shape().numel()) * 8.0 + 2.0 * pm.compulsory_bytes +
                                pm.im2col_bytes;
            if (need > 0.85 * double(b.dev->global_mem_bytes))
              throw Error(StatusCode::kUnsupported, "skipped_memory: working set exceeds the device memory budget");
          }
          Inputs in = make_inputs(b, prob);
          if (b.gpu && b.opt.e2e && !b.opt.skip_transfers) run_transfers(b, wl, prob);
          std::vector<std::string> fusions = {b.opt.fusion};
          if (b.opt.fusion == "both") fusions = {"fused", "unfused"};
          const bool epilogue = prob.has_bias || prob.activation != Activation::kNone;
          for (const std::string& fusion : fusions) {
            if (fusion == "unfused" && !epilogue) continue;  // would repeat the fused rows
            for (const std::string& be : b.opt.backends) {
              // the fusion experiment is per kernel: the dispatcher and the CPU reference take no part in it
              if (fusion == "unfused" && be != "tensor_core" && be != "implicit_gemm") continue;
              std::string why;
              if (reference_only_backend(be, &why)) {
                Value r = new_row(b, wl, prob, fusion, be, "n/a");
                mark_failed(r, "unsupported", why);
                files.append(r);
                continue;
              }
              if (be == "cpu_reference") run_cpu_reference(b, wl, prob, in, fusion);
              else if (be == "dispatcher") run_dispatcher(b, wl, prob, in, fusion);
              else if (be == "tensor_core" || be == "implicit_gemm") run_custom_backend(b, wl, prob, in, be, fusion);
              else {
                Value r = new_row(b, wl, prob, fusion, be, "n/a");
                mark_failed(r, "unsupported", "unknown backend " + be);
                files.append(r);
                continue;
              }
              if (b.gpu) stop_if_device_lost(be);
            }
            if (fusion == "fused")
              for (const std::string& kn : b.opt.kernels) {
                run_named(b, wl, prob, in, kn, fusion);
                stop_if_device_lost(kn);
              }
          }
        } catch (const Error& e) {
          // the workload itself failed: one row per requested backend, nothing silently dropped
          for (const std::string& be : b.opt.backends) {
            Value r = new_row(b, wl, prob, "fused", be, "n/a");
            mark_failed(r, status_of(e), e.what());
            files.append(r);
          }
          std::cerr << "  workload failed: " << e.what() << "\n";
          if (b.gpu) (void)hipGetLastError();
        }
      }
    }
    std::cerr << "[gie_bench] done: " << files.rows() << " rows\n";
    if (b.stream) (void)hipStreamDestroy(b.stream);
  } catch (const std::exception& e) {
    std::cerr << "fatal: " << e.what() << "\n";
    return 1;
  }
  return 0;
}
