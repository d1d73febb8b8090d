// gie_graph_bench — launch overhead on one MI355X: what replaying a recorded HIP graph buys over enqueueing the same
// convolution layers one by one, what several streams buy for independent layers, and what a graph launch itself
// costs. The questions, the four layer cases and the depth list are those of the reference's
// benchmarks/graph_bench.cpp (:55-58 cases and depths), and each JSON record carries that program's field names
// (:120-139, :172-184) so the two result files line up; the program is this build's own.
//
// How it is organised:
//   * Rig — one layer: its plan, weights, bias, workspace and three activation buffers (the pristine input, and the
//     two buffers a chain alternates between). chain(stream, L) enqueues L layers; restore() resets the input.
//   * Probe — every timing: device time per iteration through the library's time_stream_work, host time as the
//     median over batches of enqueues. When two ways of enqueueing are compared their host batches alternate, so both
//     see the same machine state (clocks, queue depth, other load).
//   * Three experiments, each a function returning records: chain (graph vs eager per depth, with a bitwise check of
//     repeated replays against the eager chain), fanout (S independent layers on one stream vs one stream each, joined
//     back), and floor (graphs of N empty kernels launched as instantiated, and again after hipGraphUpload, against N
//     eager empty launches) — the floor separates what a graph launch costs from what the layers cost — and launch
//     arguments (one eager empty launch with 0, 8, 128 and 1024 argument bytes).
//   * Output: one JSON record per measurement appended to <out>/graphs.jsonl; with --md FILE the same results as
//     markdown tables.
//
//   gie_graph_bench [--out DIR] [--md FILE] [--precision fp16|bf16] [--kernel NAME] [--cases N]
//                   [--depths 1,4,16,48] [--no-floor]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iomanip>
#include <iterator>
#include <iostream>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "gie_hip.h"
#include "gpu_inference/dispatcher.h"
#include "gpu_inference/execution_plan.h"
#include "gpu_inference/hip_graph.h"
#include "gpu_inference/json_lite.h"
#include "gpu_inference/testing.h"
#include "gpu_inference/timing.h"

using namespace gie;

namespace {

struct LayerCase {
  const char* name;
  int batch, channels, hw, k;
};
constexpr LayerCase kLayerCases[] = {{"b1_c32_14x14_k3", 1, 32, 14, 3},
                                     {"b1_c64_7x7_k1", 1, 64, 7, 1},
                                     {"b1_c64_28x28_k3", 1, 64, 28, 3},
                                     {"b4_c128_14x14_k3", 4, 128, 14, 3}};
constexpr int kFanouts[] = {2, 4, 8};
constexpr int kFloorNodes[] = {1, 4, 16, 64};

using Enqueue = std::function<void(hipStream_t)>;

// ---- timing ---------------------------------------------------------------------------------------------------------

class Probe {
 public:
  explicit Probe(hipStream_t s) : s_(s) {
    dev_.warmup_iters = 10;
    dev_.samples = 30;
    dev_.min_sample_ms = 2.0;
  }

  // device microseconds per call of `work`, back to back on the stream (median sample)
  double device_us(const Enqueue& work) const { return time_stream_work(work, s_, dev_).median_us; }

  // host microseconds to enqueue one call of a and of b: batches of each, in alternation, the stream drained after
  // every batch so queue depth does not build up; median per-call time of each
  std::pair<double, double> host_us(const Enqueue& a, const Enqueue& b) const {
    for (int i = 0; i < 16; ++i) {
      a(s_);
      b(s_);
    }
    drain();
    std::vector<double> ta, tb;
    for (int round = 0; round < kRounds; ++round) {
      ta.push_back(batch_us(a));
      tb.push_back(batch_us(b));
    }
    return {summarize(ta, 1).median_us, summarize(tb, 1).median_us};
  }

  void drain() const { GIE_HIP_CHECK(hipStreamSynchronize(s_)); }
  hipStream_t stream() const { return s_; }

 private:
  static constexpr int kRounds = 9, kCalls = 128;
  double batch_us(const Enqueue& f) const {
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < kCalls; ++i) f(s_);
    const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    drain();
    return us / kCalls;
  }
  hipStream_t s_;
  TimingOptions dev_;
};

// ---- one layer and its buffers ---------------------------------------------------------------------------------------

class Rig {
 public:
  Rig(const ConvProblem& prob, const KernelDesc& kernel, uint64_t seed)
      : prob_(prob), kernel_(kernel), plan_(ExecutionPlan::create(prob, kernel, 0)),
        data_(make_conv_data(prob, seed)), bytes_(data_.dy.size()), act_{DeviceBuffer(bytes_), DeviceBuffer(bytes_)},
        ws_(std::max<size_t>(plan_->workspace_bytes(), 256)) {
    GIE_REQUIRE(data_.dx.size() == bytes_, StatusCode::kInvalidArgument,
                "a chain layer must keep its activation shape (same channels in and out, stride 1, same padding)");
  }

  // layer l reads act_[l % 2] and writes act_[(l + 1) % 2]
  void chain(hipStream_t s, int layers) const {
    for (int l = 0; l < layers; ++l)
      plan_->execute_unchecked(act_[l % 2].data(), data_.dw.data(), data_.db.data(), act_[(l + 1) % 2].data(),
                               ws_.data(), ws_.size(), s);
  }
  // one layer on the rig's own input and output (independent of every other rig)
  void single(hipStream_t s) const {
    plan_->execute_unchecked(data_.dx.data(), data_.dw.data(), data_.db.data(), data_.dy.data(), ws_.data(), ws_.size(),
                             s);
  }
  void restore(hipStream_t s) const {
    GIE_HIP_CHECK(hipMemcpyAsync(act_[0].data(), data_.dx.data(), bytes_, hipMemcpyDeviceToDevice, s));
  }
  // raw bytes of a chain's output, after the stream has finished
  std::vector<unsigned char> result(hipStream_t s, int layers) const {
    std::vector<unsigned char> h(bytes_);
    GIE_HIP_CHECK(hipStreamSynchronize(s));
    GIE_HIP_CHECK(hipMemcpy(h.data(), act_[layers % 2].data(), bytes_, hipMemcpyDeviceToHost));
    return h;
  }
  const ConvProblem& problem() const { return prob_; }
  const KernelDesc& kernel() const { return kernel_; }

 private:
  ConvProblem prob_;
  const KernelDesc& kernel_;
  std::shared_ptr<ExecutionPlan> plan_;
  ConvData data_;
  size_t bytes_;
  DeviceBuffer act_[2];
  DeviceBuffer ws_;
};

ConvProblem problem_of(const LayerCase& c, Precision prec) {
  ConvProblem p;
  p.p.batch = c.batch;
  p.p.in_channels = p.p.out_channels = c.channels;
  p.p.in_h = p.p.in_w = c.hw;
  p.p.kernel_h = p.p.kernel_w = c.k;
  p.p.pad_h = p.p.pad_w = c.k / 2;
  p.precision = prec;
  p.has_bias = true;
  p.activation = Activation::kReLU;
  return p;
}

// the named kernel, else the cost model's first choice (no tuning: the question is launch overhead, not the kernel)
const KernelDesc& kernel_for(const ConvProblem& p, const DeviceInfo& dev, const std::string& forced) {
  if (!forced.empty()) {
    const KernelDesc* k = find_kernel(forced);
    GIE_REQUIRE(k != nullptr, StatusCode::kInvalidArgument, "unknown kernel " + forced);
    return *k;
  }
  const auto ranked = Dispatcher::rank_by_model(p, dev, Dispatcher::compatible_kernels(p, dev));
  GIE_REQUIRE(!ranked.empty(), StatusCode::kUnsupported, "no kernel for " + p.key());
  return *ranked.front().first;
}

// ---- experiments -------------------------------------------------------------------------------------------------------

json::Value record(const char* experiment, const DeviceInfo& dev) {
  json::Value r = json::Value::object();
  r["experiment"] = experiment;
  r["gpu"] = dev.name;
  return r;
}

std::vector<json::Value> chain_experiment(const Rig& rig, const std::vector<int>& depths, const Probe& probe,
                                          const DeviceInfo& dev, const std::string& case_name) {
  std::vector<json::Value> out;
  for (const int L : depths) {
    const Enqueue eager = [&](hipStream_t s) { rig.chain(s, L); };
    HipGraphExecutor graph;
    graph.capture(eager);
    const Enqueue replay = [&](hipStream_t s) { graph.launch(s); };

    // every replay must reproduce the eager chain bit for bit, each from the restored input
    rig.restore(probe.stream());
    eager(probe.stream());
    const std::vector<unsigned char> want = rig.result(probe.stream(), L);
    bool identical = true;
    for (int rep = 0; rep < 5; ++rep) {
      rig.restore(probe.stream());
      replay(probe.stream());
      identical = identical && rig.result(probe.stream(), L) == want;
    }

    const double dev_eager = probe.device_us(eager), dev_graph = probe.device_us(replay);
    const auto [host_eager, host_graph] = probe.host_us(eager, replay);
    json::Value r = record("F_hip_graphs", dev);
    r["case"] = case_name;
    r["precision"] = to_string(rig.problem().precision);
    r["kernel"] = rig.kernel().name;
    r["layers"] = L;
    r["graph_nodes"] = double(graph.node_count());
    r["capture_us"] = graph.capture_us();
    r["instantiate_us"] = graph.instantiate_us();
    r["eager_device_us"] = dev_eager;
    r["graph_device_us"] = dev_graph;
    r["eager_host_launch_us"] = host_eager;
    r["graph_host_launch_us"] = host_graph;
    r["device_speedup"] = dev_eager / dev_graph;
    r["bitwise_identical_replays"] = identical;
    out.push_back(r);
  }
  return out;
}

// S streams that fan out from a parent stream and join back into it
class Fanout {
 public:
  explicit Fanout(int n) : lanes_(size_t(n)), joined_(size_t(n)) {
    for (size_t i = 0; i < lanes_.size(); ++i) {
      GIE_HIP_CHECK(hipStreamCreateWithFlags(&lanes_[i], hipStreamNonBlocking));
      GIE_HIP_CHECK(hipEventCreateWithFlags(&joined_[i], hipEventDisableTiming));
    }
    GIE_HIP_CHECK(hipEventCreateWithFlags(&forked_, hipEventDisableTiming));
  }
  ~Fanout() {
    for (size_t i = 0; i < lanes_.size(); ++i) {
      (void)hipStreamSynchronize(lanes_[i]);
      (void)hipEventDestroy(joined_[i]);
      (void)hipStreamDestroy(lanes_[i]);
    }
    (void)hipEventDestroy(forked_);
  }
  Fanout(const Fanout&) = delete;
  Fanout& operator=(const Fanout&) = delete;

  // lane i runs work(i, lane i) after everything already on `parent`; parent continues once every lane is done
  void run(hipStream_t parent, const std::function<void(int, hipStream_t)>& work) const {
    GIE_HIP_CHECK(hipEventRecord(forked_, parent));
    for (size_t i = 0; i < lanes_.size(); ++i) {
      GIE_HIP_CHECK(hipStreamWaitEvent(lanes_[i], forked_, 0));
      work(int(i), lanes_[i]);
      GIE_HIP_CHECK(hipEventRecord(joined_[i], lanes_[i]));
    }
    for (hipEvent_t e : joined_) GIE_HIP_CHECK(hipStreamWaitEvent(parent, e, 0));
  }

 private:
  std::vector<hipStream_t> lanes_;
  std::vector<hipEvent_t> joined_;
  hipEvent_t forked_ = nullptr;
};

std::vector<json::Value> fanout_experiment(const ConvProblem& prob, const KernelDesc& kernel, const Probe& probe,
                                           const DeviceInfo& dev, const std::string& case_name) {
  std::vector<json::Value> out;
  for (const int S : kFanouts) {
    std::vector<std::unique_ptr<Rig>> rigs;
    for (int i = 0; i < S; ++i) rigs.push_back(std::make_unique<Rig>(prob, kernel, 100 + uint64_t(i)));
    const Fanout fan(S);
    const Enqueue one_stream = [&](hipStream_t s) {
      for (const auto& r : rigs) r->single(s);
    };
    const Enqueue own_streams = [&](hipStream_t s) { fan.run(s, [&](int i, hipStream_t lane) { rigs[size_t(i)]->single(lane); }); };
    const double t1 = probe.device_us(one_stream), tn = probe.device_us(own_streams);
    probe.drain();
    json::Value r = record("F_stream_concurrency", dev);
    r["case"] = case_name;
    r["kernel"] = kernel.name;
    r["independent_convs"] = S;
    r["one_stream_us"] = t1;
    r["multi_stream_us"] = tn;
    r["speedup"] = t1 / tn;
    out.push_back(r);
  }
  return out;
}

std::vector<json::Value> floor_experiment(const Probe& probe, const DeviceInfo& dev) {
  std::vector<json::Value> out;
  for (const int n : kFloorNodes) {
    const Enqueue eager = [n](hipStream_t s) {
      for (int i = 0; i < n; ++i) check_kernel_status(gie_hip_ceiling_empty(s), "empty kernel");
    };
    HipGraphExecutor plain, uploaded;
    plain.capture(eager);
    uploaded.capture(eager);
    uploaded.upload(probe.stream());
    probe.drain();
    const Enqueue launch_plain = [&](hipStream_t s) { plain.launch(s); };
    const Enqueue launch_uploaded = [&](hipStream_t s) { uploaded.launch(s); };
    const auto [host_eager, host_plain] = probe.host_us(eager, launch_plain);
    const auto [host_eager2, host_uploaded] = probe.host_us(eager, launch_uploaded);
    json::Value r = record("F_graph_launch_floor", dev);
    r["empty_kernels"] = n;
    r["graph_nodes"] = double(plain.node_count());
    r["eager_host_launch_us"] = 0.5 * (host_eager + host_eager2);
    r["graph_host_launch_us"] = host_plain;
    r["uploaded_graph_host_launch_us"] = host_uploaded;
    r["eager_device_us"] = probe.device_us(eager);
    r["graph_device_us"] = probe.device_us(launch_plain);
    r["uploaded_graph_device_us"] = probe.device_us(launch_uploaded);
    out.push_back(r);
  }
  return out;
}

// What one eager launch costs the host as a function of its argument block: the empty kernel with 0, 8, 128 and
// 1024 argument bytes, host time per enqueue (batches alternating with the 0-byte launch) and device time per launch
// back to back. The record carries HIP_FORCE_DEV_KERNARG as set for the run (HIP's default copies a non-empty block
// to device memory).
std::vector<json::Value> launch_args_experiment(const Probe& probe, const DeviceInfo& dev) {
  std::vector<json::Value> out;
  const char* env = std::getenv("HIP_FORCE_DEV_KERNARG");
  const Enqueue none = [](hipStream_t s) { check_kernel_status(gie_hip_ceiling_empty(s), "empty kernel"); };
  for (const int bytes : {0, 8, 128, 1024}) {
    const Enqueue with_args = [bytes](hipStream_t s) {
      if (bytes == 0) check_kernel_status(gie_hip_ceiling_empty(s), "empty kernel");
      else check_kernel_status(gie_hip_ceiling_empty_args(bytes, s), "empty kernel with arguments");
    };
    const auto [host_none, host_args] = probe.host_us(none, with_args);
    json::Value r = record("F_launch_args", dev);
    r["arg_bytes"] = bytes;
    r["HIP_FORCE_DEV_KERNARG"] = env ? std::string(env) : std::string("unset");
    r["host_launch_us"] = host_args;
    r["host_launch_us_no_args"] = host_none;
    r["device_us"] = probe.device_us(with_args);
    out.push_back(r);
  }
  return out;
}

// ---- reporting ---------------------------------------------------------------------------------------------------------

std::string fmt(double v, int digits = 1) {
  std::ostringstream o;
  o << std::fixed << std::setprecision(digits) << v;
  return o.str();
}

std::string markdown(const std::vector<json::Value>& rows) {
  std::ostringstream md;
  auto num = [](const json::Value& r, const char* k) { return r.find(k) ? r.find(k)->as_double() : 0.0; };
  auto str = [](const json::Value& r, const char* k) { return r.find(k) ? r.find(k)->as_string() : std::string(); };
  auto of = [&](const char* experiment) {
    std::vector<const json::Value*> v;
    for (const auto& r : rows)
      if (str(r, "experiment") == experiment) v.push_back(&r);
    return v;
  };
  if (const auto f = of("F_graph_launch_floor"); !f.empty()) {
    md << "| empty kernels | graph nodes | host µs eager → graph → uploaded graph | device µs eager → graph → "
          "uploaded graph |\n|---|---|---|---|\n";
    for (const json::Value* r : f)
      md << "| " << num(*r, "empty_kernels") << " | " << num(*r, "graph_nodes") << " | "
         << fmt(num(*r, "eager_host_launch_us")) << " → " << fmt(num(*r, "graph_host_launch_us")) << " → "
         << fmt(num(*r, "uploaded_graph_host_launch_us")) << " | " << fmt(num(*r, "eager_device_us")) << " → "
         << fmt(num(*r, "graph_device_us")) << " → " << fmt(num(*r, "uploaded_graph_device_us")) << " |\n";
    md << "\n";
  }
  if (const auto a = of("F_launch_args"); !a.empty()) {
    md << "| argument bytes | HIP_FORCE_DEV_KERNARG | host µs per launch (0-byte launch alongside) | device µs per "
          "launch |\n|---|---|---|---|\n";
    for (const json::Value* r : a)
      md << "| " << num(*r, "arg_bytes") << " | " << str(*r, "HIP_FORCE_DEV_KERNARG") << " | "
         << fmt(num(*r, "host_launch_us"), 2) << " (" << fmt(num(*r, "host_launch_us_no_args"), 2) << ") | "
         << fmt(num(*r, "device_us"), 2) << " |\n";
    md << "\n";
  }
  if (const auto c = of("F_hip_graphs"); !c.empty()) {
    md << "| case | kernel | L | eager device µs | graph device µs | speedup | host µs eager → graph | capture + "
          "instantiate µs | replays bitwise |\n|---|---|---|---|---|---|---|---|---|\n";
    for (const json::Value* r : c)
      md << "| " << str(*r, "case") << " | `" << str(*r, "kernel") << "` | " << num(*r, "layers") << " | "
         << fmt(num(*r, "eager_device_us")) << " | " << fmt(num(*r, "graph_device_us")) << " | "
         << fmt(num(*r, "device_speedup"), 2) << " | " << fmt(num(*r, "eager_host_launch_us")) << " → "
         << fmt(num(*r, "graph_host_launch_us")) << " | " << fmt(num(*r, "capture_us"), 0) << " + "
         << fmt(num(*r, "instantiate_us"), 0) << " | "
         << (r->find("bitwise_identical_replays")->as_bool() ? "yes" : "NO") << " |\n";
    md << "\n";
  }
  if (const auto s = of("F_stream_concurrency"); !s.empty()) {
    md << "| case | independent convs S | one stream µs | S streams µs | speedup |\n|---|---|---|---|---|\n";
    for (const json::Value* r : s)
      md << "| " << str(*r, "case") << " | " << num(*r, "independent_convs") << " | " << fmt(num(*r, "one_stream_us"))
         << " | " << fmt(num(*r, "multi_stream_us")) << " | " << fmt(num(*r, "speedup"), 2) << " |\n";
  }
  return md.str();
}

struct Args {
  std::string out_dir = "results/graphs", md_path, kernel;
  Precision precision = Precision::kFp16;
  int cases = int(std::size(kLayerCases));
  std::vector<int> depths = {1, 4, 16, 48};
  bool floor = true;
};

Args parse(int argc, char** argv) {
  Args a;
  for (int i = 1; i < argc; ++i) {
    const std::string opt = argv[i];
    const auto value = [&]() -> std::string {
      GIE_REQUIRE(i + 1 < argc, StatusCode::kInvalidArgument, opt + " needs a value");
      return argv[++i];
    };
    if (opt == "--out") {
      a.out_dir = value();
    } else if (opt == "--md") {
      a.md_path = value();
    } else if (opt == "--precision") {
      a.precision = precision_from_string(value());
    } else if (opt == "--kernel") {
      a.kernel = value();
    } else if (opt == "--cases") {
      a.cases = std::clamp(std::stoi(value()), 1, int(std::size(kLayerCases)));
    } else if (opt == "--depths") {
      a.depths.clear();
      std::stringstream list(value());
      for (std::string d; std::getline(list, d, ',');)
        if (!d.empty()) a.depths.push_back(std::stoi(d));
    } else if (opt == "--no-floor") {
      a.floor = false;
    } else {
      throw Error(StatusCode::kInvalidArgument, "unknown option " + opt);
    }
  }
  return a;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Args args = parse(argc, argv);
    GIE_HIP_CHECK(hipSetDevice(0));
    const DeviceInfo& dev = DeviceInfo::get(0);
    std::filesystem::create_directories(args.out_dir);
    std::ofstream jsonl(args.out_dir + "/graphs.jsonl", std::ios::app);
    hipStream_t stream = nullptr;
    GIE_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    std::vector<json::Value> all;
    {
      const Probe probe(stream);
      auto emit = [&](std::vector<json::Value> rows) {
        for (json::Value& r : rows) {
          jsonl << r.dump() << "\n";
          std::cout << r.dump() << "\n";
          all.push_back(std::move(r));
        }
        jsonl.flush();
        std::cout.flush();
      };
      if (args.floor) {
        emit(launch_args_experiment(probe, dev));
        emit(floor_experiment(probe, dev));
      }
      for (int ci = 0; ci < args.cases; ++ci) {
        const ConvProblem prob = problem_of(kLayerCases[ci], args.precision);
        const KernelDesc& kernel = kernel_for(prob, dev, args.kernel);
        const Rig rig(prob, kernel, 11);
        emit(chain_experiment(rig, args.depths, probe, dev, kLayerCases[ci].name));
        emit(fanout_experiment(prob, kernel, probe, dev, kLayerCases[ci].name));
      }
      probe.drain();
    }
    if (!args.md_path.empty()) std::ofstream(args.md_path) << markdown(all);
    GIE_HIP_CHECK(hipStreamDestroy(stream));
  } catch (const std::exception& e) {
    std::cerr << "gie_graph_bench: " << e.what() << "\n";
    return 1;
  }
  return 0;
}
