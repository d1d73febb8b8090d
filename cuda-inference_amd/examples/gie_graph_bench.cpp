// gie_graph_bench: what a hipGraph buys over eager dispatch for a chain of convolution layers, and what several
// streams buy for independent convolutions — the measurements of the reference's benchmarks/graph_bench.cpp
// (cases :58-59, depths :60, record fields :124-139 and :175-184 kept so the two result files line up).
//
// Chain: L layers of one plan ping-ponging between two activation buffers (channels and spatial size preserved),
//   eager: L ExecutionPlan::execute_unchecked calls per iteration from the host,
//   graph: one launch of the HipGraphExecutor capture of the same L calls.
// Per (case, L): capture and instantiate cost, device time per iteration (time_stream_work: event pairs around
// back-to-back iterations), host enqueue time per iteration (wall clock, no synchronization inside the loop), and
// whether five graph replays reproduce the eager chain's output bit for bit (input restored before each run).
// Concurrency: S independent convolutions on one stream vs forked over S streams (default priority) and joined.
//
//   gie_graph_bench [--out DIR] [--precision fp16|bf16] [--kernel NAME] [--cases N] [--depths 1,4,16,48]
#include <hip/hip_runtime.h>

#include <chrono>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "gpu_inference/dispatcher.h"
#include "gpu_inference/execution_plan.h"
#include "gpu_inference/hip_graph.h"
#include "gpu_inference/json_lite.h"
#include "gpu_inference/testing.h"
#include "gpu_inference/timing.h"

using namespace gie;

namespace {

struct ChainCase {
  const char* name;
  int batch, channels, hw, k;
};
const ChainCase kCases[] = {{"b1_c32_14x14_k3", 1, 32, 14, 3},
                            {"b1_c64_7x7_k1", 1, 64, 7, 1},
                            {"b1_c64_28x28_k3", 1, 64, 28, 3},
                            {"b4_c128_14x14_k3", 4, 128, 14, 3}};

// median over 7 rounds of the host wall time per call of `enqueue`, the stream drained between rounds only
double host_us_per_call(const std::function<void()>& enqueue, hipStream_t s, int calls = 200) {
  for (int i = 0; i < 20; ++i) enqueue();
  GIE_HIP_CHECK(hipStreamSynchronize(s));
  std::vector<double> per_call;
  for (int round = 0; round < 7; ++round) {
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < calls; ++i) enqueue();
    const auto t1 = std::chrono::steady_clock::now();
    per_call.push_back(std::chrono::duration<double, std::micro>(t1 - t0).count() / calls);
    GIE_HIP_CHECK(hipStreamSynchronize(s));
  }
  return summarize(per_call, 1).median_us;
}

std::vector<unsigned char> bytes_of(const void* dev, size_t n, hipStream_t s) {
  std::vector<unsigned char> h(n);
  GIE_HIP_CHECK(hipStreamSynchronize(s));
  GIE_HIP_CHECK(hipMemcpy(h.data(), dev, n, hipMemcpyDeviceToHost));
  return h;
}

std::vector<int> parse_list(const std::string& s) {
  std::vector<int> v;
  std::stringstream ss(s);
  for (std::string item; std::getline(ss, item, ',');)
    if (!item.empty()) v.push_back(std::stoi(item));
  return v;
}

TimingOptions chain_timing() {
  TimingOptions t;
  t.warmup_iters = 10;
  t.samples = 30;
  t.min_sample_ms = 2.0;
  return t;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    std::string out_dir = "results/graphs", kernel_name;
    Precision prec = Precision::kFp16;
    int n_cases = int(sizeof(kCases) / sizeof(kCases[0]));
    std::vector<int> depths = {1, 4, 16, 48};
    for (int i = 1; i < argc; ++i) {
      const std::string a = argv[i];
      auto next = [&]() -> std::string {
        if (i + 1 >= argc) throw Error(StatusCode::kInvalidArgument, a + " needs a value");
        return argv[++i];
      };
      if (a == "--out") out_dir = next();
      else if (a == "--precision") prec = precision_from_string(next());
      else if (a == "--kernel") kernel_name = next();
      else if (a == "--cases") n_cases = std::min(n_cases, std::max(1, std::stoi(next())));
      else if (a == "--depths") depths = parse_list(next());
      else throw Error(StatusCode::kInvalidArgument, "unknown option " + a);
    }
    GIE_HIP_CHECK(hipSetDevice(0));
    const DeviceInfo& dev = DeviceInfo::get(0);
    std::filesystem::create_directories(out_dir);
    std::ofstream out(out_dir + "/graphs.jsonl", std::ios::app);
    hipStream_t stream = nullptr;
    GIE_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));

    for (int ci = 0; ci < n_cases; ++ci) {
      const ChainCase& c = kCases[ci];
      ConvProblem prob;
      prob.p.batch = c.batch;
      prob.p.in_channels = prob.p.out_channels = c.channels;
      prob.p.in_h = prob.p.in_w = c.hw;
      prob.p.kernel_h = prob.p.kernel_w = c.k;
      prob.p.pad_h = prob.p.pad_w = c.k / 2;
      prob.precision = prec;
      prob.has_bias = true;
      prob.activation = Activation::kReLU;
      // the kernel: named, else the cost model's first choice (no tuning, as the reference's bench)
      const KernelDesc* k = kernel_name.empty() ? nullptr : find_kernel(kernel_name);
      if (!kernel_name.empty() && k == nullptr) throw Error(StatusCode::kInvalidArgument, "no kernel " + kernel_name);
      if (k == nullptr) {
        const auto cands = Dispatcher::compatible_kernels(prob, dev);
        if (cands.empty()) throw Error(StatusCode::kUnsupported, "no kernel runs " + prob.key());
        k = Dispatcher::rank_by_model(prob, dev, cands).front().first;
      }
      const std::shared_ptr<ExecutionPlan> plan = ExecutionPlan::create(prob, *k, 0);
      ConvData d = make_conv_data(prob, 11);
      const size_t act_bytes = d.dy.size();  // == d.dx.size(): the layer preserves the activation shape
      DeviceBuffer ping(act_bytes), pong(act_bytes), ws(plan->workspace_bytes());

      for (int depth : depths) {
        auto chain = [&](hipStream_t s) {
          const void* src = ping.data();
          void* dst = pong.data();
          for (int l = 0; l < depth; ++l) {
            plan->execute_unchecked(src, d.dw.data(), d.db.data(), dst, ws.data(), ws.size(), s);
            const void* prev_dst = dst;
            dst = const_cast<void*>(src);
            src = prev_dst;
          }
        };
        void* last = depth % 2 == 1 ? pong.data() : ping.data();  // buffer the last layer writes
        auto restore_input = [&]() {
          GIE_HIP_CHECK(hipMemcpyAsync(ping.data(), d.dx.data(), act_bytes, hipMemcpyDeviceToDevice, stream));
        };
        HipGraphExecutor graph;
        graph.capture(chain);

        restore_input();
        chain(stream);
        const std::vector<unsigned char> eager_out = bytes_of(last, act_bytes, stream);
        bool identical = true;
        for (int rep = 0; rep < 5; ++rep) {
          restore_input();
          graph.launch(stream);
          identical = identical && bytes_of(last, act_bytes, stream) == eager_out;
        }

        const TimingStats te = time_stream_work(chain, stream, chain_timing());
        const TimingStats tg = time_stream_work([&](hipStream_t s) { graph.launch(s); }, stream, chain_timing());
        const double he = host_us_per_call([&] { chain(stream); }, stream);
        const double hg = host_us_per_call([&] { graph.launch(stream); }, stream);

        json::Value r = json::Value::object();
        r["experiment"] = "F_hip_graphs";
        r["gpu"] = dev.name;
        r["case"] = c.name;
        r["precision"] = to_string(prec);
        r["kernel"] = k->name;
        r["layers"] = depth;
        r["graph_nodes"] = double(graph.node_count());
        r["capture_us"] = graph.capture_us();
        r["instantiate_us"] = graph.instantiate_us();
        r["eager_device_us"] = te.median_us;
        r["graph_device_us"] = tg.median_us;
        r["eager_host_launch_us"] = he;
        r["graph_host_launch_us"] = hg;
        r["device_speedup"] = te.median_us / tg.median_us;
        r["bitwise_identical_replays"] = identical;
        out << r.dump() << "\n";
        out.flush();
        std::cout << c.name << " L=" << depth << " [" << k->name << "] eager " << te.median_us << " us, graph "
                  << tg.median_us << " us (x" << te.median_us / tg.median_us << "), host " << he << " -> " << hg
                  << " us, identical=" << identical << std::endl;
      }

      // S independent copies of the layer: one stream back to back vs one stream each, forked and joined by events
      for (int S : {2, 4, 8}) {
        std::vector<ConvData> data;
        std::vector<DeviceBuffer> wss;
        std::vector<hipStream_t> side(static_cast<size_t>(S));
        std::vector<hipEvent_t> joined(static_cast<size_t>(S));
        for (int s = 0; s < S; ++s) {
          data.push_back(make_conv_data(prob, 100 + uint64_t(s)));
          wss.emplace_back(plan->workspace_bytes());
          GIE_HIP_CHECK(hipStreamCreateWithFlags(&side[size_t(s)], hipStreamNonBlocking));
          GIE_HIP_CHECK(hipEventCreateWithFlags(&joined[size_t(s)], hipEventDisableTiming));
        }
        hipEvent_t forked = nullptr;
        GIE_HIP_CHECK(hipEventCreateWithFlags(&forked, hipEventDisableTiming));
        auto conv = [&](int s, hipStream_t st) {
          const ConvData& cd = data[size_t(s)];
          plan->execute_unchecked(cd.dx.data(), cd.dw.data(), cd.db.data(), cd.dy.data(), wss[size_t(s)].data(),
                                  wss[size_t(s)].size(), st);
        };
        auto one_stream = [&](hipStream_t st) {
          for (int s = 0; s < S; ++s) conv(s, st);
        };
        auto many_streams = [&](hipStream_t st) {
          GIE_HIP_CHECK(hipEventRecord(forked, st));
          for (int s = 0; s < S; ++s) {
            GIE_HIP_CHECK(hipStreamWaitEvent(side[size_t(s)], forked, 0));
            conv(s, side[size_t(s)]);
            GIE_HIP_CHECK(hipEventRecord(joined[size_t(s)], side[size_t(s)]));
          }
          for (int s = 0; s < S; ++s) GIE_HIP_CHECK(hipStreamWaitEvent(st, joined[size_t(s)], 0));
        };
        const TimingStats t1 = time_stream_work(one_stream, stream, chain_timing());
        const TimingStats tn = time_stream_work(many_streams, stream, chain_timing());
        GIE_HIP_CHECK(hipStreamSynchronize(stream));
        json::Value r = json::Value::object();
        r["experiment"] = "F_stream_concurrency";
        r["gpu"] = dev.name;
        r["case"] = c.name;
        r["kernel"] = k->name;
        r["independent_convs"] = S;
        r["one_stream_us"] = t1.median_us;
        r["multi_stream_us"] = tn.median_us;
        r["speedup"] = t1.median_us / tn.median_us;
        out << r.dump() << "\n";
        out.flush();
        std::cout << c.name << " " << S << " independent convs: 1 stream " << t1.median_us << " us, " << S
                  << " streams " << tn.median_us << " us (x" << t1.median_us / tn.median_us << ")" << std::endl;
        for (int s = 0; s < S; ++s) {
          (void)hipStreamDestroy(side[size_t(s)]);
          (void)hipEventDestroy(joined[size_t(s)]);
        }
        (void)hipEventDestroy(forked);
      }
    }
    (void)hipStreamDestroy(stream);
  } catch (const std::exception& e) {
    std::cerr << "error: " << e.what() << "\n";
    return 1;
  }
  return 0;
}
