// hipGraph capture / update / replay of an enqueue function (the reference's cuda_graph.cpp on HIP graphs).
#include "gpu_inference/hip_graph.h"

#include <hip/hip_runtime.h>

#include <chrono>

#include "gpu_inference/roctx.h"

namespace gie {
namespace {
using clock = std::chrono::steady_clock;
double us_since(clock::time_point t0) { return std::chrono::duration<double, std::micro>(clock::now() - t0).count(); }

struct StreamGuard {
  hipStream_t s;
  ~StreamGuard() { (void)hipStreamDestroy(s); }
};
}  // namespace

HipGraphExecutor::~HipGraphExecutor() { reset(); }

void HipGraphExecutor::reset() {
  if (exec_) (void)hipGraphExecDestroy(exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  exec_ = nullptr;
  graph_ = nullptr;
  nodes_ = 0;
}

void HipGraphExecutor::capture_graph(const Enqueue& enqueue, hipGraph_t* g, double* us) {
  hipStream_t s;
  GIE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  StreamGuard guard{s};
  const auto t0 = clock::now();
  GIE_HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  try {
    enqueue(s);
  } catch (...) {
    hipGraph_t partial = nullptr;
    (void)hipStreamEndCapture(s, &partial);
    if (partial) (void)hipGraphDestroy(partial);
    throw;
  }
  GIE_HIP_CHECK(hipStreamEndCapture(s, g));
  *us = us_since(t0);
}

void HipGraphExecutor::capture(const Enqueue& enqueue) {
  RoctxRange range("gie::HipGraphExecutor::capture");
  reset();
  {
    hipStream_t warm;
    GIE_HIP_CHECK(hipStreamCreateWithFlags(&warm, hipStreamNonBlocking));
    StreamGuard guard{warm};
    enqueue(warm);
    GIE_HIP_CHECK(hipStreamSynchronize(warm));
  }
  capture_graph(enqueue, &graph_, &capture_us_);
  const auto t0 = clock::now();
  GIE_HIP_CHECK(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0));
  instantiate_us_ = us_since(t0);
  size_t n = 0;
  GIE_HIP_CHECK(hipGraphGetNodes(graph_, nullptr, &n));
  nodes_ = n;
}

bool HipGraphExecutor::recapture_update(const Enqueue& enqueue) {
  if (!exec_) {
    capture(enqueue);
    return false;
  }
  hipGraph_t g2 = nullptr;
  double us = 0;
  capture_graph(enqueue, &g2, &us);
  capture_us_ = us;
  hipGraphNode_t err_node = nullptr;
  hipGraphExecUpdateResult result = hipGraphExecUpdateError;
  const hipError_t e = hipGraphExecUpdate(exec_, g2, &err_node, &result);
  if (e == hipSuccess && result == hipGraphExecUpdateSuccess) {
    (void)hipGraphDestroy(graph_);
    graph_ = g2;
    return true;
  }
  (void)hipGetLastError();
  (void)hipGraphExecDestroy(exec_);
  exec_ = nullptr;
  (void)hipGraphDestroy(graph_);
  graph_ = g2;
  const auto t0 = clock::now();
  GIE_HIP_CHECK(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0));
  instantiate_us_ = us_since(t0);
  size_t n = 0;
  GIE_HIP_CHECK(hipGraphGetNodes(graph_, nullptr, &n));
  nodes_ = n;
  return false;
}

void HipGraphExecutor::launch(hipStream_t stream) const {
  RoctxRange range("gie::HipGraphExecutor::launch");
  GIE_REQUIRE(exec_ != nullptr, StatusCode::kInvalidArgument, "HipGraphExecutor::launch before capture()");
  GIE_HIP_CHECK(hipGraphLaunch(exec_, stream));
}

}  // namespace gie
