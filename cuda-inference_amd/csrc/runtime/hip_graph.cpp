// HipGraphExecutor (the role of src/runtime/cuda_graph.cpp:13-97): record a chain of asynchronous launches once as
// a HIP graph and replay it with one hipGraphLaunch, which removes the per-launch host cost and the gaps between
// small kernels.
//
// Recording happens on a private non-blocking stream in thread-local capture mode, so work other threads enqueue
// meanwhile is neither captured nor made illegal. The enqueue function runs once eagerly before the first recording:
// one-time work it may trigger (function attributes, lazy module loads) is not legal inside a capture. If the
// enqueue function throws mid-recording, the capture is ended and its partial graph discarded before the exception
// leaves. recapture_update() records again and first tries to patch the executable graph in place (same topology,
// new kernel arguments such as buffer addresses); only when HIP refuses is the graph instantiated afresh.
#include "gpu_inference/hip_graph.h"

#include <hip/hip_runtime.h>

#include <chrono>

#include "gpu_inference/roctx.h"

namespace gie {
namespace {

double micros_since(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
}

class PrivateStream {
 public:
  PrivateStream() { GIE_HIP_CHECK(hipStreamCreateWithFlags(&s_, hipStreamNonBlocking)); }
  ~PrivateStream() { (void)hipStreamDestroy(s_); }
  PrivateStream(const PrivateStream&) = delete;
  PrivateStream& operator=(const PrivateStream&) = delete;
  hipStream_t get() const { return s_; }

 private:
  hipStream_t s_ = nullptr;
};

// Records `enqueue` into a new graph; *us receives the recording time.
hipGraph_t record(const HipGraphExecutor::Enqueue& enqueue, double* us) {
  PrivateStream stream;
  const auto t0 = std::chrono::steady_clock::now();
  GIE_HIP_CHECK(hipStreamBeginCapture(stream.get(), hipStreamCaptureModeThreadLocal));
  try {
    enqueue(stream.get());
  } catch (...) {
    hipGraph_t partial = nullptr;
    (void)hipStreamEndCapture(stream.get(), &partial);
    if (partial != nullptr) (void)hipGraphDestroy(partial);
    throw;
  }
  hipGraph_t g = nullptr;
  GIE_HIP_CHECK(hipStreamEndCapture(stream.get(), &g));
  *us = micros_since(t0);
  return g;
}

}  // namespace

HipGraphExecutor::~HipGraphExecutor() { reset(); }

void HipGraphExecutor::reset() {
  if (exec_ != nullptr) (void)hipGraphExecDestroy(exec_);
  if (graph_ != nullptr) (void)hipGraphDestroy(graph_);
  exec_ = nullptr;
  graph_ = nullptr;
  nodes_ = 0;
}

void HipGraphExecutor::adopt(hipGraph_t g, double capture_us) {
  reset();
  graph_ = g;
  capture_us_ = capture_us;
  const auto t0 = std::chrono::steady_clock::now();
  GIE_HIP_CHECK(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0));
  instantiate_us_ = micros_since(t0);
  size_t n = 0;
  GIE_HIP_CHECK(hipGraphGetNodes(graph_, nullptr, &n));
  nodes_ = n;
}

void HipGraphExecutor::capture(const Enqueue& enqueue) {
  RoctxRange range("gie::HipGraphExecutor::capture");
  {
    PrivateStream warm;
    enqueue(warm.get());
    GIE_HIP_CHECK(hipStreamSynchronize(warm.get()));
  }
  double us = 0;
  hipGraph_t g = record(enqueue, &us);  // recorded before `us` is read (argument order is unspecified)
  adopt(g, us);
}

bool HipGraphExecutor::recapture_update(const Enqueue& enqueue) {
  RoctxRange range("gie::HipGraphExecutor::recapture_update");
  if (exec_ == nullptr) {
    capture(enqueue);
    return false;
  }
  double us = 0;
  hipGraph_t fresh = record(enqueue, &us);
  hipGraphNode_t failed_node = nullptr;
  hipGraphExecUpdateResult outcome = hipGraphExecUpdateError;
  if (hipGraphExecUpdate(exec_, fresh, &failed_node, &outcome) == hipSuccess && outcome == hipGraphExecUpdateSuccess) {
    (void)hipGraphDestroy(graph_);
    graph_ = fresh;
    capture_us_ = us;
    return true;
  }
  (void)hipGetLastError();  // the refused update leaves an error code behind
  try {
    adopt(fresh, us);
  } catch (...) {
    if (graph_ != fresh) (void)hipGraphDestroy(fresh);
    throw;
  }
  return false;
}

void HipGraphExecutor::upload(hipStream_t stream) const {
  GIE_REQUIRE(exec_ != nullptr, StatusCode::kInvalidArgument, "HipGraphExecutor::upload called before capture()");
  GIE_HIP_CHECK(hipGraphUpload(exec_, stream));
}

void HipGraphExecutor::launch(hipStream_t stream) const {
  RoctxRange range("gie::HipGraphExecutor::launch");
  GIE_REQUIRE(exec_ != nullptr, StatusCode::kInvalidArgument, "HipGraphExecutor::launch called before capture()");
  GIE_HIP_CHECK(hipGraphLaunch(exec_, stream));
}

}  // namespace gie
