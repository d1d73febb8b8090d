// Stream timing with HIP events (the role of src/runtime/timing.cpp:42-83).
//
// Steady-state protocol: after the warm-up launches, `samples` batches of `inner` launches are enqueued back to
// back with one event between consecutive batches (samples + 1 events), and the host synchronizes once at the end;
// sample i is the time between events i and i + 1 divided by `inner`. The GPU never idles between samples waiting
// for the host, so the samples measure the stream as a serving loop drives it. `inner` <= 0 is chosen from a
// four-launch probe so that one sample lasts at least min_sample_ms.
// Cold-cache protocol (flush_bytes > 0): each sample is one launch between its own event pair, preceded by an
// untimed copy over flush_bytes of device memory, which evicts the working set from L2 and the Infinity Cache.
// Statistics: order statistics with linear interpolation between closest ranks.
#include "gpu_inference/timing.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <numeric>
#include <vector>

#include "gie_hip.h"
#include "gpu_inference/error.h"

namespace gie {
namespace {

// q-quantile of ascending `v` (0 <= q <= 1), interpolating linearly between the two closest ranks.
double quantile(const std::vector<double>& v, double q) {
  if (v.empty()) return 0;
  const double rank = q * double(v.size() - 1);
  const size_t below = size_t(rank);
  const size_t above = std::min(below + 1, v.size() - 1);
  return v[below] + (v[above] - v[below]) * (rank - double(below));
}

class EventSet {
 public:
  explicit EventSet(size_t n) : ev_(n, nullptr) {
    for (hipEvent_t& e : ev_) GIE_HIP_CHECK(hipEventCreate(&e));
  }
  ~EventSet() {
    for (hipEvent_t e : ev_)
      if (e) (void)hipEventDestroy(e);
  }
  EventSet(const EventSet&) = delete;
  EventSet& operator=(const EventSet&) = delete;
  hipEvent_t operator[](size_t i) const { return ev_[i]; }
  double ms_between(size_t a, size_t b) const {
    float ms = 0;
    GIE_HIP_CHECK(hipEventElapsedTime(&ms, ev_[a], ev_[b]));
    return double(ms);
  }

 private:
  std::vector<hipEvent_t> ev_;
};

}  // namespace

TimingStats summarize(std::vector<double> per_launch_us, int inner) {
  TimingStats t;
  t.inner_iters = inner;
  t.samples = int(per_launch_us.size());
  t.raw_us = per_launch_us;
  if (per_launch_us.empty()) return t;
  std::vector<double>& v = per_launch_us;
  std::sort(v.begin(), v.end());
  t.min_us = v.front();
  t.max_us = v.back();
  t.median_us = quantile(v, 0.50);
  t.p10_us = quantile(v, 0.10);
  t.p90_us = quantile(v, 0.90);
  t.p99_us = quantile(v, 0.99);
  t.iqr_us = quantile(v, 0.75) - quantile(v, 0.25);
  t.mean_us = std::accumulate(v.begin(), v.end(), 0.0) / double(v.size());
  if (v.size() > 1) {
    double sq = 0;
    for (double x : v) sq += (x - t.mean_us) * (x - t.mean_us);
    t.stddev_us = std::sqrt(sq / double(v.size() - 1));  // sample standard deviation
  }
  return t;
}

TimingStats time_stream_work(const std::function<void(hipStream_t)>& launch, hipStream_t stream,
                             const TimingOptions& opt) {
  const int samples = std::max(opt.samples, 1);
  for (int i = 0; i < opt.warmup_iters; ++i) launch(stream);

  if (opt.flush_bytes > 0 && opt.flush_buffer != nullptr) {
    const size_t half = (opt.flush_bytes / 2) & ~size_t(15);
    EventSet ev(2 * size_t(samples));
    for (int s = 0; s < samples; ++s) {
      check_kernel_status(
          gie_hip_ceiling_copy(opt.flush_buffer, static_cast<char*>(opt.flush_buffer) + half, half, stream),
          "cache flush");
      GIE_HIP_CHECK(hipEventRecord(ev[2 * size_t(s)], stream));
      launch(stream);
      GIE_HIP_CHECK(hipEventRecord(ev[2 * size_t(s) + 1], stream));
    }
    GIE_HIP_CHECK(hipEventSynchronize(ev[2 * size_t(samples) - 1]));
    std::vector<double> us(static_cast<size_t>(samples));
    for (int s = 0; s < samples; ++s) us[size_t(s)] = 1000.0 * ev.ms_between(2 * size_t(s), 2 * size_t(s) + 1);
    return summarize(std::move(us), 1);
  }

  int inner = opt.inner;
  if (inner <= 0) {
    EventSet probe(2);
    GIE_HIP_CHECK(hipEventRecord(probe[0], stream));
    for (int i = 0; i < 4; ++i) launch(stream);
    GIE_HIP_CHECK(hipEventRecord(probe[1], stream));
    GIE_HIP_CHECK(hipEventSynchronize(probe[1]));
    const double per_launch_ms = std::max(probe.ms_between(0, 1) / 4.0, 1e-4);
    inner = int(std::clamp(std::ceil(opt.min_sample_ms / per_launch_ms), 1.0, double(std::max(opt.max_inner, 1))));
  }
  EventSet ev(size_t(samples) + 1);
  GIE_HIP_CHECK(hipEventRecord(ev[0], stream));
  for (int s = 0; s < samples; ++s) {
    for (int i = 0; i < inner; ++i) launch(stream);
    GIE_HIP_CHECK(hipEventRecord(ev[size_t(s) + 1], stream));
  }
  GIE_HIP_CHECK(hipEventSynchronize(ev[size_t(samples)]));
  std::vector<double> us(static_cast<size_t>(samples));
  for (int s = 0; s < samples; ++s) us[size_t(s)] = 1000.0 * ev.ms_between(size_t(s), size_t(s) + 1) / inner;
  return summarize(std::move(us), inner);
}

}  // namespace gie
