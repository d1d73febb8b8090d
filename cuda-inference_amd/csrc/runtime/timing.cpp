// Event timing with batched back-to-back launches (the reference's timing.cpp protocol: warmup, pick the
// inner count so a sample lasts >= min_sample_ms, median over samples).
#include "gpu_inference/timing.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <numeric>

#include "gie_hip.h"
#include "gpu_inference/error.h"

namespace gie {
namespace {

double percentile(const std::vector<double>& sorted, double q) {
  if (sorted.empty()) return 0;
  const double pos = q * double(sorted.size() - 1);
  const size_t lo = size_t(std::floor(pos)), hi = size_t(std::ceil(pos));
  return sorted[lo] + (sorted[hi] - sorted[lo]) * (pos - double(lo));
}

}  // namespace

TimingStats summarize(std::vector<double> v, int inner) {
  TimingStats t;
  t.inner_iters = inner;
  t.samples = int(v.size());
  t.raw_us = v;
  if (v.empty()) return t;
  std::sort(v.begin(), v.end());
  t.min_us = v.front();
  t.max_us = v.back();
  t.median_us = percentile(v, 0.5);
  t.p10_us = percentile(v, 0.10);
  t.p90_us = percentile(v, 0.90);
  t.p99_us = percentile(v, 0.99);
  t.iqr_us = percentile(v, 0.75) - percentile(v, 0.25);
  t.mean_us = std::accumulate(v.begin(), v.end(), 0.0) / double(v.size());
  double ss = 0;
  for (double x : v) ss += (x - t.mean_us) * (x - t.mean_us);
  t.stddev_us = v.size() > 1 ? std::sqrt(ss / double(v.size() - 1)) : 0;
  return t;
}

TimingStats time_stream_work(const std::function<void(hipStream_t)>& launch, hipStream_t stream,
                             const TimingOptions& opt) {
  hipEvent_t start, stop;
  GIE_HIP_CHECK(hipEventCreate(&start));
  GIE_HIP_CHECK(hipEventCreate(&stop));
  struct Guard {
    hipEvent_t a, b;
    ~Guard() {
      (void)hipEventDestroy(a);
      (void)hipEventDestroy(b);
    }
  } guard{start, stop};

  auto time_batch = [&](int n) {
    GIE_HIP_CHECK(hipEventRecord(start, stream));
    for (int i = 0; i < n; ++i) launch(stream);
    GIE_HIP_CHECK(hipEventRecord(stop, stream));
    GIE_HIP_CHECK(hipEventSynchronize(stop));
    float ms = 0;
    GIE_HIP_CHECK(hipEventElapsedTime(&ms, start, stop));
    return double(ms);
  };

  for (int i = 0; i < opt.warmup_iters; ++i) launch(stream);
  GIE_HIP_CHECK(hipStreamSynchronize(stream));

  int inner = opt.inner;
  if (opt.flush_bytes > 0) inner = 1;
  if (inner <= 0) {
    const double probe_ms = std::max(time_batch(4) / 4.0, 1e-4);
    inner = int(std::clamp(std::ceil(opt.min_sample_ms / probe_ms), 1.0, double(opt.max_inner)));
  }

  std::vector<double> us;
  us.reserve(size_t(opt.samples));
  if (opt.flush_bytes > 0 && opt.flush_buffer != nullptr) {
    for (int s = 0; s < opt.samples; ++s) {
      // untimed overwrite of a buffer larger than the L2 + MALL evicts inputs and weights
      check_kernel_status(gie_hip_ceiling_copy(opt.flush_buffer, static_cast<char*>(opt.flush_buffer) +
                                                                     (opt.flush_bytes / 2 / 16) * 16,
                                               (opt.flush_bytes / 2 / 16) * 16, stream),
                          "cache flush");
      us.push_back(time_batch(1) * 1000.0);
    }
    return summarize(std::move(us), 1);
  }
  for (int s = 0; s < opt.samples; ++s) us.push_back(time_batch(inner) * 1000.0 / inner);
  return summarize(std::move(us), inner);
}

}  // namespace gie
