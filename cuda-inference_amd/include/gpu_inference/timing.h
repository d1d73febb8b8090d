// HIP-event timing with robust summary statistics (the reference's include/gpu_inference/timing.h).
#pragma once

#include <hip/hip_runtime_api.h>

#include <functional>
#include <vector>

namespace gie {

struct TimingStats {
  int samples = 0;
  int inner_iters = 1;
  double median_us = 0, mean_us = 0, min_us = 0, max_us = 0;
  double p10_us = 0, p90_us = 0, p99_us = 0;
  double stddev_us = 0;
  double iqr_us = 0;
  std::vector<double> raw_us;  // per-sample (per-launch average) latency
};

struct TimingOptions {
  int warmup_iters = 5;
  int samples = 20;
  // Each sample times `inner` back-to-back launches between one event pair; inner <= 0 picks it so a sample
  // lasts at least min_sample_ms.
  int inner = 0;
  double min_sample_ms = 1.0;
  int max_inner = 4096;
  // Cold-cache protocol: flush_bytes > 0 -> each sample is one launch after an untimed fill of flush_buffer.
  void* flush_buffer = nullptr;
  size_t flush_bytes = 0;
};

TimingStats time_stream_work(const std::function<void(hipStream_t)>& launch, hipStream_t stream,
                             const TimingOptions& opt = {});
TimingStats summarize(std::vector<double> per_launch_us, int inner);

}  // namespace gie
