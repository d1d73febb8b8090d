// Kernel autotuner and persistent tuning cache (the reference's include/gpu_inference/autotuner.h).
//
// Per workload: enumerate registered kernels -> capability filter -> (optional) cost-model pruning ->
// validation against the GPU double-precision reference -> warmup -> event timing -> median -> persist winner.
// A candidate that fails validation or errors out is never selected.
#pragma once

#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "gpu_inference/dispatcher.h"
#include "gpu_inference/timing.h"

namespace gie {

struct TuneOptions {
  TimingOptions timing;
  uint64_t seed = 0x5eed1234abcdULL;
  bool validate = true;
  Backend only_backend = Backend::kAuto;
  int model_keep = 0;        // >0: keep only the N best candidates per the cost model
  int max_candidates = 128;
  bool use_cache = true;
  bool force_retune = false;
  std::string cache_path;    // empty -> TuneCache::default_path()
  bool verbose = false;
};

struct CandidateResult {
  std::string kernel;
  Backend backend = Backend::kDirect;
  bool measured = false;
  std::string status;  // "ok", "rejected: ...", "failed validation: ...", "error: ..."
  double predicted_us = 0;
  TimingStats timing;
  double max_abs_err = 0, frac_over_tol = 0;
};

struct TuneResult {
  ConvProblem problem;
  std::string best_kernel;
  double best_us = 0;
  bool from_cache = false;
  double search_seconds = 0;
  int candidates_total = 0;
  int candidates_measured = 0;
  std::vector<CandidateResult> candidates;
};

// JSON cache keyed by GPU arch / CU count / HIP runtime + driver / library version / source fingerprint /
// problem. Stale or mismatching entries are ignored.
class TuneCache {
 public:
  static std::string default_path();  // $GIE_TUNE_CACHE or ~/.cache/gpu_inference/tune_cache.json
  explicit TuneCache(std::string path = "");
  static std::string make_key(const ConvProblem& prob, const DeviceInfo& dev, Backend scope = Backend::kAuto);

  bool lookup(const ConvProblem& prob, const DeviceInfo& dev, std::string* kernel, double* us,
              double* tuned_seconds = nullptr, Backend scope = Backend::kAuto) const;
  void store(const TuneResult& r, const DeviceInfo& dev, Backend scope = Backend::kAuto);
  void clear();
  size_t size() const;
  const std::string& path() const { return path_; }

  // one persisted winner (the file's per-key record)
  struct Entry {
    std::string kernel;
    int kernel_version = 0;
    double us = 0;
    double tuned_seconds = 0;
    std::string timestamp;
  };

 private:
  void load_locked() const;
  void save_locked() const;
  std::string path_;
  mutable std::mutex mu_;
  mutable std::map<std::string, Entry> entries_;
  mutable std::string text_;  // file contents entries_ was parsed from
  mutable bool loaded_ = false;
};

class Autotuner {
 public:
  static TuneResult tune(const ConvProblem& prob, const DeviceInfo& dev, const TuneOptions& opt = {});
};

}  // namespace gie
