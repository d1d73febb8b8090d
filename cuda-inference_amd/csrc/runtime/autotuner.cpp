// Autotuner (the role of src/autotuner/autotuner.cpp:15-140): measure the registered kernels that can run a problem
// and keep the fastest correct one.
//
// A fused-conv problem here has up to a few dozen capable entries (several kernel families x tile shapes x split-K
// factors), so the search runs in passes over one shared set of seeded inputs:
//   1. capability filter (rejections are recorded with their reasons), cost-model order, optional pruning to the
//      model's best model_keep / max_candidates;
//   2. correctness: one launch per candidate on a NaN-poisoned output, compared with the GPU double reference
//      under the problem's tolerance; a candidate that fails or throws is out for good;
//   3. screening: every correct candidate is timed with a short protocol (a third of the samples);
//   4. final: the candidates within 15 % of the best screening median (at least three) are timed with the full
//      protocol and the lowest median wins. With three or fewer correct candidates the screening pass is skipped.
// The winner is written to the tuning cache. One workspace, sized for the largest candidate, serves every launch.
#include "gpu_inference/autotuner.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <iostream>
#include <memory>

#include "gpu_inference/execution_plan.h"
#include "gpu_inference/perf_model.h"
#include "gpu_inference/reference.h"
#include "gpu_inference/roctx.h"
#include "gpu_inference/testing.h"

namespace gie {
namespace {

constexpr double kFinalistBand = 1.15;  // screening medians within this factor of the best go to the final pass
constexpr int kMinFinalists = 3;

struct StreamOwner {
  hipStream_t s = nullptr;
  StreamOwner() { GIE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)); }
  ~StreamOwner() { (void)hipStreamDestroy(s); }
};

struct DeviceScope {
  int saved = 0;
  explicit DeviceScope(int device) {
    GIE_HIP_CHECK(hipGetDevice(&saved));
    if (saved != device) GIE_HIP_CHECK(hipSetDevice(device));
  }
  ~DeviceScope() { (void)hipSetDevice(saved); }
};

// A candidate under measurement: its plan (null once it has failed) and its result record.
struct Trial {
  const KernelDesc* kernel = nullptr;
  std::shared_ptr<ExecutionPlan> plan;
  CandidateResult result;
};

// The seeded inputs, the reference output and a workspace shared by every trial.
class Bench {
 public:
  Bench(const ConvProblem& prob, const TuneOptions& opt)
      : prob_(prob), opt_(opt), data_(make_conv_data(prob, opt.seed, Distribution::kUniform)),
        n_out_(prob.p.output_shape().numel()) {
    if (opt.validate) {
      DeviceBuffer ref(size_t(n_out_) * 4), scale(size_t(n_out_) * 4);
      gpu_conv2d_reference(prob, data_.dx.data(), data_.dw.data(), data_.db.data(), static_cast<float*>(ref.data()),
                           static_cast<float*>(scale.data()), stream_.s);
      GIE_HIP_CHECK(hipStreamSynchronize(stream_.s));
      ref_.resize(size_t(n_out_));
      scale_.resize(size_t(n_out_));
      GIE_HIP_CHECK(hipMemcpy(ref_.data(), ref.data(), size_t(n_out_) * 4, hipMemcpyDeviceToHost));
      GIE_HIP_CHECK(hipMemcpy(scale_.data(), scale.data(), size_t(n_out_) * 4, hipMemcpyDeviceToHost));
    }
  }

  void reserve_workspace(size_t bytes) {
    if (bytes > ws_.size()) ws_ = DeviceBuffer(bytes);
  }

  void launch(const ExecutionPlan& plan, hipStream_t s) {
    plan.execute_unchecked(data_.dx.data(), data_.dw.data(), prob_.has_bias ? data_.db.data() : nullptr,
                           data_.dy.data(), ws_.data(), ws_.size(), s);
  }

  // One launch on a poisoned output; false, with the reason in cr->status, when the result is out of tolerance.
  bool check(const ExecutionPlan& plan, CandidateResult* cr) {
    GIE_HIP_CHECK(hipMemsetAsync(data_.dy.data(), 0xFF, data_.dy.size(), stream_.s));
    launch(plan, stream_.s);
    GIE_HIP_CHECK(hipStreamSynchronize(stream_.s));
    GIE_HIP_CHECK(hipGetLastError());
    if (!opt_.validate) return true;
    const std::vector<float> out = download_as_float(data_.dy.data(), prob_.dtype(), n_out_);
    const ErrorMetrics m = compare_outputs(out.data(), ref_.data(), scale_.data(), n_out_,
                                           TolerancePolicy::for_problem(prob_, false));
    cr->max_abs_err = m.max_abs;
    cr->frac_over_tol = m.frac_over_tol;
    if (m.passed()) return true;
    cr->status = "failed validation: " + m.summary();
    return false;
  }

  TimingStats time(const ExecutionPlan& plan, const TimingOptions& t) {
    return time_stream_work([&](hipStream_t s) { launch(plan, s); }, stream_.s, t);
  }

  void recover() {
    (void)hipStreamSynchronize(stream_.s);
    (void)hipGetLastError();
  }

 private:
  const ConvProblem& prob_;
  const TuneOptions& opt_;
  StreamOwner stream_;
  ConvData data_;
  int64_t n_out_;
  std::vector<float> ref_, scale_;
  DeviceBuffer ws_;
};

void say(const TuneOptions& opt, const ConvProblem& prob, const CandidateResult& cr, const char* pass) {
  if (!opt.verbose) return;
  std::cerr << "[tune] " << prob.key() << " " << cr.kernel << ": " << cr.status;
  if (cr.measured) std::cerr << " " << cr.timing.median_us << " us (" << pass << ")";
  std::cerr << "\n";
}

}  // namespace

TuneResult Autotuner::tune(const ConvProblem& prob, const DeviceInfo& dev, const TuneOptions& opt) {
  RoctxRange range("gie::Autotuner::tune");
  const auto started = std::chrono::steady_clock::now();
  validate_problem(prob);
  TuneResult res;
  res.problem = prob;

  TuneCache cache(opt.cache_path);
  if (opt.use_cache && !opt.force_retune) {
    std::string name;
    double us = 0, seconds = 0;
    if (cache.lookup(prob, dev, &name, &us, &seconds, opt.only_backend) && find_kernel(name) != nullptr) {
      res.best_kernel = name;
      res.best_us = us;
      res.from_cache = true;
      res.search_seconds = seconds;
      return res;
    }
  }

  DeviceScope scope(dev.device);
  std::vector<Rejection> rejected;
  const std::vector<const KernelDesc*> capable = Dispatcher::compatible_kernels(prob, dev, opt.only_backend, &rejected);
  for (const Rejection& r : rejected) {
    CandidateResult cr;
    cr.kernel = r.kernel;
    cr.status = "rejected: " + r.reason;
    res.candidates.push_back(std::move(cr));
  }
  res.candidates_total = int(capable.size());
  if (capable.empty()) throw Error(StatusCode::kUnsupported, "autotune: no registered kernel runs " + prob.key());

  auto order = Dispatcher::rank_by_model(prob, dev, capable);
  size_t keep = order.size();
  if (opt.model_keep > 0) keep = std::min(keep, size_t(opt.model_keep));
  keep = std::min(keep, size_t(std::max(opt.max_candidates, 1)));
  order.resize(keep);

  Bench bench(prob, opt);
  std::vector<Trial> trials(order.size());
  for (size_t i = 0; i < order.size(); ++i) {
    Trial& t = trials[i];
    t.kernel = order[i].first;
    t.result.kernel = t.kernel->name;
    t.result.backend = t.kernel->backend;
    t.result.predicted_us = order[i].second;
    try {
      t.plan = ExecutionPlan::create(prob, *t.kernel, dev.device);
      bench.reserve_workspace(t.plan->workspace_bytes());
    } catch (const Error& e) {
      t.plan.reset();
      t.result.status = std::string("error: ") + e.what();
    }
  }

  // pass 2: correctness
  std::vector<Trial*> alive;
  for (Trial& t : trials) {
    if (!t.plan) continue;
    try {
      if (bench.check(*t.plan, &t.result)) alive.push_back(&t);
      else t.plan.reset();
    } catch (const Error& e) {
      t.plan.reset();
      t.result.status = std::string("error: ") + e.what();
      bench.recover();
    }
  }

  // passes 3 and 4: screening, then the full protocol for the finalists
  auto measure = [&](Trial& t, const TimingOptions& to) {
    try {
      t.result.timing = bench.time(*t.plan, to);
      GIE_HIP_CHECK(hipGetLastError());
      t.result.measured = true;
      t.result.status = "ok";
      return true;
    } catch (const Error& e) {
      t.plan.reset();
      t.result.measured = false;
      t.result.status = std::string("error: ") + e.what();
      bench.recover();
      return false;
    }
  };
  std::vector<Trial*> finalists;
  if (alive.size() > size_t(kMinFinalists)) {
    TimingOptions quick = opt.timing;
    quick.samples = std::max(3, opt.timing.samples / 3);
    quick.warmup_iters = std::min(opt.timing.warmup_iters, 2);
    double best = 0;
    std::vector<Trial*> screened;
    for (Trial* t : alive) {
      if (!measure(*t, quick)) continue;
      say(opt, prob, t->result, "screening");
      screened.push_back(t);
      if (screened.size() == 1 || t->result.timing.median_us < best) best = t->result.timing.median_us;
    }
    std::stable_sort(screened.begin(), screened.end(), [](const Trial* a, const Trial* b) {
      return a->result.timing.median_us < b->result.timing.median_us;
    });
    for (size_t i = 0; i < screened.size(); ++i)
      if (i < size_t(kMinFinalists) || screened[i]->result.timing.median_us <= kFinalistBand * best)
        finalists.push_back(screened[i]);
  } else {
    finalists = alive;
  }
  const Trial* winner = nullptr;
  for (Trial* t : finalists) {
    if (!measure(*t, opt.timing)) continue;
    say(opt, prob, t->result, "final");
    if (winner == nullptr || t->result.timing.median_us < winner->result.timing.median_us) winner = t;
  }

  for (Trial& t : trials) {
    if (!t.result.measured) say(opt, prob, t.result, "");
    res.candidates.push_back(t.result);
  }
  res.candidates_measured = int(trials.size());
  if (winner == nullptr)
    throw Error(StatusCode::kUnsupported, "autotune: no candidate ran correctly for " + prob.key());
  res.best_kernel = winner->kernel->name;
  res.best_us = winner->result.timing.median_us;
  res.search_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - started).count();
  if (opt.use_cache) cache.store(res, dev, opt.only_backend);
  return res;
}

}  // namespace gie
