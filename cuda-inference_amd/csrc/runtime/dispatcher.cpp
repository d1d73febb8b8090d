// Dispatcher: which registered kernel runs a problem (the behaviour of src/runtime/dispatcher.cpp:23-105).
//
// Selection is a fixed chain of rules, each of which either decides or passes to the next:
//   1. a kernel named in the options (it must exist, belong to the forced backend if one is given, and support
//      the problem; otherwise the call fails rather than silently running something else);
//   2. the CPU reference is never a GPU choice;
//   3. the capability filter leaves at least one candidate, or the call fails listing every rejected kernel with
//      its reason, one "- name: reason" line each;
//   4. a tuning-cache entry whose kernel is still among the candidates;
//   5. a fresh autotune when the options ask for one;
//   6. the best candidate under the cost model.
#include "gpu_inference/dispatcher.h"

#include <algorithm>
#include <string>

#include "gpu_inference/autotuner.h"
#include "gpu_inference/perf_model.h"
#include "gpu_inference/roctx.h"

namespace gie {
namespace {

Selection chosen(const KernelDesc* k, SelectionSource src, double us, const char* reason) {
  Selection s;
  s.kernel = k;
  s.source = src;
  s.predicted_us = us;
  s.reason = reason;
  return s;
}

Selection forced_kernel(const ConvProblem& prob, const DeviceInfo& dev, const Conv2DOptions& opt) {
  const KernelDesc* k = find_kernel(opt.kernel);
  if (k == nullptr) throw Error(StatusCode::kInvalidArgument, "no registered kernel is named '" + opt.kernel + "'");
  if (opt.backend != Backend::kAuto && k->backend != opt.backend)
    throw Error(StatusCode::kInvalidArgument, "kernel '" + opt.kernel + "' is a " + to_string(k->backend) +
                                                  " kernel; the options force backend " + to_string(opt.backend));
  std::string why;
  if (!k->supports(prob, dev, &why)) throw Error(StatusCode::kUnsupported, k->name + " cannot run this problem: " + why);
  return chosen(k, SelectionSource::kForcedKernel, 0.0, "kernel named in the options");
}

[[noreturn]] void nothing_runs(const ConvProblem& prob, const DeviceInfo& dev, Backend backend,
                               const std::vector<Rejection>& rejected) {
  std::string msg = "no " + std::string(backend == Backend::kAuto ? "" : to_string(backend)) +
                    (backend == Backend::kAuto ? "" : " ") + "kernel runs " + prob.key() + " on " + dev.name + " (" +
                    dev.gcn_arch + ")";
  if (rejected.empty()) msg += ": the " + std::string(to_string(backend)) + " backend has no registered kernels";
  for (const Rejection& r : rejected) msg += "\n  - " + r.kernel + ": " + r.reason;
  throw Error(StatusCode::kUnsupported, msg);
}

bool contains(const std::vector<const KernelDesc*>& v, const KernelDesc* k) {
  return std::find(v.begin(), v.end(), k) != v.end();
}

}  // namespace

const char* to_string(SelectionSource s) {
  switch (s) {
    case SelectionSource::kForcedKernel: return "forced_kernel";
    case SelectionSource::kForcedBackend: return "forced_backend";
    case SelectionSource::kTuningCache: return "tuning_cache";
    case SelectionSource::kTuned: return "tuned";
    case SelectionSource::kCostModel: return "cost_model";
  }
  return "?";
}

std::vector<const KernelDesc*> Dispatcher::compatible_kernels(const ConvProblem& prob, const DeviceInfo& dev,
                                                              Backend only, std::vector<Rejection>* rejected) {
  std::vector<const KernelDesc*> accepted;
  std::string why;
  for (const KernelDesc& k : kernel_registry()) {
    if (only != Backend::kAuto && k.backend != only) continue;
    why.clear();
    if (k.supports(prob, dev, &why))
      accepted.push_back(&k);
    else if (rejected != nullptr)
      rejected->push_back({k.name, why.empty() ? std::string("unsupported") : why});
  }
  return accepted;
}

std::vector<std::pair<const KernelDesc*, double>> Dispatcher::rank_by_model(const ConvProblem& prob,
                                                                             const DeviceInfo& dev,
                                                                             const std::vector<const KernelDesc*>& cands) {
  DeviceCeilings ceil;
  if (!load_cached_ceilings(dev.device, &ceil)) ceil = theoretical_ceilings(dev);
  std::vector<std::pair<const KernelDesc*, double>> order;
  order.reserve(cands.size());
  for (const KernelDesc* k : cands) order.emplace_back(k, estimate_kernel(prob, *k, dev, ceil).time_us);
  // stable: equal estimates keep registry order, so the ranking is deterministic
  std::stable_sort(order.begin(), order.end(),
                   [](const std::pair<const KernelDesc*, double>& a, const std::pair<const KernelDesc*, double>& b) {
                     return a.second < b.second;
                   });
  return order;
}

Selection Dispatcher::select(const ConvProblem& prob, const DeviceInfo& dev, const Conv2DOptions& opt) {
  RoctxRange range("gie::Dispatcher::select");
  validate_problem(prob);
  if (!opt.kernel.empty()) return forced_kernel(prob, dev, opt);
  if (opt.backend == Backend::kCpuReference)
    throw Error(StatusCode::kUnsupported,
                "cpu_reference is a host routine (cpu_conv2d_reference on host buffers), not a GPU backend");

  std::vector<Rejection> rejected;
  const std::vector<const KernelDesc*> cands = compatible_kernels(prob, dev, opt.backend, &rejected);
  if (cands.empty()) nothing_runs(prob, dev, opt.backend, rejected);

  if (!opt.force_retune) {
    std::string name;
    double us = 0;
    if (TuneCache(opt.cache_path).lookup(prob, dev, &name, &us, nullptr, opt.backend)) {
      const KernelDesc* k = find_kernel(name);
      if (k != nullptr && contains(cands, k))
        return chosen(k, SelectionSource::kTuningCache, us, "fastest measured kernel, from the tuning cache");
    }
  }
  if (opt.autotune || opt.force_retune) {
    TuneOptions to;
    to.only_backend = opt.backend;
    to.cache_path = opt.cache_path;
    to.force_retune = opt.force_retune;
    const TuneResult r = Autotuner::tune(prob, dev, to);
    return chosen(find_kernel(r.best_kernel), SelectionSource::kTuned, r.best_us, "fastest measured kernel, tuned now");
  }
  const auto ranked = rank_by_model(prob, dev, cands);
  return chosen(ranked.front().first,
                opt.backend == Backend::kAuto ? SelectionSource::kCostModel : SelectionSource::kForcedBackend,
                ranked.front().second, "lowest cost-model estimate (nothing measured for this problem)");
}

}  // namespace gie
