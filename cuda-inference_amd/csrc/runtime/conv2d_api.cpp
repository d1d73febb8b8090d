// Conv2D::forward / workspace_size / clear_plan_cache: the public entry points of src/runtime/conv2d.cpp:113-164,
// over a process-wide plan table.
//
// Design (a serving loop calls forward on the same few problems millions of times):
//   * the table key is a fixed-size binary record (geometry, precision, epilogue, device, option flags and 64-bit
//     hashes of the forced kernel name and cache path); nothing is formatted into a string to find a plan. The
//     two strings are kept beside the record and compared on a hit, so a hash collision cannot alias two plans;
//   * each thread remembers the last (record, plan) it used together with the table generation it saw, so a loop
//     over one problem costs one 112-byte compare and no lock; clear_plan_cache() bumps the generation;
//   * a record only enters the table after its problem passed validate_problem(), and validity is a function of
//     the record alone, so a hit skips validation;
//   * on a miss the kernel is selected and the plan built without holding the table lock (selection may
//     autotune for seconds); if two threads race, the first plan inserted is the one every caller gets.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstring>
#include <memory>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <unordered_map>

#include "gpu_inference/conv2d.h"
#include "gpu_inference/dispatcher.h"
#include "gpu_inference/execution_plan.h"

namespace gie {
namespace {

uint64_t hash_bytes(const void* data, size_t n, uint64_t h = 0xcbf29ce484222325ULL) {
  const auto* b = static_cast<const unsigned char*>(data);
  for (size_t i = 0; i < n; ++i) h = (h ^ b[i]) * 0x100000001b3ULL;  // FNV-1a, 64-bit
  return h;
}

// 24 x 4-byte fields then two 8-byte hashes: no padding, so the bytes define equality and the hash.
struct PlanRecord {
  int32_t f[24];
  uint64_t kernel_hash;
  uint64_t cache_hash;

  bool operator==(const PlanRecord& o) const { return std::memcmp(this, &o, sizeof(*this)) == 0; }
};
static_assert(sizeof(PlanRecord) == 112, "PlanRecord must have no padding");

PlanRecord make_record(const ConvProblem& prob, const Conv2DOptions& opt, int device) {
  PlanRecord r;
  std::memset(&r, 0, sizeof(r));
  const Conv2DParams& p = prob.p;
  const int32_t v[] = {p.batch,      p.in_channels, p.in_h,       p.in_w,       p.out_channels,
                       p.kernel_h,   p.kernel_w,    p.stride_h,   p.stride_w,   p.pad_h,
                       p.pad_w,      p.dilation_h,  p.dilation_w, p.groups,     int32_t(prob.precision),
                       int32_t(prob.has_bias),      int32_t(prob.activation), int32_t(opt.backend),
                       device,       int32_t(opt.autotune) | int32_t(opt.force_retune) << 1,
                       int32_t(opt.kernel.size()), int32_t(opt.cache_path.size())};
  static_assert(sizeof(v) / sizeof(v[0]) <= 24, "PlanRecord field count");
  std::memcpy(r.f, v, sizeof(v));
  r.kernel_hash = hash_bytes(opt.kernel.data(), opt.kernel.size());
  r.cache_hash = hash_bytes(opt.cache_path.data(), opt.cache_path.size());
  return r;
}

struct RecordHash {
  size_t operator()(const PlanRecord& r) const { return size_t(hash_bytes(&r, sizeof(r))); }
};

struct Slot {
  std::string kernel, cache;  // the hashed strings, compared on every hit
  std::shared_ptr<ExecutionPlan> plan;
};

struct PlanTable {
  std::shared_mutex mu;
  std::unordered_multimap<PlanRecord, Slot, RecordHash> slots;
  std::atomic<uint64_t> generation{1};
};

PlanTable& table() {
  static PlanTable t;
  return t;
}

// The thread's last lookup. It holds its plan weakly: once clear_plan_cache() drops the table's reference, a thread
// that never calls again does not keep the plan (and the device memory it owns) alive.
struct LastPlan {
  uint64_t generation = 0;
  PlanRecord record{};
  std::string kernel, cache;
  std::weak_ptr<ExecutionPlan> plan;
};
thread_local LastPlan t_last;

bool same_strings(const std::string& k, const std::string& c, const Conv2DOptions& opt) {
  return k == opt.kernel && c == opt.cache_path;
}

std::shared_ptr<ExecutionPlan> find_in_table(PlanTable& t, const PlanRecord& rec, const Conv2DOptions& opt) {
  std::shared_lock<std::shared_mutex> lock(t.mu);
  const auto range = t.slots.equal_range(rec);
  for (auto it = range.first; it != range.second; ++it)
    if (same_strings(it->second.kernel, it->second.cache, opt)) return it->second.plan;
  return nullptr;
}

std::shared_ptr<ExecutionPlan> plan_for(const ConvProblem& prob, const Conv2DOptions& opt) {
  int device = 0;
  GIE_HIP_CHECK(hipGetDevice(&device));
  const PlanRecord rec = make_record(prob, opt, device);
  PlanTable& t = table();
  const uint64_t gen = t.generation.load(std::memory_order_acquire);
  LastPlan& last = t_last;
  if (last.generation == gen && last.record == rec && same_strings(last.kernel, last.cache, opt)) {
    if (std::shared_ptr<ExecutionPlan> hit = last.plan.lock()) return hit;
  }

  std::shared_ptr<ExecutionPlan> plan = find_in_table(t, rec, opt);
  if (!plan) {
    validate_problem(prob);
    const Selection sel = Dispatcher::select(prob, DeviceInfo::get(device), opt);
    std::shared_ptr<ExecutionPlan> built = ExecutionPlan::create(prob, *sel.kernel, device);
    std::unique_lock<std::shared_mutex> lock(t.mu);
    const auto range = t.slots.equal_range(rec);
    for (auto it = range.first; it != range.second && !plan; ++it)
      if (same_strings(it->second.kernel, it->second.cache, opt)) plan = it->second.plan;  // another thread won
    if (!plan) {
      plan = std::move(built);
      // a clear_plan_cache() that ran while this plan was being built empties the table for good: the plan then
      // serves this call only and is neither inserted nor remembered
      if (t.generation.load(std::memory_order_acquire) != gen) return plan;
      t.slots.emplace(rec, Slot{opt.kernel, opt.cache_path, plan});
    }
  }
  last.generation = gen;
  last.record = rec;
  last.kernel = opt.kernel;
  last.cache = opt.cache_path;
  last.plan = plan;
  return plan;
}

}  // namespace

void Conv2D::forward(const ConstTensorRef& input, const ConstTensorRef& weights, const ConstTensorRef* bias,
                     const ConvProblem& problem, const TensorRef& output, void* workspace, size_t workspace_bytes,
                     hipStream_t stream, const Conv2DOptions& options) {
  plan_for(problem, options)->execute(input, weights, bias, output, workspace, workspace_bytes, stream);
}

size_t Conv2D::workspace_size(const ConvProblem& problem, const Conv2DOptions& options) {
  return plan_for(problem, options)->workspace_bytes();
}

void Conv2D::clear_plan_cache() {
  PlanTable& t = table();
  std::unique_lock<std::shared_mutex> lock(t.mu);
  t.slots.clear();
  t.generation.fetch_add(1, std::memory_order_acq_rel);
}

}  // namespace gie
