// Kernel registry (the reference's registry.cpp contract: unique names, mandatory function pointers, stable
// element addresses) and the gather-table builders of the registry interface (the reference's
// src/kernels/conv_common.cu:22-50 format). No kernel here reads a table — each walks the filter taps with offsets
// held in registers — so the builders serve kernels registered with needs_lut (ExecutionPlan uploads the table).
#include <cstdint>
#include <limits>
#include <set>
#include <sstream>

#include "gpu_inference/kernel_registry.h"

namespace gie {

void register_mfma_family(std::vector<KernelDesc>& out);  // mfma_family.cpp
void register_halo_family(std::vector<KernelDesc>& out);  // halo_family.cpp
void register_band_family(std::vector<KernelDesc>& out);  // band_family.cpp
void register_pw_family(std::vector<KernelDesc>& out);    // pw_family.cpp
void register_f32_family(std::vector<KernelDesc>& out);   // f32_family.cpp
void register_stem_family(std::vector<KernelDesc>& out);  // stem_family.cpp
void register_narrow_family(std::vector<KernelDesc>& out);  // narrow_family.cpp
void register_slab_family(std::vector<KernelDesc>& out);    // slab_family.cpp
void register_stack_family(std::vector<KernelDesc>& out);   // stack_family.cpp
void register_deep_family(std::vector<KernelDesc>& out);    // deep_family.cpp

std::string KernelDesc::describe() const {
  std::ostringstream os;
  os << name << " [" << to_string(backend) << ", " << threads_per_block << " thr";
  for (const auto& kv : params) os << ", " << kv.first << "=" << kv.second;
  os << "]";
  return os.str();
}

namespace {
std::vector<KernelDesc>& registry_storage() {
  static std::vector<KernelDesc> registry = [] {
    std::vector<KernelDesc> r;
    r.reserve(1024);  // stable element addresses even if tests inject extra entries
    register_band_family(r);
    register_halo_family(r);
    register_mfma_family(r);
    register_pw_family(r);  // after mfma: its unaligned-pointer fallback is an mfma entry
    register_f32_family(r);
    register_stem_family(r);  // after mfma: its unaligned-pointer fallback is an mfma entry
    register_narrow_family(r);  // likewise
    register_slab_family(r);    // likewise
    register_stack_family(r);   // likewise
    register_deep_family(r);    // likewise
    std::set<std::string> names;
    for (const auto& k : r) {
      if (!names.insert(k.name).second) throw Error(StatusCode::kInternal, "duplicate kernel name " + k.name);
      if (!k.supports || !k.launch || !k.workspace_bytes)
        throw Error(StatusCode::kInternal, "incomplete kernel descriptor " + k.name);
    }
    return r;
  }();
  return registry;
}
}  // namespace

const std::vector<KernelDesc>& kernel_registry() { return registry_storage(); }
std::vector<KernelDesc>& kernel_registry_for_testing() { return registry_storage(); }

const KernelDesc* find_kernel(const std::string& name) {
  for (const auto& k : kernel_registry())
    if (k.name == name) return &k;
  return nullptr;
}

std::vector<const KernelDesc*> kernels_for_backend(Backend b) {
  std::vector<const KernelDesc*> out;
  for (const auto& k : kernel_registry())
    if (b == Backend::kAuto || k.backend == b) out.push_back(&k);
  return out;
}

namespace {
// Offsets are 32-bit element counts: the channel displacement (C - 1) * H * W and the dilated tap extents must fit.
void check_table_range(const Conv2DParams& p) {
  const int64_t plane = int64_t(p.in_h) * p.in_w;
  const int64_t lim = std::numeric_limits<int32_t>::max();
  GIE_REQUIRE(p.in_channels > 0 && p.kernel_h > 0 && p.kernel_w > 0 && plane > 0, StatusCode::kInvalidArgument,
              "gather table of an empty problem");
  GIE_REQUIRE(int64_t(p.in_channels) * plane <= lim &&
                  int64_t(p.kernel_h) * p.dilation_h <= lim && int64_t(p.kernel_w) * p.dilation_w <= lim,
              StatusCode::kUnsupported, "gather-table offsets exceed 32 bits");
}
}  // namespace

std::vector<LutEntry> build_conv_lut(const Conv2DParams& p) {
  check_table_range(p);
  const int32_t plane = p.in_h * p.in_w;
  std::vector<LutEntry> table;
  table.reserve(size_t(p.gemm_k()));
  for (int c = 0; c < p.in_channels; ++c)  // k = (c * KH + r) * KW + s
    for (int r = 0; r < p.kernel_h; ++r)
      for (int s = 0; s < p.kernel_w; ++s) table.push_back({c * plane, r * p.dilation_h, s * p.dilation_w, 0});
  return table;
}

std::vector<LutEntry> build_conv_lut_chunked(const Conv2DParams& p) {
  check_table_range(p);
  GIE_REQUIRE(p.in_channels % 8 == 0, StatusCode::kInvalidArgument,
              "chunked gather table needs in_channels % 8 == 0 (in_channels = " + std::to_string(p.in_channels) + ")");
  std::vector<LutEntry> table;
  table.reserve(size_t(p.gemm_k() / 8));
  for (int r = 0; r < p.kernel_h; ++r)  // q = (r * KW + s) * C/8 + chunk: taps outer, 8-channel chunks inner
    for (int s = 0; s < p.kernel_w; ++s)
      for (int c8 = 0; c8 < p.in_channels; c8 += 8) table.push_back({c8, r * p.dilation_h, s * p.dilation_w, 0});
  return table;
}

}  // namespace gie
