// Kernel registry (the reference's registry.cpp contract: unique names, mandatory function pointers, stable
// element addresses). The reference's per-(c,r,s) gather tables (src/kernels/conv_common.cu:39-50) have no
// counterpart: every kernel here walks the filter taps with incremental offsets computed in registers.
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

}  // namespace gie
