// Kernel registry (the reference's registry.cpp contract: unique names, mandatory function pointers, stable
// element addresses) + the LUT builders of the reference's API.
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

std::vector<LutEntry> build_conv_lut(const Conv2DParams& p) {
  const int64_t K = p.gemm_k();
  std::vector<LutEntry> lut(static_cast<size_t>(K));
  const int khw = p.kernel_h * p.kernel_w;
  for (int64_t k = 0; k < K; ++k) {
    const int c = int(k / khw), rs = int(k % khw);
    lut[size_t(k)] = {c * p.in_h * p.in_w, (rs / p.kernel_w) * p.dilation_h, (rs % p.kernel_w) * p.dilation_w, 0};
  }
  return lut;
}

std::vector<LutEntry> build_conv_lut_chunked(const Conv2DParams& p) {
  if (p.in_channels % 8 != 0) throw Error(StatusCode::kInvalidArgument, "chunked LUT needs C % 8 == 0");
  const int cv = p.in_channels / 8;
  const int64_t chunks = p.gemm_k() / 8;
  std::vector<LutEntry> lut(static_cast<size_t>(chunks));
  for (int64_t q = 0; q < chunks; ++q) {
    const int rs = int(q / cv);
    lut[size_t(q)] = {int32_t(8 * (q % cv)), (rs / p.kernel_w) * p.dilation_h, (rs % p.kernel_w) * p.dilation_w, 0};
  }
  return lut;
}

}  // namespace gie
