// Build provenance; the GIE_* macros are defined by the library's Makefile.
#include "gpu_inference/build_info.h"

#include <string>

#ifndef GIE_SOURCE_FINGERPRINT
#define GIE_SOURCE_FINGERPRINT "unknown"
#endif
#ifndef GIE_BUILD_TYPE
#define GIE_BUILD_TYPE "Release"
#endif
#ifndef GIE_OFFLOAD_ARCHS
#define GIE_OFFLOAD_ARCHS "gfx950"
#endif
#ifndef GIE_HIPCC_VERSION
#define GIE_HIPCC_VERSION "unknown"
#endif
#ifndef GIE_HIP_FLAGS_STR
#define GIE_HIP_FLAGS_STR ""
#endif

namespace gie {

const BuildInfo& build_info() {
  static const BuildInfo info = [] {
    BuildInfo b;
    b.source_fingerprint = GIE_SOURCE_FINGERPRINT;
    b.build_type = GIE_BUILD_TYPE;
    b.offload_archs = GIE_OFFLOAD_ARCHS;
    b.hipcc_version = GIE_HIPCC_VERSION;
#if defined(__clang__)
    b.cxx_compiler = std::string("clang ") + __clang_version__;
#elif defined(__GNUC__)
    b.cxx_compiler = std::string("g++ ") + __VERSION__;
#else
    b.cxx_compiler = "unknown";
#endif
    b.hip_flags = GIE_HIP_FLAGS_STR;
#ifdef GIE_HAS_ROCTX
    b.has_roctx = true;
#endif
    return b;
  }();
  return info;
}

}  // namespace gie
