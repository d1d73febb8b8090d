// Build provenance recorded in tuning-cache keys and benchmark metadata: a SHA-256 fingerprint over the
// library sources taken at build time, plus the compiler and flags.
#pragma once

#include <string>

namespace gie {

struct BuildInfo {
  std::string source_fingerprint;  // first 16 hex chars of SHA-256 over csrc/ and include/
  std::string build_type;
  std::string offload_archs;       // e.g. "gfx950"
  std::string hipcc_version;
  std::string cxx_compiler;
  std::string hip_flags;
  bool has_roctx = false;
};

const BuildInfo& build_info();

}  // namespace gie
