// RAII roctx range (the reference's NvtxRange): visible in rocprofv3 --marker-trace timelines when the library
// is built against roctx; a no-op otherwise.
#pragma once

namespace gie {

class RoctxRange {
 public:
  explicit RoctxRange(const char* name);
  ~RoctxRange();
  RoctxRange(const RoctxRange&) = delete;
  RoctxRange& operator=(const RoctxRange&) = delete;
};

}  // namespace gie
