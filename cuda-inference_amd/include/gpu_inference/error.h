// Error handling for the MI355X Conv2D library (same contract as the reference's include/gpu_inference/error.h).
//
// Every recoverable failure (invalid arguments, unsupported configurations, HIP runtime errors) is reported by
// throwing gie::Error with a StatusCode. The execution path never swallows an error and never returns a result
// that was not computed. API delta from the reference: the CUDA/cuBLAS/cuDNN codes become one kHipError
// (this library has no BLAS/DNN dependency).
#pragma once

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

namespace gie {

enum class StatusCode {
  kOk = 0,
  kInvalidArgument,  // caller error: bad shape, null pointer, aliasing, ...
  kUnsupported,      // valid request that the chosen kernel / hardware can't run
  kWorkspaceTooSmall,
  kHipError,
  kInternal,
  kIo,
};

const char* to_string(StatusCode code);

class Error : public std::runtime_error {
 public:
  Error(StatusCode code, const std::string& message)
      : std::runtime_error(std::string(gie::to_string(code)) + ": " + message), code_(code) {}
  StatusCode code() const noexcept { return code_; }

 private:
  StatusCode code_;
};

[[noreturn]] void throw_hip_error(hipError_t err, const char* expr, const char* file, int line);
// Maps a status returned by the kernel C-ABI (include/gie_hip.h) to an exception; no-op for 0.
void check_kernel_status(int status, const char* what);

}  // namespace gie

#define GIE_HIP_CHECK(expr)                                                                     \
  do {                                                                                          \
    hipError_t gie_err_ = (expr);                                                               \
    if (gie_err_ != hipSuccess) ::gie::throw_hip_error(gie_err_, #expr, __FILE__, __LINE__);    \
  } while (0)

// Validates a caller-supplied condition; throws gie::Error(code, msg) on failure.
#define GIE_REQUIRE(cond, code, msg)              \
  do {                                            \
    if (!(cond)) throw ::gie::Error((code), (msg)); \
  } while (0)
