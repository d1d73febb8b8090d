// L1 vocabulary: errors, device buffers, tensor shapes, problem keys and validation, roctx ranges.
#include <limits>
#include <sstream>

#include "gie_hip.h"
#include "gpu_inference/conv2d.h"
#include "gpu_inference/error.h"
#include "gpu_inference/roctx.h"
#include "gpu_inference/tensor.h"

#ifdef GIE_HAS_ROCTX
#include <roctracer/roctx.h>
#endif

namespace gie {

const char* to_string(StatusCode code) {
  switch (code) {
    case StatusCode::kOk: return "Ok";
    case StatusCode::kInvalidArgument: return "InvalidArgument";
    case StatusCode::kUnsupported: return "Unsupported";
    case StatusCode::kWorkspaceTooSmall: return "WorkspaceTooSmall";
    case StatusCode::kHipError: return "HipError";
    case StatusCode::kInternal: return "Internal";
    case StatusCode::kIo: return "Io";
  }
  return "Unknown";
}

void throw_hip_error(hipError_t err, const char* expr, const char* file, int line) {
  (void)hipGetLastError();  // clear the non-sticky error so a caller that catches can continue
  std::ostringstream os;
  os << expr << " failed with " << hipGetErrorName(err) << " (" << hipGetErrorString(err) << ") at " << file << ":"
     << line;
  throw Error(StatusCode::kHipError, os.str());
}

void check_kernel_status(int status, const char* what) {
  if (status == GIE_HIP_OK) return;
  if (status == GIE_HIP_EINVAL) throw Error(StatusCode::kInvalidArgument, std::string(what) + ": invalid argument");
  if (status == GIE_HIP_EUNSUPPORTED)
    throw Error(StatusCode::kUnsupported, std::string(what) + ": unsupported by this kernel configuration");
  (void)hipGetLastError();
  throw Error(StatusCode::kHipError, std::string(what) + " failed with " +
                                         hipGetErrorName(static_cast<hipError_t>(status)) + " (" +
                                         hipGetErrorString(static_cast<hipError_t>(status)) + ")");
}

// ---- tensor.h ----
const char* to_string(DataType t) {
  switch (t) {
    case DataType::kFloat32: return "float32";
    case DataType::kFloat16: return "float16";
    case DataType::kBFloat16: return "bfloat16";
  }
  return "?";
}

DeviceBuffer::DeviceBuffer(size_t bytes) : bytes_(bytes) {
  if (bytes > 0) GIE_HIP_CHECK(hipMalloc(&ptr_, bytes));
}

DeviceBuffer::~DeviceBuffer() { reset(); }

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
  if (this != &o) {
    reset();
    ptr_ = o.ptr_;
    bytes_ = o.bytes_;
    o.ptr_ = nullptr;
    o.bytes_ = 0;
  }
  return *this;
}

void DeviceBuffer::memset_async(int value, hipStream_t stream) {
  if (ptr_) GIE_HIP_CHECK(hipMemsetAsync(ptr_, value, bytes_, stream));
}

void DeviceBuffer::reset() {
  if (ptr_) (void)hipFree(ptr_);
  ptr_ = nullptr;
  bytes_ = 0;
}

std::string TensorShape::to_string() const {
  std::ostringstream os;
  os << "[" << n << "," << c << "," << h << "," << w << "]";
  return os.str();
}

// ---- conv2d.h (the reference's conv2d.cpp:16-109) ----
DataType tensor_dtype(Precision p) {
  switch (p) {
    case Precision::kFp32:
    case Precision::kTf32: return DataType::kFloat32;
    case Precision::kFp16: return DataType::kFloat16;
    case Precision::kBf16: return DataType::kBFloat16;
  }
  return DataType::kFloat32;
}

const char* to_string(Precision p) {
  switch (p) {
    case Precision::kFp32: return "fp32";
    case Precision::kFp16: return "fp16";
    case Precision::kBf16: return "bf16";
    case Precision::kTf32: return "tf32";
  }
  return "?";
}

Precision precision_from_string(const std::string& s) {
  if (s == "fp32") return Precision::kFp32;
  if (s == "fp16") return Precision::kFp16;
  if (s == "bf16") return Precision::kBf16;
  if (s == "tf32") return Precision::kTf32;
  throw Error(StatusCode::kInvalidArgument, "unknown precision '" + s + "' (fp32|fp16|bf16|tf32)");
}

const char* to_string(Activation a) { return a == Activation::kReLU ? "relu" : "none"; }

const char* to_string(Backend b) {
  switch (b) {
    case Backend::kAuto: return "auto";
    case Backend::kCpuReference: return "cpu_reference";
    case Backend::kDirect: return "direct";
    case Backend::kIm2colGemm: return "im2col_gemm";
    case Backend::kSimtTiled: return "simt_tiled";
    case Backend::kImplicitGemm: return "implicit_gemm";
    case Backend::kTensorCore: return "tensor_core";
  }
  return "?";
}

Backend backend_from_string(const std::string& s) {
  for (Backend b : {Backend::kAuto, Backend::kCpuReference, Backend::kDirect, Backend::kIm2colGemm,
                    Backend::kSimtTiled, Backend::kImplicitGemm, Backend::kTensorCore}) {
    if (s == to_string(b)) return b;
  }
  throw Error(StatusCode::kInvalidArgument, "unknown backend '" + s + "'");
}

std::string Conv2DParams::to_string() const {
  std::ostringstream os;
  os << "B" << batch << "_C" << in_channels << "_" << in_h << "x" << in_w << "_O" << out_channels << "_K" << kernel_h
     << "x" << kernel_w << "_s" << stride_h << "x" << stride_w << "_p" << pad_h << "x" << pad_w << "_d" << dilation_h
     << "x" << dilation_w << "_g" << groups;
  return os.str();
}

bool Conv2DParams::operator==(const Conv2DParams& o) const { return to_string() == o.to_string(); }

std::string ConvProblem::key() const {
  std::ostringstream os;
  os << p.to_string() << "_" << gie::to_string(precision) << "_b" << int(has_bias) << "_"
     << gie::to_string(activation);
  return os.str();
}

void validate_problem(const ConvProblem& prob) {
  const Conv2DParams& p = prob.p;
  auto bad = [](const std::string& m) { throw Error(StatusCode::kInvalidArgument, m); };
  if (p.batch <= 0 || p.in_channels <= 0 || p.in_h <= 0 || p.in_w <= 0 || p.out_channels <= 0 || p.kernel_h <= 0 ||
      p.kernel_w <= 0)
    bad("all extents must be positive: " + p.to_string());
  if (p.stride_h <= 0 || p.stride_w <= 0) bad("strides must be positive");
  if (p.pad_h < 0 || p.pad_w < 0) bad("padding must be non-negative");
  if (p.dilation_h != 1 || p.dilation_w != 1) throw Error(StatusCode::kUnsupported, "dilation != 1 is not supported");
  if (p.groups != 1) throw Error(StatusCode::kUnsupported, "grouped convolution is not supported");
  const int64_t eff_h = int64_t(p.dilation_h) * (p.kernel_h - 1) + 1;
  const int64_t eff_w = int64_t(p.dilation_w) * (p.kernel_w - 1) + 1;
  if (int64_t(p.in_h) + 2 * int64_t(p.pad_h) < eff_h || int64_t(p.in_w) + 2 * int64_t(p.pad_w) < eff_w)
    bad("kernel larger than padded input: " + p.to_string());
  if (p.out_h() <= 0 || p.out_w() <= 0) bad("empty output: " + p.to_string());
  const int64_t lim = std::numeric_limits<int32_t>::max();
  if (p.gemm_n() > lim || p.gemm_k() > lim || p.gemm_m() > lim)
    bad("GEMM extents exceed 32-bit indexing: " + p.to_string());
  if (int64_t(p.in_channels) * p.in_h * p.in_w > lim) bad("per-image input size exceeds 32-bit indexing: " + p.to_string());
  if (int64_t(p.out_channels) * p.out_h() * p.out_w() > lim)
    bad("per-image output size exceeds 32-bit indexing: " + p.to_string());
}

// ---- roctx.h ----
#ifdef GIE_HAS_ROCTX
RoctxRange::RoctxRange(const char* name) { roctxRangePush(name); }
RoctxRange::~RoctxRange() { roctxRangePop(); }
#else
RoctxRange::RoctxRange(const char*) {}
RoctxRange::~RoctxRange() {}
#endif

}  // namespace gie
