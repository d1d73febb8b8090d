// Host side of the stand-alone bias / ReLU passes (the reference's src/kernels/elementwise.cu:37-56): argument
// checks and the call into the gie_hip_bias_act kernel entry.
#include "gpu_inference/fused_ops.h"

#include "gie_hip.h"
#include "gpu_inference/error.h"

namespace gie {

void launch_bias_act(const Conv2DParams& p, Precision prec, const void* bias, bool relu, void* y,
                     hipStream_t stream) {
  if (bias == nullptr && !relu) return;
  if (y == nullptr) throw Error(StatusCode::kInvalidArgument, "bias/ReLU pass: output pointer is null");
  // TF32 keeps FP32 storage, so its output is processed as FP32
  const int dtype = prec == Precision::kFp16 ? GIE_HIP_FP16 : prec == Precision::kBf16 ? GIE_HIP_BF16 : GIE_HIP_FP32;
  check_kernel_status(gie_hip_bias_act(dtype, y, bias, p.output_shape().numel(), p.out_channels,
                                       p.out_h() * p.out_w(), relu ? 1 : 0, stream),
                      "bias/ReLU pass");
}

void launch_bias_add(const Conv2DParams& p, Precision prec, const void* bias, void* y, hipStream_t stream) {
  launch_bias_act(p, prec, bias, false, y, stream);
}

void launch_relu(const Conv2DParams& p, Precision prec, void* y, hipStream_t stream) {
  launch_bias_act(p, prec, nullptr, true, y, stream);
}

}  // namespace gie
