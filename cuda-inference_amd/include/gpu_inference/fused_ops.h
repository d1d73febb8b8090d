// Stand-alone elementwise passes over an NCHW convolution output (the reference's include/gpu_inference/
// fused_ops.h:1-26, same names and meaning): the unfused side of the epilogue-fusion experiment. The MFMA
// convolution families never call these; they apply bias + ReLU to the FP32 accumulators before their single
// rounding. Each pass reads and writes the whole output once and enqueues one kernel on `stream` (no
// allocation, no synchronization).
#pragma once

#include <hip/hip_runtime_api.h>

#include "gpu_inference/conv2d.h"

namespace gie {

// y[b,o,:,:] = round(y[b,o,:,:] + bias[o])   (in place)
void launch_bias_add(const Conv2DParams& p, Precision prec, const void* bias, void* y, hipStream_t stream);
// y = max(y, 0)                              (in place)
void launch_relu(const Conv2DParams& p, Precision prec, void* y, hipStream_t stream);
// y = round(act(y + bias)) in one pass (either part optional; nothing is launched when both are off)
void launch_bias_act(const Conv2DParams& p, Precision prec, const void* bias_or_null, bool relu, void* y,
                     hipStream_t stream);

}  // namespace gie
