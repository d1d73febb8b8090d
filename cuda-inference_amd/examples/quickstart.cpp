// Minimal use of the public API: one fused FP16 conv + bias + ReLU through Conv2D::forward
// (what the reference's examples/quickstart.cpp shows, on HIP).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <vector>

#include "gpu_inference/conv2d.h"
#include "gpu_inference/reference.h"
#include "gpu_inference/testing.h"

int main() {
  using namespace gie;
  ConvProblem prob;
  prob.p.batch = 2;
  prob.p.in_channels = 64;
  prob.p.in_h = prob.p.in_w = 14;
  prob.p.out_channels = 64;
  prob.p.kernel_h = prob.p.kernel_w = 3;
  prob.p.pad_h = prob.p.pad_w = 1;
  prob.precision = Precision::kFp16;
  prob.has_bias = true;
  prob.activation = Activation::kReLU;
  try {
    ConvData d = make_conv_data(prob, 0x1234ABCD, Distribution::kUniform, Scaling::kBenchmark);
    DeviceBuffer ws(Conv2D::workspace_size(prob));
    const ConstTensorRef bias = d.b_ref();
    Conv2D::forward(d.x_ref(), d.w_ref(), &bias, prob, d.y_ref(), ws.data(), ws.size(), nullptr);
    GIE_HIP_CHECK(hipDeviceSynchronize());
    ReferenceOutput ref;
    cpu_conv2d_reference(prob, d.hx.data(), d.hw.data(), d.hb.data(), &ref);
    const auto y = download_as_float(d.dy.data(), prob.dtype(), prob.p.output_shape().numel());
    const ErrorMetrics m = compare_outputs(y.data(), ref.y.data(), ref.scale.data(), int64_t(y.size()),
                                           TolerancePolicy::for_problem(prob));
    std::printf("%s: %s -> %s\n", prob.key().c_str(), m.summary().c_str(), m.passed() ? "PASS" : "FAIL");
    return m.passed() ? 0 : 1;
  } catch (const Error& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 2;
  }
}
