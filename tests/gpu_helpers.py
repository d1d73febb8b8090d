"""Shared machinery of the GPU parity tests: seeded data from the oracle, device upload through the library's
C-ABI, and comparison against the oracle with the reference's tolerance model plus the benchmark gates
(rel-L2 <= 1e-3 and max-abs <= 2e-2 for FP16/BF16; BF16 rel-L2 against the reference rounded once to BF16).
Plays the role of the reference's tests/conv_test_common.h (make_bundle / run_kernel / run_suite)."""
from __future__ import annotations

import numpy as np

import gie
import oracle as O

# tests/shapes.h:27-57 (name, B, C, H, W, O, Kh, Kw, Sh, Sw, Ph, Pw)
SHAPES = [
    ("tiny_1ch_5x5_k3", 1, 1, 5, 5, 1, 3, 3, 1, 1, 0, 0),
    ("scalar_1x1_k1", 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0),
    ("rgb_8x8_k3p1", 1, 3, 8, 8, 4, 3, 3, 1, 1, 1, 1),
    ("rgb_32x32_k3p1_b2", 2, 3, 32, 32, 16, 3, 3, 1, 1, 1, 1),
    ("odd_unequal_k5s2", 1, 3, 33, 31, 8, 5, 5, 2, 2, 2, 2),
    ("pointwise_odd_b2", 2, 16, 15, 17, 24, 1, 1, 1, 1, 0, 0),
    ("resnet_14x14_b8_k3", 8, 64, 14, 14, 64, 3, 3, 1, 1, 1, 1),
    ("resnet_56x56_1x1", 1, 64, 56, 56, 64, 1, 1, 1, 1, 0, 0),
    ("resnet_down_28_s2_b2", 2, 64, 28, 28, 128, 3, 3, 2, 2, 1, 1),
    ("k7_b16_c32", 16, 32, 20, 20, 48, 7, 7, 1, 1, 3, 3),
    ("deep_512ch_7x7", 1, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1),
    ("b32_c16_16x16", 32, 16, 16, 16, 32, 3, 3, 1, 1, 1, 1),
    ("irregular_c7_o9_s2", 2, 7, 11, 13, 9, 3, 3, 2, 2, 0, 0),
    ("kernel_eq_map_7x7", 1, 3, 7, 7, 5, 7, 7, 1, 1, 3, 3),
    ("c130_o130_9x9", 2, 130, 9, 9, 130, 3, 3, 1, 1, 1, 1),
    ("o255_pointwise_13", 1, 64, 13, 13, 255, 1, 1, 1, 1, 0, 0),
    ("k5_b4_c96_27", 4, 96, 27, 27, 192, 5, 5, 1, 1, 2, 2),
    ("stem_7x7_s2_64", 2, 3, 64, 64, 64, 7, 7, 2, 2, 3, 3),
    ("down_14_s2_c256", 1, 256, 14, 14, 256, 3, 3, 2, 2, 1, 1),
    ("small_b8_4x4", 8, 8, 4, 4, 8, 3, 3, 1, 1, 1, 1),
    ("boundary_pad2_3x3", 1, 2, 3, 3, 3, 3, 3, 1, 1, 2, 2),
    ("boundary_pad4_k5", 1, 16, 10, 10, 16, 5, 5, 1, 1, 4, 4),
    ("aniso_k3x5_s2x1", 2, 8, 17, 23, 12, 3, 5, 2, 1, 1, 2),
    ("k1x3", 1, 4, 12, 12, 6, 1, 3, 1, 1, 0, 1),
    ("k3x1", 1, 4, 12, 12, 6, 3, 1, 1, 1, 1, 0),
    ("wide_1x1_b32", 32, 24, 7, 7, 40, 1, 1, 1, 1, 0, 0),
]

DISTS = [O.UNIFORM, O.NORMAL, O.SPARSE, O.POSITIVE]

# BASELINE.json configs 2-5 (config 1 is the CPU-only FP32 case)
BENCH_CONFIGS = {
    "c2_fp16_3x3": dict(batch=32, in_channels=256, in_h=14, in_w=14, out_channels=256, kernel_h=3, kernel_w=3,
                        stride_h=1, stride_w=1, pad_h=1, pad_w=1, precision="fp16"),
    "c3_fp16_1x1": dict(batch=64, in_channels=256, in_h=28, in_w=28, out_channels=1024, kernel_h=1, kernel_w=1,
                        stride_h=1, stride_w=1, pad_h=0, pad_w=0, precision="fp16"),
    "c4_fp16_7x7s2": dict(batch=64, in_channels=3, in_h=224, in_w=224, out_channels=64, kernel_h=7, kernel_w=7,
                          stride_h=2, stride_w=2, pad_h=3, pad_w=3, precision="fp16"),
    "c5_bf16_3x3_splitk": dict(batch=8, in_channels=512, in_h=7, in_w=7, out_channels=512, kernel_h=3, kernel_w=3,
                               stride_h=1, stride_w=1, pad_h=1, pad_w=1, precision="bf16"),
}
BENCH_SEED = 0x1234ABCD


def problem(shape, precision: str, bias: bool, relu: bool) -> gie.Problem:
    _, B, C, H, W, Oc, Kh, Kw, Sh, Sw, Ph, Pw = shape
    return gie.Problem(B, C, H, W, Oc, Kh, Kw, Sh, Sw, Ph, Pw, precision=precision, has_bias=bias, relu=relu)


def oracle_conv(p: gie.Problem) -> O.Conv:
    return O.Conv(p.batch, p.in_channels, p.in_h, p.in_w, p.out_channels, p.kernel_h, p.kernel_w, p.stride_h,
                  p.stride_w, p.pad_h, p.pad_w, p.dilation_h, p.dilation_w, p.groups, has_bias=p.has_bias,
                  relu=p.relu, precision=p.precision)


class Bundle:
    """Seeded data (oracle draw), device tensors, and the oracle's reference output (make_bundle)."""

    def __init__(self, p: gie.Problem, seed: int, dist: int = O.UNIFORM, scaling: int = O.SCALING_REFERENCE,
                 full_reference: bool = True, sample: int = 0):
        self.p = p
        self.c = oracle_conv(p)
        self.x, self.w, self.b = O.make_data(self.c, seed, dist, scaling)
        self.t = gie.ConvTensors(p, self.x, self.w, self.b)
        self.idx = None
        if full_reference:
            self.ref, self.scale = O.conv2d(self.c, self.x, self.w, self.b)
        else:
            n = int(np.prod(p.y_shape()))
            rng = np.random.default_rng(seed)
            self.idx = np.unique(np.concatenate([rng.integers(0, n, sample), np.arange(min(n, 4096)),
                                                 np.arange(max(0, n - 4096), n)]))
            self.ref, self.scale = O.conv2d_points(self.c, self.x, self.w, self.b, self.idx)

    def compare(self, y: np.ndarray) -> O.Metrics:
        test = y.ravel() if self.idx is None else y.ravel()[self.idx]
        return O.compare(test, self.ref, self.scale, self.c)

    def gates(self, y: np.ndarray) -> dict:
        """Benchmark gates: rel-L2 and max-abs (BF16 rel-L2 against the reference rounded once to BF16)."""
        test = (y.ravel() if self.idx is None else y.ravel()[self.idx]).astype(np.float64)
        ref = self.ref.ravel().astype(np.float64)
        ref_r = O.quantize(self.p.precision, self.ref.ravel()).astype(np.float64) if self.p.precision == "bf16" \
            else ref
        rel = np.linalg.norm(test - ref_r) / max(np.linalg.norm(ref_r), 1e-30)
        rel_raw = np.linalg.norm(test - ref) / max(np.linalg.norm(ref), 1e-30)
        return {"rel_l2": float(rel), "rel_l2_vs_unrounded": float(rel_raw),
                "max_abs": float(np.max(np.abs(test - ref))) if test.size else 0.0}


def run_plan(kernel: str, bundle: Bundle, repeats: int = 1):
    """Capability check -> plan -> poison -> execute -> download (the reference's run_kernel)."""
    ok, why = gie.kernel_supports(kernel, bundle.p)
    if not ok:
        return None, why
    plan = gie.Plan(bundle.p, kernel)
    ws = gie.DeviceBuffer(plan.workspace_bytes) if plan.workspace_bytes else None
    bundle.t.poison()
    for _ in range(repeats):
        plan.execute(bundle.t, ws)
    gie.synchronize()
    return bundle.t.y(), ""


def kernels(precision: str | None = None) -> list[str]:
    ks = gie.registry()
    return [k for k in ks if precision is None or f"_{precision}_" in k]
