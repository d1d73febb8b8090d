"""bench.py on the host: the driver's contract (one GPU only), the kernel labels the roofline object carries for
every registry family, the per-kernel HBM traffic lookup from the committed profile, and that the bench configs
are BASELINE.json's configs 2-5."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr


@pytest.mark.parametrize("name,fn", [
    ("slab_fp16_3x3_32x14r16_k32_s2_l_o2_sk1", "slab_lean_kernel"),
    ("slab_fp16_3x3_32x14r16_k32_s3_p_sk1", "slab_pipe_kernel"),
    ("slab_fp16_3x3_32x14r16_k32_s3_ld_sk1", "slab_split_kernel"),
    ("deep_bf16_3x3_16x8r8_k32x4_ld", "deep_kernel"),
    ("stack_bf16_3x3_32x8r8_k32_sk2", "stack_kernel"),
    ("slab_bf16_3x3_32x8r8_k32_s3_sk2", "slab_kernel"),
    ("band_fp16_3x3_32x224x32_s4_sk1", "band_kernel"),
    ("halo_bf16_3x3_64x128x32_s2_sk4", "halo_kernel"),
    ("pw_fp16_1x1_256x64x16_s4_wreg", "pws_kernel"),
    ("pw_bf16_1x1_128x128x32_s4_sk1", "pw_kernel"),
    ("stem_fp16_7x7s2_64x32x16_wreg", "stem_kernel"),
    ("narrow_bf16_3x3_32x32x16_k8w", "narrow_kernel"),
    ("implicit_gemm_fp32_128x128x16_mfma_sk1", "f32_kernel"),
    ("mfma_tf32_64x128x16_sk2", "f32_kernel"),
    ("mfma_fp16_128x128x64_w4x2_s3_sk1", "igemm_kernel"),
])
def test_roofline_names_the_device_function(name, fn):
    assert bench.dominant_kernel(name).startswith(fn + " ")


def test_traffic_lookup_is_per_kernel():
    with open(os.path.join(ROOT, "profiles", "traffic_c2_fp16_3x3.json")) as f:
        profiled = json.load(f)["kernels"]
    for k, v in profiled.items():
        assert bench.load_traffic(k) == pytest.approx(v["bytes_per_launch"])
        assert 1e6 < v["bytes_per_launch"] < 1e8
    assert bench.load_traffic("mfma_fp16_128x128x64_w4x2_s3_sk1") is None


def test_bench_configs_are_the_baseline_configs():
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        base = json.load(f)
    cfgs = base["configs"]
    assert len(cfgs) >= 5
    assert bench.HEADLINE == "c2_fp16_3x3"
    c2 = bench.CONFIGS["c2_fp16_3x3"]
    assert (c2["batch"], c2["in_channels"], c2["in_h"], c2["out_channels"], c2["kernel_h"]) == (32, 256, 14, 256, 3)
    c4 = bench.CONFIGS["c4_fp16_7x7s2_stem"]
    assert (c4["in_channels"], c4["kernel_h"], c4["stride_h"], c4["pad_h"]) == (3, 7, 2, 3)


class _P:
    """The attributes of gie.Problem that the byte accounting reads."""

    def __init__(self, b, c, h, w, o, k, esize=2):
        self.batch, self.in_channels, self.in_h, self.in_w, self.out_channels = b, c, h, w, o
        self.kernel_h = self.kernel_w = k
        self.esize = esize

    def x_shape(self):
        return (self.batch, self.in_channels, self.in_h, self.in_w)

    def w_shape(self):
        return (self.out_channels, self.in_channels, self.kernel_h, self.kernel_w)

    def y_shape(self):
        return (self.batch, self.out_channels, self.in_h, self.in_w)


def test_stage_bytes_follow_each_family():
    p = _P(32, 256, 14, 14, 256, 3)
    nx, nw = 32 * 256 * 196, 256 * 256 * 9
    # families reading NCHW x and OIHW w directly have no repack stage: no bytes, so no GB/s figure
    for k in ("slab_fp16_3x3_32x14r16_k32_s2_sk1", "pw_fp16_1x1_256x64x16_s4_wreg", "stem_fp16_7x7s2_64x32x16_wreg",
              "narrow_bf16_3x3_32x32x16_k8w"):
        assert bench.repack_bytes(k, p) is None
    # band repacks the weights only: OIHW read, 32-channel blocks written
    assert bench.repack_bytes("band_fp16_3x3_32x224x32_s4_sk1", p) == (nw + 256 * 9 * 256) * 2
    # the implicit GEMM repacks both operands
    assert bench.repack_bytes("mfma_fp16_128x128x64_w4x2_s3_sk1", p) == (nx + nw + (32 * 196 + 256 * 9) * 256) * 2
    # C = 250: the halo copy pads channels to whole 32-channel slices (256)
    q = _P(2, 250, 7, 7, 64, 3)
    assert bench.repack_bytes("halo_bf16_3x3_64x128x32_s2_sk4", q) == \
        (2 * 250 * 49 + 64 * 250 * 9 + (2 * 49 + 64 * 9) * 256) * 2
    # the reduce exists only with split-K: FP32 partials in, output and bias
    assert bench.reduce_bytes(1, p) is None
    ny = 32 * 256 * 196
    assert bench.reduce_bytes(4, p) == 4 * ny * 4 + ny * 2 + 256 * 2
