"""GPU parity of the strict-FP32 and TF32 path (conv_f32.hip through gie_hip_conv_f32 and the plan API).

* FP32 on every correctness shape of the reference (tests/shapes.h) for both tile configurations, against the
  oracle's double reference under the reference's FP32 tolerance (tests/conv_test_common.h:83-127) and the FP32
  gate rel-L2 <= 1e-5; split-K partials + the FP32 reduce on long reductions;
* TF32: inputs uploaded unrounded, compared with the double reference computed on the TF32-rounded inputs under
  the FP32 tolerance — products of TF32 values are exact, so only a wrong rounding of the inputs (mode, tie
  direction, bit position) could exceed it; and the plan API under the reference's TF32 tolerance;
* BASELINE config 1 (the FP32 3x3 layer N1 C64 56x56 K64) on the GPU through Conv2D::forward, gates included;
* the dispatcher routes FP32 to the implicit_gemm FP32 entries and TF32 to the tensor-core TF32 entries;
* argument rejection.
"""
import ctypes

import numpy as np
import pytest

import gie
import oracle as O
from gpu_helpers import SHAPES, Bundle, problem, run_plan

pytestmark = pytest.mark.gpu


def _geom(p):
    return p.geom(p.in_channels)


def _stages(p):
    return p.kernel_h * p.kernel_w * ((p.in_channels + 15) // 16)


def _run_cabi(config, dtype, p, t, split, x=None, w=None):
    ny = int(np.prod(p.y_shape()))
    part = gie.DeviceBuffer(split * ny * 4) if split > 1 else None
    g = _geom(p)
    t.poison()
    gie.check_hip(gie.hip().gie_hip_conv_f32(config, dtype, ctypes.byref(g), x or t.dx.addr, w or t.dw.addr,
                                             t.bias_addr(), t.dy.addr, part.addr if part else None, split, None),
                  f"conv_f32 config {config} split {split}")
    if split > 1:
        gie.check_hip(gie.hip().gie_hip_splitk_reduce(dtype, part.addr, t.bias_addr(), t.dy.addr, ny, split,
                                                      p.out_channels, p.out_h * p.out_w, int(p.relu), None),
                      "reduce")
    gie.synchronize()
    return t.y()


def _rel_l2(y, ref):
    y, ref = y.ravel().astype(np.float64), ref.ravel().astype(np.float64)
    return np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)


@pytest.mark.parametrize("si", range(len(SHAPES)), ids=[s[0] for s in SHAPES])
def test_fp32_on_correctness_shapes(si):
    mode = si % 3
    p = problem(SHAPES[si], "fp32", mode >= 1, mode == 2)
    b = Bundle(p, 0xF32 + si, [O.UNIFORM, O.NORMAL, O.SPARSE, O.POSITIVE][si % 4])
    for config in range(gie.hip().gie_hip_f32_config_count()):
        assert gie.hip().gie_hip_f32_check(config, ctypes.byref(_geom(p)), None) == 0
        y = _run_cabi(config, gie.PRECISIONS["fp32"], p, b.t, 1)
        m = b.compare(y)
        assert m.passed(), f"config {config}: {m.summary()}"
        assert _rel_l2(y, b.ref) <= 1e-5


SPLIT_CASES = [(SHAPES[10], 4), (SHAPES[14], 3), (SHAPES[16], 8), (SHAPES[6], 2), (SHAPES[2], 1)]


@pytest.mark.parametrize("shape,split", SPLIT_CASES, ids=[f"{s[0]}-sk{k}" for s, k in SPLIT_CASES])
def test_fp32_split_k(shape, split):
    p = problem(shape, "fp32", True, True)
    b = Bundle(p, 0x5F32 + split, O.NORMAL)
    assert split <= _stages(p)
    for config in (0, 1):
        y = _run_cabi(config, gie.PRECISIONS["fp32"], p, b.t, split)
        m = b.compare(y)
        assert m.passed(), f"config {config}: {m.summary()}"
        assert _rel_l2(y, b.ref) <= 1e-5


@pytest.mark.parametrize("si", [2, 6, 9, 14, 16, 22], ids=lambda i: SHAPES[i][0])
def test_tf32_rounds_inputs_like_the_reference(si):
    """Raw FP32 inputs in, TF32 (ties away) rounding in the kernel: matches the reference on rounded inputs."""
    p32 = problem(SHAPES[si], "fp32", True, si % 2 == 0)
    b = Bundle(p32, 0x7F32 + si, O.NORMAL)
    # the raw values sit off the TF32 grid
    assert np.mean(O.quantize("tf32", b.x) != b.x) > 0.9
    x_t, w_t = O.quantize("tf32", b.x), O.quantize("tf32", b.w)
    ref, scale = O.conv2d(b.c, x_t, w_t, b.b)  # FP32 conv on the rounded values (double accumulation)
    for config in (0, 1):
        for split in (1, 2):
            y = _run_cabi(config, gie.PRECISIONS["tf32"], p32, b.t, split)
            m = O.compare(y.ravel(), ref, scale, b.c)
            assert m.passed(), f"config {config} split {split}: {m.summary()}"
    # a plain FP32 run on the same raw inputs differs from the rounded reference (the rounding is really applied)
    y32 = _run_cabi(0, gie.PRECISIONS["fp32"], p32, b.t, 1)
    assert not np.array_equal(y32, y)


def test_tf32_round_ties_away_from_zero():
    """x exactly halfway between two TF32 values (bit 12 set, bits 0-11 clear): rounds away from zero."""
    p = gie.Problem(1, 1, 1, 4, 1, 1, 1, 1, 1, 0, 0, precision="fp32", has_bias=False, relu=False)
    base = np.array([1.0, -1.0, 3.0, -0.75], np.float32)
    tie = (base.view(np.uint32) | np.uint32(0x1000)).view(np.float32)   # 1 + 2^-11 etc.: halfway cases
    x, w = tie, np.ones(1, np.float32)
    t = gie.ConvTensors(p, x.reshape(1, 1, 1, 4), w.reshape(1, 1, 1, 1), None)
    y = _run_cabi(0, gie.PRECISIONS["tf32"], p, t, 1).ravel()
    away = ((tie.view(np.uint32) + np.uint32(0x1000)) & np.uint32(0xFFFFE000)).view(np.float32)
    assert np.array_equal(y, away) and np.all(np.abs(away) > np.abs(base))
    assert np.array_equal(y, O.quantize("tf32", tie))


@pytest.mark.parametrize("prec", ["fp32", "tf32"])
def test_plan_api_and_dispatcher_route_fp32_and_tf32(prec):
    p = problem(SHAPES[8], prec, True, True)
    b = Bundle(p, 0xD1 + (prec == "tf32"), O.UNIFORM)
    k, src, _ = gie.select(p)
    stem = "implicit_gemm_fp32_" if prec == "fp32" else "mfma_tf32_"
    assert k.startswith(stem), k
    picks = [n for n in gie.registry() if n.startswith(stem)]
    assert len(picks) == 8
    for n in picks:
        y, why = run_plan(n, b)
        if y is None:
            assert "split-K" in why, why
            continue
        m = b.compare(y)
        assert m.passed(), f"{n}: {m.summary()}"
    # the whole API: workspace query + forward
    ws_n = gie.workspace_size(p)
    ws = gie.DeviceBuffer(ws_n) if ws_n else None
    b.t.poison()
    gie.forward(p, b.t, ws)
    gie.synchronize()
    assert b.compare(b.t.y()).passed()


def test_baseline_config1_fp32_on_gpu():
    """FP32 N1 C64 56x56 K64 3x3 s1 p1, bias + ReLU, benchmark scaling, seeded."""
    p = gie.Problem(1, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, precision="fp32", has_bias=True, relu=True)
    b = Bundle(p, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)
    ws_n = gie.workspace_size(p, autotune=False)
    ws = gie.DeviceBuffer(ws_n) if ws_n else None
    b.t.poison()
    gie.forward(p, b.t, ws)
    gie.synchronize()
    y = b.t.y()
    m = b.compare(y)
    assert m.passed(), m.summary()
    assert _rel_l2(y, b.ref) <= 1e-5


def test_fp32_rejects_bad_arguments():
    p = problem(SHAPES[6], "fp32", True, True)
    g = _geom(p)
    d = gie.DeviceBuffer(1 << 22)
    h = gie.hip()
    assert h.gie_hip_conv_f32(0, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 1, None) == -2  # fp16
    assert h.gie_hip_conv_f32(0, 0, ctypes.byref(g), d.addr + 2, d.addr, None, d.addr, None, 1, None) == -1
    assert h.gie_hip_conv_f32(0, 0, ctypes.byref(g), d.addr, d.addr, None, None, None, 1, None) == -1
    assert h.gie_hip_conv_f32(0, 0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 2, None) == -1  # no partial
    assert h.gie_hip_conv_f32(0, 0, ctypes.byref(g), d.addr, d.addr, None, d.addr, d.addr, _stages(p) + 1,
                              None) == -1
    assert h.gie_hip_conv_f32(2, 0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 1, None) == -1
    big = gie.Problem(64, 1024, 256, 256, 64, 3, 3, 1, 1, 1, 1, precision="fp32")  # 2^32 input elements
    assert h.gie_hip_f32_check(0, ctypes.byref(_geom(big)), None) == -2
