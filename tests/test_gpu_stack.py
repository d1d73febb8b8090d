"""GPU parity of the stack kernel (conv_stack.hip: 3x3, stride 1, padding 1, small images stacked into one zero-
separated plane per workgroup, straight from NCHW x and OIHW w) through its C-ABI, against the oracle's double
reference under the reference's tolerance (tests/conv_test_common.h:83-127) and, at BASELINE size, the benchmark
gates.

Cases cover every registered configuration: image groups that fill the stack and groups left partial by the batch,
rows of 1 to 7 pixels starting at either 2-byte parity (the row loads shift by one element), image heights that
leave dummy rows at the end of the stack, filter counts past and below a 32-filter block, split-K 1 to 8 with the
reduce kernel (ranges of unequal slice counts), no bias / no ReLU, both precisions, an x offset by 4 bytes, a second
launch giving the same bits, and argument rejection.
"""
import ctypes

import numpy as np
import pytest

import gie
import oracle as O
from gpu_helpers import BENCH_CONFIGS, Bundle

pytestmark = pytest.mark.gpu


def _problem(B, C, H, W, K, prec, bias=True, relu=True):
    return gie.Problem(B, C, H, W, K, 3, 3, 1, 1, 1, 1, precision=prec, has_bias=bias, relu=relu)


def _configs():
    out = []
    for i in range(gie.hip().gie_hip_stack_config_count()):
        c = gie.GieStackConfig()
        gie.check_hip(gie.hip().gie_hip_stack_config_get(i, ctypes.byref(c)), "stack_config_get")
        out.append(c)
    return out


def _run(p, b, ci, split=1, xoff=0, reps=1):
    """One stack launch (plus the reduce for split > 1) through the C-ABI; returns the outputs as floats."""
    g = p.geom(p.in_channels)
    dt = gie.PRECISIONS[p.precision]
    ny = int(np.prod(p.y_shape()))
    x = b.t.dx.addr
    keep = []
    if xoff:
        xs = gie.DeviceBuffer(b.t.dx.nbytes + 16)
        gie.check(gie.capi().gie_memcpy_d2d_async(xs.addr + xoff, b.t.dx.addr, b.t.dx.nbytes, None))
        x = xs.addr + xoff
        keep.append(xs)
    part = gie.DeviceBuffer(split * ny * 4) if split > 1 else None
    outs = []
    for _ in range(reps):
        b.t.poison()
        rc = gie.hip().gie_hip_conv_stack(ci, dt, ctypes.byref(g), x, b.t.dw.addr, b.t.bias_addr(), b.t.dy.addr,
                                          part.addr if part else None, split, None)
        gie.check_hip(rc, f"conv_stack {ci}")
        if split > 1:
            gie.check_hip(gie.hip().gie_hip_splitk_reduce(dt, part.addr, b.t.bias_addr(), b.t.dy.addr, ny, split,
                                                          p.out_channels, p.out_h * p.out_w, int(p.relu), None),
                          "reduce")
        gie.synchronize()
        outs.append(b.t.y())
    return outs


CASES = [
    # (B, C, H, W, O, precision, bias, relu, split, x offset)
    (8, 512, 7, 7, 64, "bf16", True, True, 8, 0),      # the benchmark layer's image shape, split 8
    (8, 256, 7, 7, 64, "fp16", True, True, 1, 0),      # split 1: bias + ReLU epilogue in the kernel
    (3, 64, 7, 7, 40, "fp16", True, False, 1, 0),      # partial image group, O past one filter block
    (5, 96, 6, 5, 20, "bf16", False, True, 2, 0),      # H + 1 = 7 (dummy stack rows), W = 5, O below a block
    (2, 32, 4, 4, 8, "bf16", True, True, 1, 0),        # one slice
    (16, 64, 3, 7, 32, "fp16", True, True, 2, 0),      # 4-row stack pitch: 8 images per group
    (4, 128, 7, 1, 16, "fp16", True, True, 4, 0),      # 1-pixel rows
    (4, 256, 7, 7, 96, "fp16", True, True, 2, 0),      # split 2, three filter blocks
    (2, 64, 15, 7, 32, "bf16", True, True, 1, 0),      # tall images: one or two per stack
    (6, 160, 5, 6, 48, "fp16", True, True, 4, 0),      # 5 slices over 4 ranges (1 or 2 slices each)
    (8, 512, 7, 7, 64, "fp16", True, True, 4, 4),      # x offset by 4 bytes
    (1, 96, 2, 3, 33, "bf16", False, False, 1, 0),     # tiny, no bias, no ReLU, O = 33
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"-{c[5]}-sk{c[8]}-o{c[9]}")
def test_stack_kernel_through_cabi(case):
    B, C, H, W, K, prec, bias, relu, split, xoff = case
    p = _problem(B, C, H, W, K, prec, bias, relu)
    b = Bundle(p, 0x57AC + C + K + split, O.NORMAL)
    g = p.geom(p.in_channels)
    ran = 0
    for ci, cfg in enumerate(_configs()):
        lds, ni = ctypes.c_int(0), ctypes.c_int(0)
        if gie.hip().gie_hip_stack_check(ci, ctypes.byref(g), ctypes.byref(lds), ctypes.byref(ni)) != 0:
            continue
        assert 0 < lds.value <= 160 * 1024
        assert 1 <= ni.value <= B and ni.value * (H + 1) <= cfg.rows
        print(f"stack config {ci} (rows {cfg.rows}, {ni.value} images per unit) on {case}", flush=True)
        first, second = _run(p, b, ci, split, xoff, reps=2)
        m = b.compare(first)
        assert m.passed(), f"config {ci}: {m.summary()}"
        assert np.array_equal(np.nan_to_num(first), np.nan_to_num(second)), f"config {ci}: second launch differs"
        ran += 1
    assert ran > 0, f"no stack configuration accepts {case}"


def test_stack_bench_config_full_size():
    c = dict(BENCH_CONFIGS["c5_bf16_3x3_splitk"])
    prec = c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    b = Bundle(p, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)
    g = p.geom(p.in_channels)
    ran = 0
    for ci, cfg in enumerate(_configs()):
        if gie.hip().gie_hip_stack_check(ci, ctypes.byref(g), None, None) != 0:
            continue
        for split in (1, 2, 4, 8):
            print(f"stack config {ci} split {split} on c5", flush=True)
            (y,) = _run(p, b, ci, split)
            m = b.compare(y)
            gates = b.gates(y)
            assert m.passed(), f"config {ci} sk{split}: {m.summary()}"
            assert gates["rel_l2"] <= 1e-3 and gates["max_abs"] <= 2e-2, f"config {ci} sk{split}: {gates}"
            ran += 1
    assert ran == 4 * len(_configs())


def test_stack_argument_checks():
    h = gie.hip()
    ok = _problem(2, 64, 7, 7, 64, "fp16")
    g = ok.geom(64)
    d = gie.DeviceBuffer(1 << 22)
    assert h.gie_hip_conv_stack(0, 1, ctypes.byref(g), d.addr, d.addr + 8, None, d.addr, None, 1, None) == -2  # w
    assert h.gie_hip_conv_stack(0, 1, ctypes.byref(g), d.addr + 2, d.addr, None, d.addr, None, 1, None) == -2  # x
    assert h.gie_hip_conv_stack(0, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr + 1, None, 1, None) == -1  # y odd
    assert h.gie_hip_conv_stack(0, 0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 1, None) != 0  # fp32
    assert h.gie_hip_conv_stack(0, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 0, None) == -1  # split 0
    assert h.gie_hip_conv_stack(0, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 2, None) == -1  # partial
    assert h.gie_hip_conv_stack(0, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, d.addr, 3, None) == -1  # > S
    assert h.gie_hip_conv_stack(99, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 1, None) == -1


def test_stack_repeated_launches_agree_bitwise():
    """Regression: register loads issued for the slices past the last one once landed in registers the epilogue had
    reused, corrupting a few outputs when the loads were slow (two workgroups sharing a CU, or real data behind
    them). Repeated launches of every configuration, including ones whose 512 or 1024 workgroups share CUs, must
    give the same bits, and those bits must pass the oracle."""
    c = dict(BENCH_CONFIGS["c5_bf16_3x3_splitk"])
    prec = c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    b = Bundle(p, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)
    for ci in range(len(_configs())):
        for split in (1, 8):
            print(f"stack config {ci} split {split}: 6 launches", flush=True)
            outs = _run(p, b, ci, split, reps=6)
            assert b.compare(outs[0]).passed(), f"config {ci} sk{split}"
            for k, y in enumerate(outs[1:], 1):
                assert np.array_equal(outs[0], y), f"config {ci} sk{split}: launch {k} differs"
    q = _problem(8, 256, 7, 7, 64, "fp16", bias=False, relu=False)
    bq = Bundle(q, 777, O.UNIFORM)
    for ci in range(len(_configs())):
        outs = _run(q, bq, ci, 1, reps=8)
        assert bq.compare(outs[0]).passed(), f"config {ci}"
        assert all(np.array_equal(outs[0], y) for y in outs[1:]), f"config {ci}: launches differ"
