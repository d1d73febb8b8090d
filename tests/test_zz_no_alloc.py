"""The allocation-free slab entry (gie_hip_conv_slab_noalloc: split-K partials in the library's static per-device
scratch) against the allocating one (gie_hip_conv_slab into a caller buffer, then gie_hip_splitk_reduce), bit for
bit, on two calls in a row with the second one smaller, plus the oracle under the reference's tolerance
(tests/conv_test_common.h:83-127) and the scratch-size rejection.
"""
import ctypes

import numpy as np
import pytest

import gie
import oracle as O
from gpu_helpers import Bundle

pytestmark = pytest.mark.gpu


def _problem(B, C, H, W, K, prec):
    return gie.Problem(B, C, H, W, K, 3, 3, 1, 1, 1, 1, precision=prec, has_bias=True, relu=True)


def _config_for(g):
    h = gie.hip()
    for ci in range(h.gie_hip_slab_config_count()):
        if h.gie_hip_slab_check(ci, ctypes.byref(g), None) == 0:
            return ci
    raise AssertionError("no slab configuration accepts the geometry")


def _with_buffer(p, b, ci, split):
    """The allocating entry: slab kernel into a caller-owned partial buffer, then the reduce."""
    g = p.geom(p.in_channels)
    dt = gie.PRECISIONS[p.precision]
    ny = int(np.prod(p.y_shape()))
    part = gie.DeviceBuffer(split * ny * 4) if split > 1 else None
    b.t.poison()
    gie.check_hip(gie.hip().gie_hip_conv_slab(ci, dt, ctypes.byref(g), b.t.dx.addr, b.t.dw.addr, b.t.bias_addr(),
                                              b.t.dy.addr, part.addr if part else None, split, None), "conv_slab")
    if split > 1:
        gie.check_hip(gie.hip().gie_hip_splitk_reduce(dt, part.addr, b.t.bias_addr(), b.t.dy.addr, ny, split,
                                                      p.out_channels, p.out_h * p.out_w, int(p.relu), None), "reduce")
    gie.synchronize()
    return b.t.y()


def _no_alloc(p, b, ci, split):
    g = p.geom(p.in_channels)
    b.t.poison()
    gie.check_hip(gie.hip().gie_hip_conv_slab_noalloc(ci, gie.PRECISIONS[p.precision], ctypes.byref(g), b.t.dx.addr,
                                                      b.t.dw.addr, b.t.bias_addr(), b.t.dy.addr, split, None),
                  "conv_slab_noalloc")
    gie.synchronize()
    return b.t.y()


@pytest.mark.parametrize("prec", ["fp16", "bf16"])
def test_no_alloc_matches_allocating_entry(prec):
    # first call: config-5 shape at split 8 (the largest partials of the sequence); second: a smaller problem at
    # split 2, so stale partials of the first call would show if the second read any of them
    for shape, split in (((8, 512, 7, 7, 512), 8), ((2, 128, 14, 14, 48), 2), ((2, 64, 14, 14, 32), 1)):
        p = _problem(*shape, prec)
        b = Bundle(p, 0x0A11C + split, O.NORMAL)
        ci = _config_for(p.geom(p.in_channels))
        print(f"no-alloc slab {shape} {prec} split {split} config {ci}", flush=True)
        ref = _with_buffer(p, b, ci, split)
        got = _no_alloc(p, b, ci, split)
        assert np.array_equal(np.nan_to_num(ref), np.nan_to_num(got)), f"{shape} split {split}: outputs differ"
        m = b.compare(got)
        assert m.passed(), f"{shape} split {split}: {m.summary()}"


def test_no_alloc_rejects_partials_beyond_scratch():
    h = gie.hip()
    cap = h.gie_hip_slab_scratch_floats()
    assert cap == 8 << 20
    # 32 x 256 x 14 x 14 outputs = 1.6M floats per split: split 8 needs 12.8M floats, more than the scratch
    p = _problem(32, 256, 14, 14, 256, "fp16")
    g = p.geom(256)
    ci = _config_for(g)
    d = gie.DeviceBuffer(1 << 20)
    rc = h.gie_hip_conv_slab_noalloc(ci, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, 8, None)
    assert rc == -3, rc
    assert b"scratch" in h.gie_hip_status_string(rc)
