"""GPU parity of the stand-alone bias / ReLU pass (gie_hip_bias_act, the reference's src/kernels/elementwise.cu:13-56).

y[i] = round(relu?(f32(y[i]) + f32(bias[(i / hw_out) % out_channels]))) is one float32 add, an optional max with 0
and one round-to-nearest-even to the storage type, so the result is bit-exact against numpy's float32 add and
the oracle's rounding (compared as values, so -0 and +0 are equal). Cases cover the 16-byte chunk path and the
element path (2-byte-offset output, element count not a multiple of the chunk), channel changes inside one
chunk (hw_out 1 and 3), bias only, ReLU only, and fp32/fp16/bf16.
"""
import ctypes

import numpy as np
import pytest

import gie
import oracle as O

pytestmark = pytest.mark.gpu

CASES = [
    # (precision, batch, channels, hw, bias, relu, byte offset of y)
    ("fp16", 2, 8, 49, True, True, 0),
    ("bf16", 3, 5, 7, True, False, 0),
    ("fp32", 2, 6, 9, False, True, 0),
    ("fp16", 1, 37, 1, True, True, 2),
    ("bf16", 4, 16, 3, True, True, 2),
    ("fp32", 1, 11, 13, True, True, 4),
    ("fp16", 32, 64, 196, True, True, 0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}x{c[3]}-b{int(c[4])}r{int(c[5])}-off{c[6]}")
def test_bias_act_bit_exact(case):
    prec, B, C, HW, has_bias, relu, off = case
    rng = np.random.default_rng(B * 1000 + C * 10 + HW)
    n = B * C * HW
    y = O.quantize(prec, rng.uniform(-2, 2, n).astype(np.float32))
    b = O.quantize(prec, rng.uniform(-1, 1, C).astype(np.float32))
    esz = 4 if prec == "fp32" else 2
    dy = gie.DeviceBuffer(n * esz + 16)
    dy.upload(gie.host_to_storage(y, prec), offset=off)
    db = gie.to_device(gie.host_to_storage(b, prec)) if has_bias else None
    gie.check_hip(gie.hip().gie_hip_bias_act(gie.PRECISIONS[prec], dy.addr + off, db.addr if db else None, n, C, HW,
                                             int(relu), None), "bias_act")
    gie.synchronize()
    raw = dy.download(np.uint8, n * esz, offset=off)
    got = gie.storage_to_float(raw.view(np.uint32 if esz == 4 else np.uint16), prec)
    want = y.astype(np.float32)
    if has_bias:
        want = want + np.repeat(np.tile(b, B), HW)
    if relu:
        want = np.maximum(want, np.float32(0))
    want = O.quantize(prec, want)
    assert np.array_equal(got, want)


def test_bias_act_rejects_bad_arguments():
    d = gie.DeviceBuffer(1024)
    h = gie.hip()
    assert h.gie_hip_bias_act(1, None, d.addr, 16, 2, 8, 1, None) == -1
    assert h.gie_hip_bias_act(1, d.addr + 1, None, 16, 2, 8, 1, None) == -1   # odd address for 2-byte storage
    assert h.gie_hip_bias_act(0, d.addr + 2, None, 16, 2, 8, 1, None) == -1   # fp32 needs 4-byte alignment
    assert h.gie_hip_bias_act(1, d.addr, None, 0, 2, 8, 1, None) == -1
    assert h.gie_hip_bias_act(7, d.addr, None, 16, 2, 8, 1, None) == -2
    assert h.gie_hip_bias_act(1, d.addr, None, 16, 2, 8, 0, None) == 0         # nothing to do
