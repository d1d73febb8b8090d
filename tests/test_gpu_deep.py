"""GPU parity of the deep kernel (conv_deep.hip: 3x3, stride 1, padding 1 over small images with a long reduction,
one workgroup per (16-filter block, image) summing the whole reduction, straight from NCHW x and OIHW w) through its
C-ABI, against the oracle's double reference under the reference's tolerance (tests/conv_test_common.h:83-127)
and, at BASELINE size, the benchmark gates.

Cases cover image sizes 1x1 to 8x7 (rows of odd width starting at either 2-byte parity, so the row loads shift by
one element), one to four steps of 128 channels, filter counts past and below a 16-filter block, batch 1 and
several images, no bias / no ReLU, both precisions, an x offset by 4 bytes, a second launch giving the same bits,
config 5 at full size, and argument rejection.
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


def _run(p, b, xoff=0, reps=1):
    """One deep launch through the C-ABI per repetition; returns the outputs as floats."""
    g = p.geom(p.in_channels)
    dt = gie.PRECISIONS[p.precision]
    x = b.t.dx.addr
    keep = []
    if xoff:
        xs = gie.DeviceBuffer(b.t.dx.nbytes + 16)
        gie.check(gie.capi().gie_memcpy_d2d_async(xs.addr + xoff, b.t.dx.addr, b.t.dx.nbytes, None))
        x = xs.addr + xoff
        keep.append(xs)
    outs = []
    for _ in range(reps):
        b.t.poison()
        gie.check_hip(gie.hip().gie_hip_conv_deep(dt, ctypes.byref(g), x, b.t.dw.addr, b.t.bias_addr(), b.t.dy.addr,
                                                  None), "conv_deep")
        gie.synchronize()
        outs.append(b.t.y())
    return outs


CASES = [  # (B, C, H, W, K, precision, bias, relu, x offset)
    (1, 128, 7, 7, 16, "fp16", True, True, 0),
    (2, 256, 7, 7, 48, "bf16", True, True, 0),
    (3, 128, 8, 7, 20, "fp16", True, False, 4),
    (1, 384, 5, 6, 33, "bf16", False, True, 0),
    (4, 128, 3, 3, 64, "fp16", True, True, 0),
    (2, 512, 4, 5, 40, "bf16", True, True, 4),
    (1, 128, 1, 1, 7, "fp16", True, True, 0),
    (5, 256, 6, 7, 31, "fp16", False, False, 0),
    (2, 128, 8, 6, 16, "bf16", True, True, 0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"-{c[5]}-b{int(c[6])}r{int(c[7])}"
                                                      f"-o{c[8]}")
def test_deep_kernel_through_cabi(case):
    B, C, H, W, K, prec, bias, relu, xoff = case
    p = _problem(B, C, H, W, K, prec, bias, relu)
    g = p.geom(p.in_channels)
    lds = ctypes.c_int(0)
    assert gie.hip().gie_hip_deep_check(ctypes.byref(g), ctypes.byref(lds)) == 0
    assert 0 < lds.value <= 160 * 1024
    b = Bundle(p, 4242 + C + K, O.NORMAL)
    print(f"deep kernel on {case}", flush=True)
    first, second = _run(p, b, xoff, reps=2)
    m = b.compare(first)
    assert m.passed(), m.summary()
    assert np.array_equal(np.nan_to_num(first), np.nan_to_num(second)), "second launch differs"


@pytest.mark.parametrize("prec", ["bf16", "fp16"])
def test_deep_bench_config_full_size(prec):
    c = dict(BENCH_CONFIGS["c5_bf16_3x3_splitk"])
    c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    b = Bundle(p, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)
    print(f"deep kernel on config 5 ({prec})", flush=True)
    (y,) = _run(p, b)
    m = b.compare(y)
    gates = b.gates(y)
    assert m.passed(), m.summary()
    assert gates["rel_l2"] <= 1e-3 and gates["max_abs"] <= 2e-2, gates


def test_deep_argument_checks():
    h = gie.hip()
    ok = _problem(2, 128, 7, 7, 64, "fp16")
    g = ok.geom(128)
    d = gie.DeviceBuffer(1 << 22)
    assert h.gie_hip_conv_deep(1, ctypes.byref(g), d.addr, d.addr + 8, None, d.addr, None) == -2   # w not 16-aligned
    assert h.gie_hip_conv_deep(1, ctypes.byref(g), d.addr + 2, d.addr, None, d.addr, None) == -2   # x not 4-aligned
    assert h.gie_hip_conv_deep(1, ctypes.byref(g), d.addr, d.addr, None, d.addr + 1, None) == -1   # odd y
    assert h.gie_hip_conv_deep(0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None) == -2       # fp32
    assert h.gie_hip_conv_deep(1, ctypes.byref(g), None, d.addr, None, d.addr, None) == -1
    for bad in (_problem(1, 96, 7, 7, 16, "fp16"), _problem(1, 128, 9, 7, 16, "fp16"),
                _problem(1, 128, 7, 8, 16, "fp16"), gie.Problem(1, 128, 7, 7, 16, 3, 3, 2, 2, 1, 1,
                                                                precision="fp16")):
        gb = bad.geom(bad.in_channels)
        assert h.gie_hip_deep_check(ctypes.byref(gb), None) == -2


def test_dispatcher_routes_config5_to_the_deep_entry():
    """The cost model alone (no tuning) picks the deep entry, measured fastest for BASELINE config 5."""
    c = dict(BENCH_CONFIGS["c5_bf16_3x3_splitk"])
    prec = c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    k, src, _ = gie.select(p)
    assert k == "deep_bf16_3x3_16x8r8_k32x4_ld" and src == "cost_model", (k, src)
