"""GPU parity of the narrow kernel (conv_narrow.hip: 3x3, stride 1, padding 1, in_channels % 128 == 0, the whole
reduction in one workgroup) through its C-ABI and through the registry entries, against the oracle's double
reference under the reference's tolerance (tests/conv_test_common.h:83-127).

Cases cover pixel blocks inside one image (14x14), straddling two (7x7) or three (4x4) images and spanning 32 1x1
images, a partial last pixel block, filter counts below and past a 32-filter block, no bias / no ReLU, both
precisions, a second launch overwriting the first with the same bits, BASELINE config 5 (N8 C512 7x7 K512 BF16)
at full size with the benchmark gates, caller tensors that are only 2-byte aligned (the entry runs the
implicit-GEMM fallback) and argument rejection.
"""
import ctypes

import numpy as np
import pytest

import gie
import oracle as O
from gpu_helpers import BENCH_CONFIGS, Bundle, run_plan

pytestmark = pytest.mark.gpu


def _problem(B, C, H, W, K, prec, bias, relu):
    return gie.Problem(B, C, H, W, K, 3, 3, 1, 1, 1, 1, precision=prec, has_bias=bias, relu=relu)


CASES = [
    # (B, C, H, W, O, precision, bias, relu)
    (2, 128, 5, 5, 40, "fp16", True, True),       # blocks straddle images, O past one 32-filter block
    (3, 256, 4, 4, 64, "bf16", True, False),      # 16-pixel images: three images per block
    (1, 128, 14, 14, 96, "fp16", True, True),     # one image, partial last block
    (40, 128, 1, 1, 20, "bf16", False, True),     # 1x1 images: 32 images per block, O below a block
    (8, 512, 7, 7, 512, "bf16", True, True),      # config 5 shape
    (2, 384, 6, 6, 33, "fp16", False, False),     # no epilogue, O = 33
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"-{c[5]}")
def test_narrow_kernel_through_cabi(case):
    p = _problem(*case)
    b = Bundle(p, 0x4A7 + case[1] + case[4], O.NORMAL)
    g = p.geom(p.in_channels)
    lds = ctypes.c_int(0)
    assert gie.hip().gie_hip_narrow_check(ctypes.byref(g), ctypes.byref(lds)) == 0
    assert 0 < lds.value <= 160 * 1024
    for rep in range(2):  # the second launch overwrites the first's output with the same bits
        b.t.poison()
        gie.check_hip(gie.hip().gie_hip_conv_narrow(gie.PRECISIONS[case[5]], ctypes.byref(g), b.t.dx.addr,
                                                    b.t.dw.addr, b.t.bias_addr(), b.t.dy.addr, None), "conv_narrow")
        gie.synchronize()
        y = b.t.y()
        m = b.compare(y)
        assert m.passed(), m.summary()
        if rep == 0:
            first = y.copy()
        else:
            assert np.array_equal(np.nan_to_num(first), np.nan_to_num(y))


def test_narrow_geometry_and_argument_checks():
    h = gie.hip()
    for bad in (gie.Problem(2, 128, 7, 7, 64, 5, 5, 1, 1, 2, 2, precision="fp16"),   # 5x5 filter
                gie.Problem(2, 128, 7, 7, 64, 3, 3, 2, 2, 1, 1, precision="fp16"),   # stride 2
                gie.Problem(2, 128, 7, 7, 64, 3, 3, 1, 1, 0, 0, precision="fp16"),   # no padding
                _problem(2, 96, 7, 7, 64, "fp16", True, True),                      # C % 128 != 0
                _problem(2, 1024, 56, 56, 64, "fp16", True, True)):                 # images too large for LDS
        assert h.gie_hip_narrow_check(ctypes.byref(bad.geom(bad.in_channels)), None) != 0
    ok = _problem(2, 128, 7, 7, 64, "fp16", True, True)
    g = ok.geom(ok.in_channels)
    d = gie.DeviceBuffer(1 << 22)
    assert h.gie_hip_conv_narrow(1, ctypes.byref(g), d.addr + 8, d.addr, None, d.addr, None) != 0   # x 8-B aligned
    assert h.gie_hip_conv_narrow(1, ctypes.byref(g), d.addr, d.addr + 8, None, d.addr, None) != 0   # w 8-B aligned
    assert h.gie_hip_conv_narrow(1, ctypes.byref(g), d.addr, d.addr, None, d.addr + 1, None) == -1  # odd y
    assert h.gie_hip_conv_narrow(0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None) != 0       # fp32
    assert h.gie_hip_conv_narrow(1, ctypes.byref(g), None, d.addr, None, d.addr, None) == -1


@pytest.mark.parametrize("prec", ["fp16", "bf16"])
def test_narrow_entry_with_unaligned_caller_tensors(prec):
    """The registry entry takes 2-byte-aligned tensors by running the implicit-GEMM entry of its precision."""
    p = _problem(2, 128, 7, 7, 64, prec, True, True)
    b = Bundle(p, 0x4E, O.UNIFORM)
    k = f"narrow_{prec}_3x3_32x32x16_k8w"
    assert gie.kernel_supports(k, p)[0]
    y, why = run_plan(k, b)
    assert y is not None, why
    assert b.compare(y).passed()
    plan = gie.Plan(p, k)
    ws = gie.DeviceBuffer(plan.workspace_bytes) if plan.workspace_bytes else None
    bufs = {n: gie.DeviceBuffer(getattr(b.t, n).nbytes + 16) for n in ("dx", "dw", "dy")}
    for n in ("dx", "dw"):
        gie.check(gie.capi().gie_memcpy_d2d_async(bufs[n].addr + 2, getattr(b.t, n).addr, getattr(b.t, n).nbytes, None))
    gie.synchronize()
    gie.check(gie.capi().gie_plan_execute_unchecked(plan.h, bufs["dx"].addr + 2, bufs["dw"].addr + 2, b.t.bias_addr(),
                                                    bufs["dy"].addr + 2, ws.addr if ws else None,
                                                    ws.nbytes if ws else 0, None), "execute")
    gie.synchronize()
    raw = np.frombuffer(bufs["dy"].download(np.uint8, b.t.dy.nbytes + 2)[2:].tobytes(), np.uint16)
    m = b.compare(gie.storage_to_float(raw, prec))
    assert m.passed(), m.summary()


def test_bench_config5_full_size():
    c = dict(BENCH_CONFIGS["c5_bf16_3x3_splitk"])
    prec = c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    b = Bundle(p, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)
    k = "narrow_bf16_3x3_32x32x16_k8w"
    y, why = run_plan(k, b)
    assert y is not None, why
    m = b.compare(y)
    gates = b.gates(y)
    assert m.passed(), f"{k}: {m.summary()}"
    assert gates["rel_l2"] <= 1e-3 and gates["max_abs"] <= 2e-2, f"{k}: {gates}"
