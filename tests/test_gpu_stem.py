"""GPU parity of the stem kernel (conv_stem.hip: 7x7 filter, stride 2, padding 3, in_channels <= 4, straight from
NCHW) through its C-ABI and through the registry entries, against the oracle's double reference under the
reference's tolerance (tests/conv_test_common.h:83-127).

Cases cover every channel count 1..4, filter counts below, at and over one 64-filter group, odd output heights
(the last 2-row tile holds one valid row), widths from 16 to the widest that fit (336 with 4 channels, 512), fewer tiles than workgroups, no bias / no ReLU, both precisions, a second launch overwriting the first
with the same bits, BASELINE config 4 (N64 C3 224x224 K64) at full size (sampled outputs + the benchmark gates),
caller tensors that are only 2-byte aligned (the entry runs the implicit-GEMM fallback) and argument rejection.
"""
import ctypes

import numpy as np
import pytest

import gie
import oracle as O
from gpu_helpers import BENCH_CONFIGS, Bundle, run_plan

pytestmark = pytest.mark.gpu


def _problem(B, C, H, W, K, prec, bias, relu):
    return gie.Problem(B, C, H, W, K, 7, 7, 2, 2, 3, 3, precision=prec, has_bias=bias, relu=relu)


CASES = [
    # (B, C, H, W, O, precision, bias, relu)
    (2, 3, 32, 32, 64, "fp16", True, True),       # one filter group, 2-row tiles
    (1, 1, 16, 16, 20, "bf16", True, False),      # C = 1, filters below one group
    (3, 2, 17, 32, 70, "fp16", True, True),       # C = 2, odd output height, two filter groups
    (2, 4, 40, 48, 128, "bf16", False, True),     # C = 4, no bias
    (1, 3, 9, 16, 64, "fp16", True, True),        # smallest width: out_w 8, three tiles only
    (1, 4, 6, 304, 64, "fp16", True, True),       # widest C = 4 rows with 4-row tiles in LDS (304 columns)
    (1, 4, 6, 464, 64, "fp16", True, True),       # widest C = 4 rows that fit LDS (464 columns, 2-row tiles)
    (2, 4, 9, 464, 64, "bf16", True, True),       # the same in BF16 with ReLU (2-row tiles always)
    (1, 3, 4, 512, 64, "bf16", True, True),       # widest rows (512 columns)
    (4, 3, 64, 64, 32, "bf16", True, True),       # filter count 32
    (2, 3, 30, 48, 64, "fp16", False, False),     # no epilogue
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"-{c[5]}")
def test_stem_kernel_through_cabi(case):
    p = _problem(*case)
    b = Bundle(p, 0x57E + case[1] * 7 + case[4], O.NORMAL)
    g = p.geom(p.in_channels)
    lds = ctypes.c_int(0)
    assert gie.hip().gie_hip_stem_check(ctypes.byref(g), ctypes.byref(lds)) == 0
    assert 0 < lds.value <= 160 * 1024
    for rep in range(2):  # the second launch overwrites the first's output with the same bits
        b.t.poison()
        gie.check_hip(gie.hip().gie_hip_conv_stem(gie.PRECISIONS[case[5]], ctypes.byref(g), b.t.dx.addr,
                                                  b.t.dw.addr, b.t.bias_addr(), b.t.dy.addr, None), "conv_stem")
        gie.synchronize()
        y = b.t.y()
        m = b.compare(y)
        assert m.passed(), m.summary()
        if rep == 0:
            first = y.copy()
        else:
            assert np.array_equal(np.nan_to_num(first), np.nan_to_num(y))


def test_stem_geometry_and_argument_checks():
    h = gie.hip()
    for bad in (gie.Problem(2, 3, 32, 32, 64, 5, 5, 2, 2, 2, 2, precision="fp16"),   # 5x5 filter
                gie.Problem(2, 3, 32, 32, 64, 7, 7, 1, 1, 3, 3, precision="fp16"),   # stride 1
                gie.Problem(2, 3, 32, 32, 64, 7, 7, 2, 2, 2, 2, precision="fp16"),   # padding 2
                _problem(2, 5, 32, 32, 64, "fp16", True, True),                     # C = 5
                _problem(2, 3, 32, 40, 64, "fp16", True, True),                     # in_w % 16 != 0
                _problem(1, 4, 6, 480, 64, "fp16", True, True),                     # rows too wide for LDS
                _problem(1, 3, 6, 528, 64, "fp16", True, True)):                    # rows over 512 columns
        assert h.gie_hip_stem_check(ctypes.byref(bad.geom(bad.in_channels)), None) != 0
    ok = _problem(2, 3, 32, 32, 64, "fp16", True, True)
    g = ok.geom(ok.in_channels)
    d = gie.DeviceBuffer(1 << 20)
    assert h.gie_hip_conv_stem(1, ctypes.byref(g), d.addr + 8, d.addr, None, d.addr, None) != 0  # x 8-B aligned
    assert h.gie_hip_conv_stem(1, ctypes.byref(g), d.addr, d.addr, None, d.addr + 8, None) != 0  # y 8-B aligned
    assert h.gie_hip_conv_stem(1, ctypes.byref(g), d.addr, d.addr + 8, None, d.addr, None) != 0  # w 8-B aligned
    assert h.gie_hip_conv_stem(1, ctypes.byref(g), d.addr, d.addr, d.addr + 1, d.addr, None) == -1  # odd bias
    assert h.gie_hip_conv_stem(0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None) != 0      # fp32
    assert h.gie_hip_conv_stem(1, ctypes.byref(g), None, d.addr, None, d.addr, None) == -1


@pytest.mark.parametrize("prec", ["fp16", "bf16"])
def test_stem_entry_with_unaligned_caller_tensors(prec):
    """The registry entry takes 2-byte-aligned tensors by running the implicit-GEMM entry of its precision."""
    p = _problem(2, 3, 16, 16, 64, prec, True, True)
    b = Bundle(p, 0x5E, O.UNIFORM)
    k = f"stem_{prec}_7x7s2_64x32x16_wreg"
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


def test_bench_config4_full_size():
    c = dict(BENCH_CONFIGS["c4_fp16_7x7s2"])
    prec = c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    b = Bundle(p, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)  # the oracle on every output
    k = "stem_fp16_7x7s2_64x32x16_wreg"
    y, why = run_plan(k, b)
    assert y is not None, why
    m = b.compare(y)
    gates = b.gates(y)
    assert m.passed(), f"{k}: {m.summary()}"
    assert gates["rel_l2"] <= 1e-3 and gates["max_abs"] <= 2e-2, f"{k}: {gates}"


def test_dispatcher_routes_config4_to_the_stem_entry():
    """The cost model alone (no tuning) picks the stem entry for BASELINE config 4."""
    c = dict(BENCH_CONFIGS["c4_fp16_7x7s2"])
    prec = c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    k, src, _ = gie.select(p)
    assert k == "stem_fp16_7x7s2_64x32x16_wreg" and src == "cost_model", (k, src)
