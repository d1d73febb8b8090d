"""GPU parity of the pointwise (1x1) kernel, which reads x as NCHW and w as [out][in] with no repack.

* gie_hip_conv_pw through the C-ABI against the oracle's double reference (tests/conv_test_common.h:83-127
  tolerance) on 1x1 shapes with C % 8 == 0 and H*W % 8 == 0: ragged pixel tiles (H*W not a multiple of 128),
  output channels not a multiple of 128, one slice and many, fp16 and bf16, with and without bias/ReLU;
* gie_hip_conv_pws (weights held in registers, streamed 32-pixel blocks) on the same kind of shapes: blocks that
  straddle two images (H*W not a multiple of 32), the three reduction depths (C <= 64, <= 128, <= 256), filters
  past a 256-filter block, one workgroup with a single block, many pixel ranges;
* its geometry checks and argument rejection (stride, padding, channel and pixel divisibility, alignment);
* the plan API with 2-byte-offset caller tensors (the registry entry runs the implicit-GEMM entry instead);
* BASELINE config 3 (N64 C256 28x28 K1024) at full size against the oracle (sampled outputs) with the
  benchmark gates.
"""
import ctypes

import numpy as np
import pytest

import gie
import oracle as O
from gpu_helpers import BENCH_CONFIGS, Bundle, run_plan

pytestmark = pytest.mark.gpu

PW_CASES = [
    # (B, C, H, W, O, precision, bias, relu)
    (2, 32, 8, 8, 40, "fp16", True, True),
    (3, 72, 16, 12, 130, "bf16", True, False),
    (1, 64, 56, 56, 64, "fp16", False, True),
    (4, 256, 7, 8, 96, "fp16", True, True),
    (2, 8, 4, 6, 8, "bf16", True, True),
    (1, 520, 10, 12, 300, "fp16", True, False),
]


def _problem(B, C, H, W, O_, prec, bias, relu):
    return gie.Problem(B, C, H, W, O_, 1, 1, 1, 1, 0, 0, precision=prec, has_bias=bias, relu=relu)


@pytest.mark.parametrize("case", PW_CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"-{c[5]}")
def test_pointwise_kernel_through_cabi(case):
    p = _problem(*case)
    b = Bundle(p, 0x9A7 + case[1], O.NORMAL)
    g = p.geom(p.in_channels)
    lds = ctypes.c_int(0)
    assert gie.hip().gie_hip_pw_check(ctypes.byref(g), ctypes.byref(lds)) == 0
    assert lds.value == 64 * 1024
    b.t.poison()
    gie.check_hip(gie.hip().gie_hip_conv_pw(gie.PRECISIONS[case[5]], ctypes.byref(g), b.t.dx.addr, b.t.dw.addr,
                                            b.t.bias_addr(), b.t.dy.addr, None), "conv_pw")
    gie.synchronize()
    m = b.compare(b.t.y())
    assert m.passed(), m.summary()


PWS_CASES = [
    # (B, C, H, W, O, precision, bias, relu)
    (2, 32, 8, 8, 40, "fp16", True, True),        # C <= 64, 4 blocks, one range each
    (3, 72, 16, 12, 130, "bf16", True, False),    # C <= 128, O past one 128-half
    (4, 256, 7, 8, 96, "fp16", True, True),       # 56-pixel images: every other block straddles two images
    (1, 8, 2, 4, 8, "bf16", False, True),         # one 8-pixel block, one filter block of 8
    (64, 256, 28, 28, 300, "fp16", True, True),   # many ranges, 784-pixel images, O over two 256-blocks
    (5, 200, 6, 8, 513, "bf16", True, True),      # 48-pixel images, C padded to 256, three filter blocks
    (2, 128, 16, 16, 256, "fp16", False, False),  # no epilogue
    (2, 32, 4, 4, 40, "fp16", True, True),        # 16-pixel images: four images per block (per-lane division)
    (3, 8, 2, 4, 8, "bf16", False, False),        # 8-pixel images, one block for all
]


@pytest.mark.parametrize("case", PWS_CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"-{c[5]}")
def test_pointwise_streaming_kernel_through_cabi(case):
    p = _problem(*case)
    b = Bundle(p, 0x57A + case[1] + case[4], O.NORMAL)
    g = p.geom(p.in_channels)
    lds = ctypes.c_int(0)
    assert gie.hip().gie_hip_pws_check(ctypes.byref(g), ctypes.byref(lds)) == 0
    # a three-stage ring + two 8 KiB output tiles per filter group
    assert lds.value in (3 * 8192 + 65536, 3 * 16384 + 65536, 3 * 32768 + 65536)
    for rep in range(2):  # the second launch overwrites the first's output with the same bits
        b.t.poison()
        gie.check_hip(gie.hip().gie_hip_conv_pws(gie.PRECISIONS[case[5]], ctypes.byref(g), b.t.dx.addr,
                                                 b.t.dw.addr, b.t.bias_addr(), b.t.dy.addr, None), "conv_pws")
        gie.synchronize()
        y = b.t.y()
        m = b.compare(y)
        assert m.passed(), m.summary()
        if rep == 0:
            first = y.copy()
        else:
            assert np.array_equal(np.nan_to_num(first), np.nan_to_num(y))


def test_pointwise_streaming_rejections():
    h = gie.hip()
    big = _problem(2, 264, 8, 8, 40, "fp16", True, True)  # C > 256: weights do not fit the registers
    assert h.gie_hip_pws_check(ctypes.byref(big.geom(big.in_channels)), None) != 0
    assert h.gie_hip_pw_check(ctypes.byref(big.geom(big.in_channels)), None) == 0  # the tiled form takes it
    ok = _problem(2, 32, 8, 8, 40, "fp16", True, True)
    g = ok.geom(ok.in_channels)
    d = gie.DeviceBuffer(1 << 20)
    assert h.gie_hip_conv_pws(1, ctypes.byref(g), d.addr + 8, d.addr, None, d.addr, None) != 0  # x 8-B aligned
    assert h.gie_hip_conv_pws(1, ctypes.byref(g), d.addr, d.addr, None, d.addr + 4, None) != 0  # y 4-B aligned
    assert h.gie_hip_conv_pws(0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None) != 0      # fp32
    assert h.gie_hip_conv_pws(1, ctypes.byref(g), None, d.addr, None, d.addr, None) == -1


def test_pointwise_geometry_and_argument_checks():
    h = gie.hip()
    ok = _problem(2, 32, 8, 8, 40, "fp16", True, True)
    for bad in (gie.Problem(2, 32, 8, 8, 40, 3, 3, 1, 1, 1, 1, precision="fp16"),   # 3x3 filter
                gie.Problem(2, 32, 8, 8, 40, 1, 1, 2, 2, 0, 0, precision="fp16"),   # stride 2
                gie.Problem(2, 32, 8, 8, 40, 1, 1, 1, 1, 1, 1, precision="fp16"),   # padding
                _problem(2, 30, 8, 8, 40, "fp16", True, True),                      # C % 8 != 0
                _problem(2, 32, 5, 5, 40, "fp16", True, True)):                     # H*W % 8 != 0
        g = bad.geom(bad.in_channels)
        assert h.gie_hip_pw_check(ctypes.byref(g), None) != 0
    g = ok.geom(ok.in_channels)
    d = gie.DeviceBuffer(1 << 20)
    assert h.gie_hip_conv_pw(1, ctypes.byref(g), d.addr + 2, d.addr, None, d.addr, None) != 0  # unaligned x
    assert h.gie_hip_conv_pw(1, ctypes.byref(g), d.addr, d.addr, None, d.addr + 8, None) != 0  # unaligned y
    assert h.gie_hip_conv_pw(0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None) != 0      # fp32
    assert h.gie_hip_conv_pw(1, ctypes.byref(g), None, d.addr, None, d.addr, None) == -1


@pytest.mark.parametrize("form", ["128x128x32_s4_sk1", "256x64x16_s4_wreg"])
@pytest.mark.parametrize("prec", ["fp16", "bf16"])
def test_pointwise_entry_with_unaligned_caller_tensors(prec, form):
    """The registry entries take 2-byte-aligned tensors by running the implicit-GEMM entry of their precision."""
    p = _problem(2, 64, 8, 16, 72, prec, True, True)
    b = Bundle(p, 0x55, O.UNIFORM)
    k = f"pw_{prec}_1x1_{form}"
    assert gie.kernel_supports(k, p)[0]
    plan = gie.Plan(p, k)
    ws = gie.DeviceBuffer(plan.workspace_bytes) if plan.workspace_bytes else None
    # shifted copies of x, w and y
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


def test_bench_config3_full_size():
    c = dict(BENCH_CONFIGS["c3_fp16_1x1"])
    prec = c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    b = Bundle(p, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)  # the oracle on every output
    for k in ("pw_fp16_1x1_256x64x16_s4_wreg", "pw_fp16_1x1_128x128x32_s4_sk1"):
        y, why = run_plan(k, b)
        assert y is not None, why
        m = b.compare(y)
        gates = b.gates(y)
        assert m.passed(), f"{k}: {m.summary()}"
        assert gates["rel_l2"] <= 1e-3 and gates["max_abs"] <= 2e-2, f"{k}: {gates}"
