"""GPU parity of the channel-blocked kernels through the C-ABI against the CPU oracle.

* gie_hip_repack_blocked / gie_hip_repack_w_blocked: bit-exact against the oracle's restatement of the
  reference's transpose_c_hw (src/kernels/tensor_core_mma.cu:61-82,309-310) with the channel index split into
  32-channel slices (xb[b][s][p][l] = x[b][32s + l][p], zero past C), including 2-byte-aligned sources;
* gie_hip_conv_band: every registered band configuration, with 8-byte and 2-byte activation loads (an x pointer
  offset by 2 bytes takes the 2-byte path), the row-shift and per-tap forms, fused epilogue and split-K partials
  + gie_hip_splitk_reduce, against the reference's per-element tolerance (tests/conv_test_common.h:83-127);
* the BASELINE configs 2 and 5 at full size through the plan API for the best kernel of each family, against the
  oracle with the benchmark gates (rel-L2 <= 1e-3, max-abs <= 2e-2).
"""
import ctypes

import numpy as np
import pytest

import gie
import oracle as O
from gpu_helpers import BENCH_CONFIGS, SHAPES, Bundle, problem, run_plan

pytestmark = pytest.mark.gpu


def _bits(n, seed):
    return np.random.default_rng(seed).integers(0, 65536, size=n, dtype=np.uint64).astype(np.uint16)


def _blocked(bits, n, C, RS):
    """[n][C][RS] -> [n][S][RS][32], zero channels past C (the oracle's repack, then a slice split)."""
    S = (C + 31) // 32
    nhwc = O.repack_c_hw(bits, n, C, RS, 32 * S).reshape(n, RS, S, 32)
    return np.ascontiguousarray(nhwc.transpose(0, 2, 1, 3)).ravel()


def _geom(p):
    return p.geom((p.in_channels + 31) // 32 * 32)


REPACK_CASES = [(SHAPES[6], 0), (SHAPES[14], 2), (SHAPES[17], 0), (SHAPES[12], 2), (SHAPES[3], 0), (SHAPES[10], 2)]


@pytest.mark.parametrize("shape,offset", REPACK_CASES, ids=[f"{s[0]}-off{o}" for s, o in REPACK_CASES])
def test_repack_blocked_bit_exact(shape, offset):
    p = problem(shape, "fp16", True, False)
    S = (p.in_channels + 31) // 32
    hw, rs = p.in_h * p.in_w, p.kernel_h * p.kernel_w
    x = _bits(int(np.prod(p.x_shape())), 3)
    w = _bits(int(np.prod(p.w_shape())), 4)
    dx, dw = gie.DeviceBuffer(x.nbytes + 16), gie.DeviceBuffer(w.nbytes + 16)
    dx.upload(x, offset=offset)
    dw.upload(w, offset=offset)
    nx, nw = p.batch * S * hw * 32, p.out_channels * S * rs * 32
    dxb, dwb = gie.DeviceBuffer(nx * 2), gie.DeviceBuffer(nw * 2)
    dxb.fill(0xAB)
    dwb.fill(0xCD)
    g = _geom(p)
    gie.check_hip(gie.hip().gie_hip_repack_blocked(dx.addr + offset, dxb.addr, dw.addr + offset, dwb.addr,
                                                   ctypes.byref(g), None), "repack_blocked")
    gie.synchronize()
    assert np.array_equal(dxb.download(np.uint16, nx), _blocked(x, p.batch, p.in_channels, hw))
    assert np.array_equal(dwb.download(np.uint16, nw), _blocked(w, p.out_channels, p.in_channels, rs))
    # weights alone: same bytes
    dwb.fill(0xEF)
    gie.check_hip(gie.hip().gie_hip_repack_w_blocked(dw.addr + offset, dwb.addr, ctypes.byref(g), None),
                  "repack_w_blocked")
    gie.synchronize()
    assert np.array_equal(dwb.download(np.uint16, nw), _blocked(w, p.out_channels, p.in_channels, rs))


def test_repack_blocked_rejects_bad_arguments():
    p = problem(SHAPES[6], "fp16", False, False)
    g = _geom(p)
    d = gie.DeviceBuffer(1 << 20)
    assert gie.hip().gie_hip_repack_w_blocked(d.addr, d.addr + 8, ctypes.byref(g), None) == -1  # wb unaligned
    assert gie.hip().gie_hip_repack_w_blocked(None, d.addr, ctypes.byref(g), None) == -1
    assert gie.hip().gie_hip_repack_blocked(None, d.addr, d.addr, d.addr, ctypes.byref(g), None) == -1


BAND_CASES = [
    # (shape, precision, bias, relu, split, x byte offset)
    (SHAPES[6], "fp16", True, True, 1, 0),    # 14x14: row shifts, 8-byte loads
    (SHAPES[6], "bf16", True, False, 2, 2),   # 14x14: row shifts, 2-byte loads, split-K
    (SHAPES[10], "bf16", True, True, 4, 0),   # 7x7, 512 channels: per-tap reads, 2-byte loads (H*W odd)
    (SHAPES[14], "fp16", False, True, 1, 0),  # C=130: partial last slice, 9x9
    (SHAPES[11], "fp16", True, True, 1, 0),   # 16x16, B=32: per-tap reads, two bands (NG=7)
    (SHAPES[3], "bf16", True, True, 1, 2),    # C=3, 32x32: five bands of 7 rows
    (SHAPES[0], "fp16", True, False, 1, 0),   # 5x5 no padding, one channel, one output channel
    (SHAPES[19], "fp16", True, True, 1, 0),   # 4x4 images, B=8
]


@pytest.mark.parametrize("case", BAND_CASES, ids=lambda c: f"{c[0][0]}-{c[1]}-sk{c[4]}-off{c[5]}")
def test_band_kernel_through_cabi(case):
    shape, prec, bias, relu, split, xoff = case
    p = problem(shape, prec, bias, relu)
    b = Bundle(p, 0xBA5D + split + xoff, O.NORMAL)
    g = _geom(p)
    S = (p.in_channels + 31) // 32
    rs = p.kernel_h * p.kernel_w
    dt = gie.PRECISIONS[prec]
    ny = int(np.prod(p.y_shape()))
    wb = gie.DeviceBuffer(p.out_channels * S * rs * 64)
    gie.check_hip(gie.hip().gie_hip_repack_w_blocked(b.t.dw.addr, wb.addr, ctypes.byref(g), None), "repack w")
    x = b.t.dx.addr
    xs = None
    if xoff:
        xs = gie.DeviceBuffer(b.t.dx.nbytes + 16)
        gie.check(gie.capi().gie_memcpy_d2d_async(xs.addr + xoff, b.t.dx.addr, b.t.dx.nbytes, None))
        x = xs.addr + xoff
    ran = 0
    for ci in range(gie.hip().gie_hip_band_config_count()):
        lds = ctypes.c_int(0)
        if gie.hip().gie_hip_band_check(ci, ctypes.byref(g), ctypes.byref(lds)) != 0:
            continue
        if split > S:
            continue
        ran += 1
        b.t.poison()
        part = gie.DeviceBuffer(split * ny * 4) if split > 1 else None
        gie.check_hip(gie.hip().gie_hip_conv_band(ci, dt, ctypes.byref(g), x, wb.addr, b.t.bias_addr(),
                                                  b.t.dy.addr, part.addr if part else None, split, None),
                      f"conv_band config {ci}")
        if split > 1:
            gie.check_hip(gie.hip().gie_hip_splitk_reduce(dt, part.addr, b.t.bias_addr(), b.t.dy.addr, ny, split,
                                                          p.out_channels, p.out_h * p.out_w, int(relu), None),
                          "reduce")
        gie.synchronize()
        m = b.compare(b.t.y())
        assert m.passed(), f"config {ci} {gie.band_configs()[ci]}: {m.summary()}"
    assert ran > 0, f"no band configuration accepts {shape[0]}"


def test_band_rejects_bad_arguments():
    p = problem(SHAPES[6], "fp16", False, False)
    g = _geom(p)
    d = gie.DeviceBuffer(1 << 22)
    h = gie.hip()
    assert h.gie_hip_conv_band(0, 1, ctypes.byref(g), d.addr + 1, d.addr, None, d.addr, None, 1, None) == -1
    assert h.gie_hip_conv_band(0, 1, ctypes.byref(g), d.addr, d.addr + 8, None, d.addr, None, 1, None) == -1
    assert h.gie_hip_conv_band(0, 1, ctypes.byref(g), d.addr, d.addr, None, None, None, 1, None) == -1
    assert h.gie_hip_conv_band(0, 0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 1, None) != 0  # fp32
    assert h.gie_hip_conv_band(99, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 1, None) == -1
    q = problem(SHAPES[7], "fp16", False, False)  # 1x1 filter: no 1x1 band configuration
    gq = _geom(q)
    for ci in range(h.gie_hip_band_config_count()):
        assert h.gie_hip_band_check(ci, ctypes.byref(gq), None) != 0


@pytest.mark.parametrize("cfg", ["c2_fp16_3x3", "c5_bf16_3x3_splitk"])
@pytest.mark.parametrize("family", ["band_", "halo_"])
def test_bench_config_full_size(cfg, family):
    c = dict(BENCH_CONFIGS[cfg])
    prec = c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    b = Bundle(p, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)
    picks = [k for k in gie.registry() if k.startswith(family) and gie.kernel_supports(k, p)[0]]
    assert picks, f"no {family} kernel runs {cfg}"
    for k in picks[:4]:
        y, why = run_plan(k, b)
        m = b.compare(y)
        gates = b.gates(y)
        assert m.passed(), f"{k}: {m.summary()}"
        assert gates["rel_l2"] <= 1e-3 and gates["max_abs"] <= 2e-2, f"{k}: {gates}"
