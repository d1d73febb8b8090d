"""GPU parity of the slab kernel (conv_slab.hip: 3x3, stride 1, padding 1, straight from NCHW x and OIHW w, per-tap-
column accumulators combined by lane shifts) through its C-ABI, against the oracle's double reference under the
reference's tolerance (tests/conv_test_common.h:83-127) and, at BASELINE sizes, the benchmark gates.

Cases cover every registered configuration on slabs that are whole images and images cut into several slabs,
rows narrower than the pitch, channel counts that are not a multiple of the slice (zero-filled channels), filter
counts past and below a 32-filter block, each activation load form (4-byte direct-to-LDS loads of even rows of a
4-byte aligned x, 2-byte loads of odd rows or a 2-byte aligned x),
pixel-pair and 2-byte output stores, the split form's LDS-staged 16-byte output stores (whole images, O % 32 == 0,
16-byte aligned y) against its pixel-pair stores bit for bit, no bias / no ReLU, both precisions, split-K with the reduce kernel, a second launch giving the
same bits, and argument rejection.
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
    for i in range(gie.hip().gie_hip_slab_config_count()):
        c = gie.GieSlabConfig()
        gie.check_hip(gie.hip().gie_hip_slab_config_get(i, ctypes.byref(c)), "slab_config_get")
        out.append(c)
    return out


def _run(p, b, ci, split=1, xoff=0, yoff=0, reps=1):
    """One slab launch (plus the reduce for split > 1) through the C-ABI; returns the output as floats."""
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
    ybuf, y = b.t.dy, b.t.dy.addr
    if yoff:
        ybuf = gie.DeviceBuffer(b.t.dy.nbytes + 16)
        y = ybuf.addr + yoff
    part = gie.DeviceBuffer(split * ny * 4) if split > 1 else None
    outs = []
    for _ in range(reps):
        b.t.poison()
        if yoff:
            gie.check_hip(gie.hip().gie_hip_fill_u16(ybuf.addr, (b.t.dy.nbytes + 16) // 2, 0xFFFF, None), "fill")
        rc = gie.hip().gie_hip_conv_slab(ci, dt, ctypes.byref(g), x, b.t.dw.addr, b.t.bias_addr(), y,
                                         part.addr if part else None, split, None)
        if rc == -2 and (xoff or yoff):
            return None  # this configuration has no load form for that alignment (the registry entry falls back)
        gie.check_hip(rc, f"conv_slab {ci}")
        if split > 1:
            gie.check_hip(gie.hip().gie_hip_splitk_reduce(dt, part.addr, b.t.bias_addr(), y, ny, split,
                                                          p.out_channels, p.out_h * p.out_w, int(p.relu), None),
                          "reduce")
        gie.synchronize()
        if yoff:
            raw = np.frombuffer(ybuf.download(np.uint8, b.t.dy.nbytes + yoff)[yoff:].tobytes(), np.uint16)
            outs.append(gie.storage_to_float(raw, p.precision).reshape(p.y_shape()))
        else:
            outs.append(b.t.y())
    return outs


CASES = [
    # (B, C, H, W, O, precision, bias, relu, split, x offset, y offset)
    (2, 64, 14, 14, 32, "fp16", True, True, 1, 0, 0),     # whole-image slabs, one 64-channel slice
    (3, 128, 14, 14, 40, "bf16", True, False, 1, 0, 0),   # O past one filter block
    (2, 72, 13, 10, 20, "fp16", False, True, 1, 0, 0),    # C % 64 != 0, narrow rows, O below a block
    (2, 72, 13, 7, 20, "fp16", False, True, 1, 0, 0),     # odd rows: 2-byte register loads
    (1, 64, 29, 14, 32, "fp16", True, True, 1, 0, 0),     # three slabs, H*W % 4 != 0 (2-byte stores)
    (2, 64, 14, 14, 32, "bf16", True, True, 1, 0, 2),     # y offset by 2 bytes
    (2, 64, 7, 6, 32, "bf16", True, True, 1, 2, 0),       # x offset by 2 bytes: 2-byte register loads
    (2, 64, 14, 14, 32, "fp16", True, True, 1, 4, 0),     # x offset by 4 bytes: 4-byte direct loads
    (8, 512, 7, 7, 64, "bf16", True, True, 1, 0, 0),      # 7x7 images
    (4, 256, 7, 7, 96, "fp16", True, True, 2, 0, 0),      # split-K 2 + reduce
    (2, 512, 7, 7, 64, "bf16", True, True, 4, 0, 0),      # split-K 4 + reduce
    (2, 64, 28, 28, 48, "fp16", True, True, 1, 0, 0),     # 28-wide rows, several slabs
    (1, 32, 5, 3, 8, "bf16", False, False, 1, 0, 0),      # tiny: one slice of 32 real channels
    (2, 8, 6, 6, 5, "fp16", True, True, 1, 0, 0),         # C = 8
    (1, 32, 10, 10, 32, "fp16", True, True, 1, 0, 0),     # one slice: fewer slices than load stages
    (2, 96, 12, 14, 64, "bf16", True, True, 2, 0, 0),     # split-K 2 over 3 slices (ranges of 1 and 2)
    (3, 320, 14, 8, 72, "fp16", True, False, 1, 0, 0),    # 10 slices: a partial loop turn, O past two blocks
    (2, 96, 14, 12, 64, "bf16", True, False, 1, 0, 0),    # 3 slices (one loop turn short), no ReLU, two blocks
    (1, 160, 9, 10, 64, "fp16", False, True, 1, 0, 0),    # 5 slices, image shorter than the slab
    (2, 64, 14, 14, 32, "fp16", True, True, 1, 0, 8),     # y offset by 8 bytes: pixel-pair stores
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"-{c[5]}-sk{c[8]}-o{c[9]}{c[10]}")
def test_slab_kernel_through_cabi(case):
    B, C, H, W, K, prec, bias, relu, split, xoff, yoff = case
    p = _problem(B, C, H, W, K, prec, bias, relu)
    b = Bundle(p, 0x51AB + C + K + split, O.NORMAL)
    g = p.geom(p.in_channels)
    ran = 0
    for ci, cfg in enumerate(_configs()):
        lds = ctypes.c_int(0)
        if gie.hip().gie_hip_slab_check(ci, ctypes.byref(g), ctypes.byref(lds)) != 0:
            continue
        if split > (C + cfg.tile_k - 1) // cfg.tile_k:
            continue
        assert 0 < lds.value <= 160 * 1024
        print(f"slab config {ci} (pitch {cfg.pitch}, rows {cfg.rows}, k {cfg.tile_k}) on {case}", flush=True)
        outs = _run(p, b, ci, split, xoff, yoff, reps=2)
        if outs is None:
            continue
        first, second = outs
        m = b.compare(first)
        assert m.passed(), f"config {ci}: {m.summary()}"
        assert np.array_equal(np.nan_to_num(first), np.nan_to_num(second)), f"config {ci}: second launch differs"
        ran += 1
    assert ran > 0, f"no slab configuration accepts {case}"


@pytest.mark.parametrize("cfg_name", ["c2_fp16_3x3", "c5_bf16_3x3_splitk"])
def test_slab_bench_config_full_size(cfg_name):
    c = dict(BENCH_CONFIGS[cfg_name])
    prec = c.pop("precision")
    p = gie.Problem(**c, precision=prec, has_bias=True, relu=True)
    b = Bundle(p, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)
    g = p.geom(p.in_channels)
    ran = 0
    for ci, cfg in enumerate(_configs()):
        if gie.hip().gie_hip_slab_check(ci, ctypes.byref(g), None) != 0:
            continue
        for split in (1, 2, 4, 8):
            if split > (p.in_channels + cfg.tile_k - 1) // cfg.tile_k:
                continue
            print(f"slab config {ci} split {split} on {cfg_name}", flush=True)
            (y,) = _run(p, b, ci, split)
            m = b.compare(y)
            gates = b.gates(y)
            assert m.passed(), f"config {ci} sk{split}: {m.summary()}"
            assert gates["rel_l2"] <= 1e-3 and gates["max_abs"] <= 2e-2, f"config {ci} sk{split}: {gates}"
            ran += 1
    assert ran > 0


def _split_config():
    for ci, cfg in enumerate(_configs()):
        if cfg.threads == 512:
            return ci
    pytest.fail("no split-form slab configuration registered")


@pytest.mark.parametrize("shape", [(2, 64, 14, 14, 32, "fp16", True, True), (2, 96, 14, 12, 64, "bf16", True, False),
                                   (1, 160, 9, 10, 64, "fp16", False, True), (1, 32, 10, 10, 32, "bf16", True, True),
                                   (32, 256, 14, 14, 256, "fp16", True, True)],
                         ids=lambda c: "x".join(map(str, c[:5])) + f"-{c[5]}")
def test_split_staged_output_matches_pixel_pair_stores(shape):
    """The split form stages a whole-image unit's output in LDS and writes it with 16-byte stores when y is 16-byte
    aligned; a y 4 bytes off that takes the direct pixel-pair stores. Same accumulators, same rounding: the bits must
    agree, on two launches each (one slice, three, five, eight: the staging stage follows the slice count)."""
    B, C, H, W, K, prec, bias, relu = shape
    p = _problem(B, C, H, W, K, prec, bias, relu)
    b = Bundle(p, 0x5E7A + C + K, O.NORMAL)
    ci = _split_config()
    print(f"split config {ci} on {shape}: staged (y offset 0) and direct (y offset 4)", flush=True)
    staged = _run(p, b, ci, 1, 0, 0, reps=2)
    direct = _run(p, b, ci, 1, 0, 4, reps=2)
    assert staged is not None and direct is not None
    m = b.compare(staged[0])
    assert m.passed(), m.summary()
    for y in staged[1:] + direct:
        assert np.array_equal(np.nan_to_num(staged[0]), np.nan_to_num(y))


def test_slab_argument_checks():
    h = gie.hip()
    for bad in (gie.Problem(2, 64, 7, 7, 64, 5, 5, 1, 1, 2, 2, precision="fp16"),   # 5x5 filter
                gie.Problem(2, 64, 7, 7, 64, 3, 3, 2, 2, 1, 1, precision="fp16"),   # stride 2
                gie.Problem(2, 64, 7, 7, 64, 3, 3, 1, 1, 0, 0, precision="fp16"),   # no padding
                _problem(2, 132, 7, 7, 64, "fp16")):                                # C % 8 != 0
        for ci in range(h.gie_hip_slab_config_count()):
            assert h.gie_hip_slab_check(ci, ctypes.byref(bad.geom(bad.in_channels)), None) != 0
    wide = _problem(1, 64, 8, 40, 32, "fp16")  # rows wider than every pitch
    for ci in range(h.gie_hip_slab_config_count()):
        assert h.gie_hip_slab_check(ci, ctypes.byref(wide.geom(64)), None) != 0
    ok = _problem(2, 64, 14, 14, 64, "fp16")
    g = ok.geom(64)
    d = gie.DeviceBuffer(1 << 22)
    assert h.gie_hip_conv_slab(0, 1, ctypes.byref(g), d.addr, d.addr + 8, None, d.addr, None, 1, None) != 0  # w
    assert h.gie_hip_conv_slab(0, 1, ctypes.byref(g), d.addr + 1, d.addr, None, d.addr, None, 1, None) == -1  # x odd
    assert h.gie_hip_conv_slab(0, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr + 1, None, 1, None) == -1  # y odd
    assert h.gie_hip_conv_slab(0, 0, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 1, None) != 0  # fp32
    assert h.gie_hip_conv_slab(0, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 0, None) == -1  # split 0
    assert h.gie_hip_conv_slab(0, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 2, None) == -1  # no partial
    assert h.gie_hip_conv_slab(99, 1, ctypes.byref(g), d.addr, d.addr, None, d.addr, None, 1, None) == -1
