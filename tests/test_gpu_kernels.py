"""GPU parity of the hot-path kernels through the C-ABI against the CPU oracle.

* repacks: bit-exact against the oracle's restatement of the reference's transpose_c_hw indexing
  (src/kernels/tensor_core_mma.cu:61-82,309-310), including zero channel padding and 2-byte-aligned sources;
* split-K reduce: bit-exact against the oracle's ascending-z FP32 sum + epilogue + one rounding;
* MFMA implicit GEMM: every registered kernel on the reference's 26 correctness shapes (tests/shapes.h) in
  FP16 and BF16, cycling epilogues and distributions like run_suite (tests/conv_test_common.h:83-127), against
  the reference's per-element tolerance; every (shape, precision) cell must be covered by >= 1 kernel;
* the library's GPU double reference against the oracle (tests/test_direct_conv.cpp:6-21);
* the HBM streaming probe behind the measured write/read ceilings: layout of its writes and its argument checks.
"""
import ctypes

import numpy as np
import pytest

import gie
import oracle as O
from gpu_helpers import DISTS, SHAPES, Bundle, kernels, problem, run_plan

pytestmark = pytest.mark.gpu


def test_device_is_gfx950():
    assert gie.device_count() >= 1
    assert gie.device_arch(0).startswith("gfx950"), gie.device_describe(0)
    print(gie.device_describe(0))


def _bits(n, seed):
    return np.random.default_rng(seed).integers(0, 65536, size=n, dtype=np.uint64).astype(np.uint16)


@pytest.mark.parametrize("B,C,HW,Cp,offset", [
    (1, 1, 1, 8, 0), (2, 3, 50176, 8, 0), (3, 64, 196, 64, 2), (2, 256, 784, 256, 0), (1, 5, 33, 8, 2),
    (2, 130, 81, 136, 0), (4, 96, 729, 96, 2), (1, 16, 7, 16, 0), (2, 24, 49, 24, 0), (1, 512, 49, 512, 2)])
def test_repack_activation_bit_exact(B, C, HW, Cp, offset):
    src = _bits(B * C * HW, B * 7 + C)
    dsrc = gie.DeviceBuffer(src.nbytes + 16)
    dsrc.upload(src, offset=offset)
    dst = gie.DeviceBuffer(B * HW * Cp * 2)
    dst.fill(0xAB)
    gie.check_hip(gie.hip().gie_hip_repack_act_nchw_to_nhwc(dsrc.addr + offset, dst.addr, B, C, HW, Cp, None),
                  "repack act")
    gie.synchronize()
    got = dst.download(np.uint16, B * HW * Cp)
    assert np.array_equal(got, O.repack_c_hw(src, B, C, HW, Cp))


@pytest.mark.parametrize("Oc,C,RS,Cp,offset", [(64, 3, 49, 8, 0), (256, 256, 9, 256, 2), (9, 7, 9, 8, 0),
                                               (130, 130, 9, 136, 2), (1024, 256, 1, 256, 0), (1, 1, 1, 8, 0)])
def test_repack_weights_bit_exact(Oc, C, RS, Cp, offset):
    src = _bits(Oc * C * RS, Oc + C)
    dsrc = gie.DeviceBuffer(src.nbytes + 16)
    dsrc.upload(src, offset=offset)
    dst = gie.DeviceBuffer(Oc * RS * Cp * 2)
    dst.fill(0xCD)
    gie.check_hip(gie.hip().gie_hip_repack_w_oihw_to_orsc(dsrc.addr + offset, dst.addr, Oc, C, RS, Cp, None),
                  "repack w")
    gie.synchronize()
    assert np.array_equal(dst.download(np.uint16, Oc * RS * Cp), O.repack_c_hw(src, Oc, C, RS, Cp))


@pytest.mark.parametrize("shape", [SHAPES[3], SHAPES[14], SHAPES[17], SHAPES[8]], ids=lambda s: s[0])
def test_fused_repack_equals_both_permutations(shape):
    p = problem(shape, "fp16", True, True)
    cp = (p.in_channels + 7) // 8 * 8
    x = _bits(int(np.prod(p.x_shape())), 1)
    w = _bits(int(np.prod(p.w_shape())), 2)
    dx, dw = gie.to_device(x), gie.to_device(w)
    nx = p.batch * p.in_h * p.in_w * cp
    nw = p.out_channels * p.kernel_h * p.kernel_w * cp
    dxn, dwk = gie.DeviceBuffer(nx * 2), gie.DeviceBuffer(nw * 2)
    g = p.geom(cp)
    gie.check_hip(gie.hip().gie_hip_repack_act_and_w(dx.addr, dxn.addr, dw.addr, dwk.addr, ctypes.byref(g), None),
                  "fused repack")
    gie.synchronize()
    assert np.array_equal(dxn.download(np.uint16, nx), O.repack_c_hw(x, p.batch, p.in_channels, p.in_h * p.in_w, cp))
    assert np.array_equal(dwk.download(np.uint16, nw),
                          O.repack_c_hw(w, p.out_channels, p.in_channels, p.kernel_h * p.kernel_w, cp))


def test_repack_rejects_bad_arguments():
    d = gie.DeviceBuffer(4096)
    assert gie.hip().gie_hip_repack_act_nchw_to_nhwc(d.addr, d.addr + 2, 1, 3, 4, 8, None) == -1  # unaligned dst
    assert gie.hip().gie_hip_repack_act_nchw_to_nhwc(d.addr, d.addr, 1, 9, 4, 8, None) == -1  # c_pad < C
    assert gie.hip().gie_hip_repack_w_oihw_to_orsc(None, d.addr, 1, 3, 4, 8, None) == -1


@pytest.mark.parametrize("precision", ["fp16", "bf16"])
@pytest.mark.parametrize("split,M,HWo,B,relu,yoff", [(2, 512, 49, 8, 1, 0), (8, 512, 49, 8, 1, 2),
                                                     (4, 7, 13, 3, 0, 0), (3, 5, 9, 1, 1, 2),
                                                     (3, 64, 49, 4, 1, 0), (6, 32, 49, 2, 0, 2)])
def test_splitk_reduce_bit_exact(precision, split, M, HWo, B, relu, yoff):
    total = B * M * HWo
    rng = np.random.default_rng(split * 31 + M)
    part = rng.normal(size=(split, total)).astype(np.float32)
    bias = O.quantize(precision, rng.uniform(-0.1, 0.1, M).astype(np.float32))
    dpart = gie.to_device(part)
    db = gie.to_device(gie.host_to_storage(bias, precision))
    dy = gie.DeviceBuffer(total * 2 + 16)
    dt = gie.PRECISIONS[precision]
    gie.check_hip(gie.hip().gie_hip_splitk_reduce(dt, dpart.addr, db.addr, dy.addr + yoff, total, split, M, HWo,
                                                  relu, None), "reduce")
    gie.synchronize()
    raw = np.frombuffer(dy.download(np.uint8, total * 2 + yoff)[yoff:].tobytes(), np.uint16)
    got = gie.storage_to_float(raw, precision)
    want = O.splitk_reduce(part, bias, total, split, M, HWo, bool(relu), precision)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("shape", [SHAPES[0], SHAPES[2], SHAPES[6], SHAPES[12], SHAPES[17], SHAPES[22]],
                         ids=lambda s: s[0])
@pytest.mark.parametrize("precision", ["fp32", "fp16", "bf16"])
def test_gpu_reference_matches_cpu_oracle(shape, precision):
    p = problem(shape, precision, True, True)
    b = Bundle(p, 77, O.NORMAL)
    y, s = gie.gpu_reference(p, b.t)
    assert np.allclose(y, b.ref, rtol=1e-6, atol=1e-7)
    assert np.allclose(s, b.scale, rtol=1e-6, atol=1e-7)


def test_library_cpu_reference_matches_oracle():
    p = problem(SHAPES[12], "fp32", True, True)
    b = Bundle(p, 5, O.UNIFORM)
    y, s = gie.cpu_reference(p, b.x, b.w, b.b)
    assert np.array_equal(y, b.ref) and np.allclose(s, b.scale, rtol=1e-7)


@pytest.mark.parametrize("precision", ["fp16", "bf16"])
@pytest.mark.parametrize("si", range(len(SHAPES)), ids=[s[0] for s in SHAPES])
def test_mfma_family_on_correctness_shapes(si, precision):
    """Every registered kernel that accepts the shape runs it and passes the reference's tolerance."""
    cell = 2 * si + (precision == "bf16")
    mode = cell % 3
    p = problem(SHAPES[si], precision, mode >= 1, mode == 2)
    b = Bundle(p, 0xC0FFEE + cell, DISTS[cell % 4])
    ran = 0
    failures = []
    for k in kernels(precision):
        y, why = run_plan(k, b)
        if y is None:
            continue
        ran += 1
        m = b.compare(y)
        if not m.passed():
            failures.append(f"{k}: {m.summary()}")
    assert ran > 0, f"no kernel could run {SHAPES[si][0]} {precision}"
    assert not failures, "\n".join(failures[:10])


def test_fp32_is_rejected_with_reason():
    """tests/test_tensor_core.cpp:13-21: FP32 problems are rejected by the matrix-core family with a reason."""
    p = problem(SHAPES[6], "fp32", False, False)
    for k in kernels()[:4]:
        ok, why = gie.kernel_supports(k, p)
        assert not ok and ("fp16" in why or "bf16" in why)


@pytest.mark.parametrize("cin", [8, 16, 3, 5, 7])
def test_any_channel_count(cin):
    """tests/test_tensor_core.cpp:23-36: C % 8 == 0 and C % 8 != 0 both run (zero channel padding)."""
    p = gie.Problem(2, cin, 17, 19, 21, 3, 3, 1, 1, 1, 1, precision="fp16", has_bias=True, relu=False)
    b = Bundle(p, 41 + cin)
    for k in kernels("fp16"):
        y, why = run_plan(k, b)
        if y is not None:
            m = b.compare(y)
            assert m.passed(), f"{k} cin={cin} {m.summary()}"


def test_large_reduction_k4608_all_positive():
    """tests/test_tensor_core.cpp:59-70: K=4608, all-positive accumulation stress."""
    p = gie.Problem(2, 512, 9, 9, 64, 3, 3, 1, 1, 1, 1, precision="fp16", has_bias=True, relu=True)
    b = Bundle(p, 123, O.POSITIVE)
    for k in kernels("fp16"):
        y, why = run_plan(k, b)
        if y is not None:
            m = b.compare(y)
            assert m.passed(), f"{k} {m.summary()}"


def test_repeated_execution_is_stable():
    """tests/test_direct_conv.cpp:35-47 idea: repeated launches give bit-identical results (no LDS race)."""
    for si in (9, 6):
        p = problem(SHAPES[si], "fp16", True, True)
        b = Bundle(p, 9)
        ok = [k for k in kernels("fp16") if gie.kernel_supports(k, p)[0]]
        for fam in ("band_", "halo_", "mfma_"):
            picks = [k for k in ok if k.startswith(fam) and k.endswith("_sk1")][:3] + \
                [k for k in ok if k.startswith(fam) and k.endswith("_sk4")][:2]
            for k in picks:
                _repeat_check(k, b)


def _repeat_check(k, b):
    first, _ = run_plan(k, b)
    for _ in range(3):
        again, _ = run_plan(k, b, repeats=2)
        assert np.array_equal(first.view(np.uint32), again.view(np.uint32)), k


@pytest.mark.parametrize("policy", [0, 1, 2])
def test_stream_ceiling_writes_each_workgroups_own_chunk(policy):
    """gie_hip_ceiling_stream: workgroup b writes exactly its own chunk, element s*512 + t of it (step s, thread t)
    holding (sum of what it read, s, t, 7); a read-only run leaves dst untouched."""
    h = gie.hip()
    wg, w16 = 4, 3 * 512 + 64  # per workgroup: 3 whole steps and a partial one
    r16 = 512 + 40
    src = gie.DeviceBuffer(wg * r16 * 16)
    src.fill(0)
    dst = gie.DeviceBuffer(wg * w16 * 16 + 64)
    dst.fill(0xAB)
    gie.check_hip(h.gie_hip_ceiling_stream(src.addr, wg * r16 * 16, dst.addr, wg * w16 * 16, policy, wg, None),
                  "ceiling_stream")
    gie.synchronize()
    out = dst.download(np.uint32, (wg * w16 * 16 + 64) // 4)
    got = out[:wg * w16 * 4].reshape(wg, w16, 4)
    i = np.arange(w16)
    want = np.stack([np.zeros(w16, np.uint32), (i // 512).astype(np.uint32), (i % 512).astype(np.uint32),
                     np.full(w16, 7, np.uint32)], axis=1)
    for b in range(wg):
        assert np.array_equal(got[b], want), b
    assert np.all(out[wg * w16 * 4:] == 0xABABABAB)  # nothing past the last chunk
    dst.fill(0xAB)
    gie.check_hip(h.gie_hip_ceiling_stream(src.addr, wg * r16 * 16, dst.addr, 0, policy, wg, None), "read only")
    gie.synchronize()
    assert np.all(dst.download(np.uint32, 16) == 0xABABABAB)


def test_stream_ceiling_argument_checks():
    h = gie.hip()
    d = gie.DeviceBuffer(1 << 16)
    assert h.gie_hip_ceiling_stream(d.addr, 4096, d.addr, 4096, 3, 16, None) != 0      # policy
    assert h.gie_hip_ceiling_stream(d.addr, 4096, d.addr, 4096, 0, 0, None) != 0      # workgroups
    assert h.gie_hip_ceiling_stream(d.addr, 4096 + 16, d.addr, 4096, 0, 16, None) != 0  # not a multiple of 16 * wg
    assert h.gie_hip_ceiling_stream(None, 4096, d.addr, 4096, 0, 16, None) != 0        # reads without src
    assert h.gie_hip_ceiling_stream(d.addr, 4096, None, 0, 0, 16, None) != 0           # no dst
    assert h.gie_hip_ceiling_stream(d.addr, 0, d.addr, 0, 0, 16, None) != 0            # nothing to do
