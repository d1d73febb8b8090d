"""Pins the CPU oracle (oracle/gie_oracle.c) before anything is checked against it.

Each check is chosen so that a plausible slip in the oracle (flipped kernel, dropped padding test, wrong
stride/pad term, transposed operand, lost bias or scale term, wrong rounding, off-by-one split) fails:
  * the reference's own known-answer tests, tests/test_cpu_reference.cpp:20-171 (values copied as data);
  * brute force through an independent formulation (numpy zero-pad + sliding windows, float64);
  * IEEE-754 binary16 rounding against numpy's float16 cast on 2^22 random bit patterns + edge cases;
  * bfloat16 rounding against a float64 nearest-candidate search (a different method than the bit trick);
  * SplitMix64 against its published first outputs for seed 0;
  * permutation identities for the repack and the LUT, partition properties for the split-K ranges.
"""
import math

import numpy as np
import pytest

import oracle as O
from oracle import P


def prob(c, bias=False, relu=False, precision="fp32"):
    c.has_bias, c.relu, c.precision = bias, relu, precision
    return c


# ---------------------------------------------------------------- test_cpu_reference.cpp known answers
def test_output_size_formula():  # test_cpu_reference.cpp:20-31
    assert P(1, 1, 7, 7, 1, 3, 3, 2, 2, 0, 0).out_h == 3
    assert P(1, 1, 8, 8, 1, 3, 3, 2, 2, 1, 1).out_h == 4
    p = P(1, 1, 5, 9, 1, 5, 3, 1, 3, 2, 1)
    assert (p.out_h, p.out_w) == (5, 3)
    p = P(2, 3, 224, 224, 64, 7, 7, 2, 2, 3, 3)
    assert p.out_h == 112
    assert p.flops() == 2 * 64 * (2 * 112 * 112) * (3 * 49)


def test_known_answer_ones_window():  # :33-40
    y, _ = O.conv2d(prob(P(1, 1, 3, 3, 1, 3, 3, 1, 1, 0, 0)), np.ones(9), np.ones(9), None)
    assert y.size == 1 and y.ravel()[0] == 9.0


def test_known_answer_cross_correlation_not_flipped():  # :42-51
    y, _ = O.conv2d(prob(P(1, 1, 3, 3, 1, 2, 2, 1, 1, 0, 0)), np.arange(1, 10), np.array([1, 0, 0, -1]), None)
    assert y.size == 4 and np.all(y == -4.0)


def test_known_answer_zero_padding():  # :53-60
    y, _ = O.conv2d(prob(P(1, 1, 2, 2, 1, 3, 3, 1, 1, 1, 1)), np.ones(4), np.ones(9), None)
    assert y.size == 4 and np.all(y == 4.0)


def test_known_answer_padding_corner():  # :62-72
    y, _ = O.conv2d(prob(P(1, 1, 3, 3, 1, 3, 3, 1, 1, 1, 1)), np.arange(1, 10), np.ones(9), None)
    y = y.ravel()
    assert y.size == 9 and y[0] == 12.0 and y[4] == 45.0 and y[8] == 5 + 6 + 8 + 9


def test_known_answer_stride():  # :74-85
    y, _ = O.conv2d(prob(P(1, 1, 4, 4, 1, 1, 1, 2, 2, 0, 0)), np.arange(16), np.array([1.0]), None)
    assert list(y.ravel()) == [0.0, 2.0, 8.0, 10.0]


def test_known_answer_channels_batch_bias_relu():  # :87-105
    c = prob(P(2, 2, 1, 1, 2, 1, 1, 1, 1, 0, 0), bias=True, relu=True)
    y, s = O.conv2d(c, np.array([1, 2, -3, 4]), np.array([1, 1, -1, 0.5]), np.array([0.25, -0.5]))
    assert list(y.ravel()) == [3.25, 0.0, 1.25, 4.5]
    assert abs(s.ravel()[0] - math.sqrt(5.0 + 9.0 + 0.0625)) < 1e-6


def test_identity_kernel_reproduces_input():  # :107-117
    c = prob(P(2, 3, 5, 6, 3, 1, 1, 1, 1, 0, 0))
    x = np.random.default_rng(7).uniform(-1, 1, c.x_shape()).astype(np.float32)
    w = np.eye(3, dtype=np.float32).reshape(3, 3, 1, 1)
    y, _ = O.conv2d(c, x, w, None)
    assert np.array_equal(y, x)


def test_cpu_reference_is_deterministic():  # :119-129
    c = prob(P(2, 5, 9, 7, 4, 3, 3, 2, 1, 1, 1))
    r = np.random.default_rng(3)
    x = r.uniform(-1, 1, c.x_shape()).astype(np.float32)
    w = r.uniform(-1, 1, c.w_shape()).astype(np.float32)
    a, _ = O.conv2d(c, x, w, None, threads=8)
    b, _ = O.conv2d(c, x, w, None, threads=1)
    assert np.array_equal(a, b)


def test_quantization_helpers():  # :131-140
    q = lambda p, v: O.lib().gie_oracle_quantize(O.PRECISIONS[p], v)
    assert q("fp32", 0.1) == np.float32(0.1)
    assert q("fp16", 1.0) == 1.0
    assert q("fp16", 0.1) != np.float32(0.1) and abs(q("fp16", 0.1) - 0.1) < 1e-4
    assert abs(q("bf16", 0.1) - 0.1) < 1e-3
    assert O.lib().gie_oracle_round_tf32(1.0 + 1.0 / 2048) == 1.0 + 1.0 / 1024
    assert O.lib().gie_oracle_round_tf32(1.0 + 1.0 / 4096) == 1.0


def test_error_metrics_detect_nan_and_over_tolerance():  # :142-156
    c = prob(P(1, 4, 4, 4, 1, 1, 1, 1, 1, 0, 0))
    ref, scale, test = np.ones(8, np.float32), np.ones(8, np.float32), np.ones(8, np.float32)
    assert O.compare(test, ref, scale, c).passed()
    test[3] = np.float32(1.0 + 1e-3)
    m = O.compare(test, ref, scale, c)
    assert not m.passed() and m.over_tol == 1
    test[3] = np.nan
    m = O.compare(test, ref, scale, c)
    assert m.nan_count == 1 and not m.passed()


def test_invalid_problems_are_rejected():  # :158-171
    assert O.validate(P(0, 1, 5, 5, 1, 3, 3, 1, 1, 0, 0)) == O.INVALID
    assert O.validate(P(1, 1, 2, 2, 1, 5, 5, 1, 1, 0, 0)) == O.INVALID
    assert O.validate(P(1, 1, 5, 5, 1, 3, 3, 0, 1, 0, 0)) == O.INVALID
    assert O.validate(P(1, 1, 5, 5, 1, 3, 3, 1, 1, -1, 0)) == O.INVALID
    d = P(1, 1, 9, 9, 1, 3, 3, 1, 1, 0, 0)
    d.dilation_h = 2
    assert O.validate(d) == O.UNSUPPORTED
    g = P(1, 4, 9, 9, 4, 3, 3, 1, 1, 0, 0)
    g.groups = 2
    assert O.validate(g) == O.UNSUPPORTED
    assert O.validate(P(30000, 1, 512, 512, 1, 1, 1, 1, 1, 0, 0)) == O.INVALID


# ---------------------------------------------------------------- brute force, independent formulation
def conv_windows_f64(c, x, w, bias):
    """Zero-pad, slice every (r, s) window with numpy strides and contract with tensordot (float64)."""
    x = x.astype(np.float64)
    w = w.astype(np.float64)
    xp = np.pad(x, ((0, 0), (0, 0), (c.pad_h, c.pad_h), (c.pad_w, c.pad_w)))
    OH, OW = c.out_h, c.out_w
    y = np.zeros((c.batch, c.out_channels, OH, OW))
    sq = np.zeros_like(y)
    for r in range(c.kernel_h):
        for s in range(c.kernel_w):
            win = xp[:, :, r:r + c.stride_h * (OH - 1) + 1:c.stride_h, s:s + c.stride_w * (OW - 1) + 1:c.stride_w]
            y += np.einsum("bchw,oc->bohw", win, w[:, :, r, s])
            sq += np.einsum("bchw,oc->bohw", win ** 2, w[:, :, r, s] ** 2)
    sq += y ** 2
    if c.has_bias:
        y += bias[None, :, None, None]
        sq += (bias.astype(np.float64) ** 2)[None, :, None, None]
    if c.relu:
        y = np.maximum(y, 0)
    return y, np.sqrt(sq)


BRUTE_SHAPES = [
    P(1, 1, 5, 5, 1, 3, 3, 1, 1, 0, 0), P(1, 3, 8, 8, 4, 3, 3, 1, 1, 1, 1), P(1, 3, 13, 11, 5, 5, 5, 2, 2, 2, 2),
    P(2, 7, 11, 13, 9, 3, 3, 2, 2, 0, 0), P(1, 2, 3, 3, 3, 3, 3, 1, 1, 2, 2), P(2, 8, 17, 23, 12, 3, 5, 2, 1, 1, 2),
    P(1, 4, 12, 12, 6, 1, 3, 1, 1, 0, 1), P(1, 4, 12, 12, 6, 3, 1, 1, 1, 1, 0), P(2, 3, 30, 30, 8, 7, 7, 2, 2, 3, 3),
    P(2, 16, 9, 9, 24, 1, 1, 1, 1, 0, 0),
]


@pytest.mark.parametrize("i", range(len(BRUTE_SHAPES)))
def test_conv_matches_window_formulation(i):
    c = prob(BRUTE_SHAPES[i], bias=i % 2 == 0, relu=i % 3 == 0)
    r = np.random.default_rng(100 + i)
    x = r.uniform(-1, 1, c.x_shape()).astype(np.float32)
    w = r.uniform(-1, 1, c.w_shape()).astype(np.float32)
    b = r.uniform(-1, 1, (c.out_channels,)).astype(np.float32)
    y, s = O.conv2d(c, x, w, b)
    ye, se = conv_windows_f64(c, x, w, b)
    assert np.allclose(y, ye, rtol=1e-6, atol=1e-6)
    assert np.allclose(s, se, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- rounding
def _edge_floats():
    v = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25,
         2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, np.inf, -np.inf, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]
    return np.array(v, np.float32)


def test_fp16_rounding_matches_numpy_ieee():
    bits = np.random.default_rng(0).integers(0, 2 ** 32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    vals = np.concatenate([bits.view(np.float32), _edge_floats()])
    vals = vals[~np.isnan(vals)]
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = O.to_bits("fp16", vals)
    assert np.array_equal(got, want)
    back = O.from_bits("fp16", got)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))
    assert O.to_bits("fp16", np.array([np.nan], np.float32))[0] & 0x7fff > 0x7c00


def _bf16_nearest(v):
    """Nearest bfloat16 by explicit candidate search in float64 (ties -> even mantissa)."""
    out = np.empty(v.size, np.uint16)
    u = v.view(np.uint32)
    for i, (x, b) in enumerate(zip(v.astype(np.float64), u)):
        if not np.isfinite(x):
            out[i] = b >> 16
            continue
        lo = int(b) >> 16
        hi = lo + 1
        flo = float(np.array([lo << 16], np.uint32).view(np.float32)[0])
        fhi = float(np.array([(hi << 16) & 0xFFFFFFFF], np.uint32).view(np.float32)[0])
        dlo, dhi = abs(x - flo), abs(fhi - x)
        out[i] = lo if (dlo < dhi or (dlo == dhi and lo % 2 == 0)) else hi
    return out


def test_bf16_rounding_matches_nearest_candidate_search():
    bits = np.random.default_rng(1).integers(0, 2 ** 32, size=1 << 14, dtype=np.uint64).astype(np.uint32)
    ties = (np.random.default_rng(2).integers(0, 2 ** 16, size=512, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    vals = np.concatenate([bits, ties]).view(np.float32)
    vals = np.concatenate([vals[~np.isnan(vals)], _edge_floats()])
    assert np.array_equal(O.to_bits("bf16", vals), _bf16_nearest(vals))


# ---------------------------------------------------------------- RNG and data
def test_splitmix64_published_first_outputs():
    assert O.splitmix64_stream(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_make_data_draw_order_and_ranges():
    c = prob(P(2, 4, 5, 5, 3, 3, 3, 1, 1, 1, 1), precision="fp16")
    x, w, b = O.make_data(c, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)
    raw = O.splitmix64_stream(0x1234ABCD, x.size + w.size + b.size)
    u = np.array([(v >> 11) for v in raw], np.float64) / 9007199254740992.0
    k = c.gemm_k
    ex = (np.float32(-1) + u[:x.size].astype(np.float32) * np.float32(2)).astype(np.float16).astype(np.float32)
    assert np.array_equal(x.ravel(), ex)
    ew = ((np.float32(-1) + u[x.size:x.size + w.size].astype(np.float32) * np.float32(2)) *
          (np.float32(1) / np.float32(math.sqrt(k)))).astype(np.float16).astype(np.float32)
    assert np.array_equal(w.ravel(), ew)
    eb = (np.float32(-0.1) + u[-b.size:].astype(np.float32) * np.float32(0.2)).astype(np.float16).astype(np.float32)
    assert np.array_equal(b, eb)
    assert np.abs(x).max() <= 1 and np.abs(w).max() <= 1 / math.sqrt(k) * 1.001 and np.abs(b).max() <= 0.1001
    x2, _, _ = O.make_data(c, 0x1234ABCD, O.UNIFORM, O.SCALING_BENCH)
    x3, _, _ = O.make_data(c, 0x1234ABCE, O.UNIFORM, O.SCALING_BENCH)
    assert np.array_equal(x, x2) and not np.array_equal(x, x3)


def test_make_data_reference_scaling_and_distributions():
    c = prob(P(1, 8, 6, 6, 8, 3, 3, 1, 1, 1, 1), precision="bf16")
    _, w, b = O.make_data(c, 5, O.UNIFORM, O.SCALING_REFERENCE)
    assert np.abs(w).max() <= math.sqrt(3 / c.gemm_k) * 1.01 and np.abs(b).max() <= 1.0
    xs, _, _ = O.make_data(c, 5, O.SPARSE, O.SCALING_REFERENCE)
    assert 0.5 < np.mean(xs == 0) < 0.9 and np.abs(xs).max() <= 2
    xp, _, _ = O.make_data(c, 5, O.POSITIVE, O.SCALING_REFERENCE)
    assert xp.min() >= 0
    xn, _, _ = O.make_data(c, 5, O.NORMAL, O.SCALING_REFERENCE)
    assert np.abs(xn).max() <= 6 and xn.std() > 0.5
    assert np.array_equal(O.quantize("bf16", xn), xn)


# ---------------------------------------------------------------- tolerance
def test_tolerance_closed_form():
    # reference.cu:165-167 with K=9: 8 * 2^-24 * 3 * scale + u_out * |ref| + floor
    assert O.tol("fp16", 9, 2.0, 4.0) == pytest.approx(8 * 2 ** -24 * 3 * 4 + 2 ** -11 * 2 + 3e-8, rel=1e-12)
    assert O.tol("bf16", 9, 2.0, 4.0) == pytest.approx(8 * 2 ** -24 * 3 * 4 + 2 ** -8 * 2, rel=1e-12)
    assert O.tol("fp32", 9, -2.0, 4.0) == pytest.approx(8 * 2 ** -24 * 3 * 4 + 2 ** -24 * 2, rel=1e-12)
    assert O.tol("fp16", 9, 2.0, 4.0, True) == pytest.approx(O.tol("fp16", 9, 2.0, 4.0) + 2 ** -11 * 4, rel=1e-12)


def test_rel_l2_metric():
    c = prob(P(1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0))
    ref = np.array([3.0, 4.0], np.float32)
    m = O.compare(ref + np.array([0.03, 0.04], np.float32), ref, np.ones(2, np.float32), c)
    assert m.rel_l2 == pytest.approx(0.01, rel=1e-5)


# ---------------------------------------------------------------- repack / LUT / split-K
@pytest.mark.parametrize("B,C,HW,Cp", [(1, 1, 1, 1), (2, 3, 7, 8), (3, 64, 196, 64), (1, 5, 33, 8), (2, 130, 9, 136)])
def test_repack_is_the_nchw_to_nhwc_permutation(B, C, HW, Cp):
    src = np.random.default_rng(B * 1000 + C).integers(0, 65536, size=B * C * HW, dtype=np.uint64).astype(np.uint16)
    dst = O.repack_c_hw(src, B, C, HW, Cp).reshape(B, HW, Cp)
    assert np.array_equal(dst[:, :, :C], src.reshape(B, C, HW).transpose(0, 2, 1))
    assert not dst[:, :, C:].any()


def test_weight_repack_gives_rsc_order():
    # OIHW -> O,R,S,C is the same permutation with batch=O, HW=R*S (tensor_core_mma.cu:310)
    O_, C, R, S = 5, 8, 3, 3
    w = np.arange(O_ * C * R * S, dtype=np.uint16)
    wk = O.repack_c_hw(w, O_, C, R * S).reshape(O_, R, S, C)
    assert np.array_equal(wk, w.reshape(O_, C, R, S).transpose(0, 2, 3, 1))


def test_lut_chunked_closed_form():
    c = P(1, 24, 9, 9, 4, 3, 2, 1, 1, 1, 0)
    lut = O.lut_chunked(c)
    k = np.arange(c.gemm_k)
    r, rem = np.divmod(k, c.kernel_w * c.in_channels)
    s, ch = np.divmod(rem, c.in_channels)
    assert lut.shape == (c.gemm_k // 8, 4)
    assert np.array_equal(lut[:, 0], ch[::8]) and np.array_equal(lut[:, 1], r[::8]) and np.array_equal(lut[:, 2], s[::8])
    assert np.all(ch[::8] % 8 == 0)
    with pytest.raises(ValueError):
        O.lut_chunked(P(1, 3, 9, 9, 4, 3, 3, 1, 1, 1, 1))


@pytest.mark.parametrize("dil", [1, 2])
def test_lut_gather_reproduces_the_convolution(dil):
    """The per-k table, used as an implicit-GEMM gather (column k of the patch matrix for output (oh, ow) is
    x[c_off + (oh + r_off) * W + ow + s_off]) against weights flattened in OIHW order, gives the convolution
    computed window by window; dilation 1 also against the oracle's own convolution."""
    c = P(1, 5, 9, 11, 3, 3, 2, 1, 1, 0, 0, dilation_h=dil, dilation_w=dil)
    t = O.lut(c)
    assert t.shape == (c.gemm_k, 4) and np.all(t[:, 3] == 0)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((c.in_channels, c.in_h, c.in_w))
    w = rng.standard_normal((c.out_channels, c.in_channels, c.kernel_h, c.kernel_w))
    oh, ow = c.in_h - dil * (c.kernel_h - 1), c.in_w - dil * (c.kernel_w - 1)
    gy, gx = np.meshgrid(np.arange(oh), np.arange(ow), indexing="ij")
    cols = np.stack([x.ravel()[e[0] + (gy + e[1]) * c.in_w + gx + e[2]] for e in t])  # [K, oh, ow]
    y_lut = w.reshape(c.out_channels, -1) @ cols.reshape(c.gemm_k, -1)
    y_win = np.zeros((c.out_channels, oh, ow))
    for ci in range(c.in_channels):
        for r in range(c.kernel_h):
            for s in range(c.kernel_w):
                y_win += w[:, ci, r, s, None, None] * x[ci, r * dil:r * dil + oh, s * dil:s * dil + ow]
    assert np.allclose(y_lut.reshape(y_win.shape), y_win, rtol=1e-12, atol=1e-12)
    if dil == 1:
        y_ref, _ = O.conv2d(prob(c), x.ravel(), w.ravel(), None)
        assert np.allclose(y_lut.ravel(), y_ref.ravel(), rtol=1e-5, atol=1e-5)  # the oracle reads float32 x, w


@pytest.mark.parametrize("ktiles,split", [(144, 1), (144, 2), (144, 8), (9, 4), (10, 3), (7, 8)])
def test_splitk_ranges_partition_the_k_tiles(ktiles, split):
    rs = [O.splitk_range(ktiles, z, split) for z in range(split)]
    assert rs[0][0] == 0 and rs[-1][1] == ktiles
    assert all(a[1] == b[0] for a, b in zip(rs, rs[1:]))
    sizes = [e - b for b, e in rs]
    assert max(sizes) - min(sizes) <= 1


def test_splitk_reduce_sequential_fp32_sum():
    split, M, HWo, Bn = 4, 6, 10, 2
    total = Bn * M * HWo
    part = np.random.default_rng(9).normal(size=(split, total)).astype(np.float32)
    bias = np.random.default_rng(10).uniform(-0.1, 0.1, M).astype(np.float32)
    y = O.splitk_reduce(part, bias, total, split, M, HWo, True, "fp16")
    s = part[0].copy()
    for z in range(1, split):
        s = (s + part[z]).astype(np.float32)
    s = s + np.tile(np.repeat(bias, HWo), Bn)
    want = np.maximum(s, 0).astype(np.float16).astype(np.float32)
    assert np.array_equal(y, want)
