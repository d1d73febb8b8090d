"""TEST INFRASTRUCTURE ONLY — numpy/ctypes view of the C oracle (liboracle.so, built from gie_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module; the product
library never does. Every function names the reference file:line it restates (paths relative to the
reference checkout); the C file holds the algorithms.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

FP32, FP16, BF16, TF32 = 0, 1, 2, 3
PRECISIONS = {"fp32": FP32, "fp16": FP16, "bf16": BF16, "tf32": TF32}
OK, INVALID, UNSUPPORTED = 0, 1, 2
UNIFORM, NORMAL, SPARSE, POSITIVE = 0, 1, 2, 3
SCALING_REFERENCE, SCALING_BENCH = 0, 1


class Params(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "batch", "in_channels", "in_h", "in_w", "out_channels", "kernel_h", "kernel_w",
        "stride_h", "stride_w", "pad_h", "pad_w", "dilation_h", "dilation_w", "groups")]


class Metrics(ctypes.Structure):
    _fields_ = [("n", ctypes.c_int64), ("over_tol", ctypes.c_int64), ("nan_count", ctypes.c_int64),
                ("inf_count", ctypes.c_int64), ("max_abs", ctypes.c_double), ("mean_abs", ctypes.c_double),
                ("rms", ctypes.c_double), ("max_rel", ctypes.c_double), ("frac_over_tol", ctypes.c_double),
                ("worst_tol_ratio", ctypes.c_double), ("rel_l2", ctypes.c_double)]

    def passed(self) -> bool:
        """reference.h:71 ErrorMetrics::passed"""
        return self.n > 0 and self.nan_count == 0 and self.inf_count == 0 and self.over_tol == 0

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}

    def summary(self) -> str:
        return (f"max_abs={self.max_abs:.3g} rel_l2={self.rel_l2:.3g} over_tol={self.over_tol}/{self.n} "
                f"worst_tol_ratio={self.worst_tol_ratio:.3g} nan={self.nan_count} inf={self.inf_count}")


def build(force: bool = False) -> str:
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE], check=True, capture_output=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.POINTER(Params)
        fp = ctypes.POINTER(ctypes.c_float)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        L.gie_oracle_out_h.argtypes = [P]
        L.gie_oracle_out_w.argtypes = [P]
        L.gie_oracle_validate.argtypes = [P]
        L.gie_oracle_conv2d.argtypes = [P, ctypes.c_int, ctypes.c_int, fp, fp, fp, fp, fp, ctypes.c_int]
        L.gie_oracle_conv2d_points.argtypes = [P, ctypes.c_int, ctypes.c_int, fp, fp, fp,
                                               ctypes.POINTER(ctypes.c_int64), ctypes.c_int64, fp, fp, ctypes.c_int]
        L.gie_oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.gie_oracle_f32_to_f16.restype = ctypes.c_uint16
        L.gie_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.gie_oracle_f16_to_f32.restype = ctypes.c_float
        L.gie_oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.gie_oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.gie_oracle_round_tf32.argtypes = [ctypes.c_float]
        L.gie_oracle_round_tf32.restype = ctypes.c_float
        L.gie_oracle_quantize.argtypes = [ctypes.c_int, ctypes.c_float]
        L.gie_oracle_quantize.restype = ctypes.c_float
        L.gie_oracle_quantize_array.argtypes = [ctypes.c_int, fp, fp, ctypes.c_int64]
        L.gie_oracle_to_bits.argtypes = [ctypes.c_int, fp, u16p, ctypes.c_int64]
        L.gie_oracle_from_bits.argtypes = [ctypes.c_int, u16p, fp, ctypes.c_int64]
        L.gie_oracle_splitmix64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.gie_oracle_splitmix64.restype = ctypes.c_uint64
        L.gie_oracle_make_data.argtypes = [P, ctypes.c_int, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, fp, fp, fp]
        L.gie_oracle_tol.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_double, ctypes.c_double]
        L.gie_oracle_tol.restype = ctypes.c_double
        L.gie_oracle_compare.argtypes = [fp, fp, fp, ctypes.c_int64, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                         ctypes.POINTER(Metrics)]
        L.gie_oracle_repack_c_hw.argtypes = [u16p, u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.gie_oracle_lut_chunked.argtypes = [P, ctypes.POINTER(ctypes.c_int32)]
        L.gie_oracle_lut_chunked.restype = ctypes.c_int64
        L.gie_oracle_lut.argtypes = [P, ctypes.POINTER(ctypes.c_int32)]
        L.gie_oracle_lut.restype = ctypes.c_int64
        L.gie_oracle_splitk_range.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                              ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
        L.gie_oracle_splitk_reduce.argtypes = [fp, fp, fp, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_int]
        _lib = L
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u16(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


@dataclass
class Conv:
    """Conv2DParams (conv2d.h:47-73) + the ConvProblem epilogue flags (conv2d.h:76-85)."""
    batch: int = 1
    in_channels: int = 1
    in_h: int = 1
    in_w: int = 1
    out_channels: int = 1
    kernel_h: int = 1
    kernel_w: int = 1
    stride_h: int = 1
    stride_w: int = 1
    pad_h: int = 0
    pad_w: int = 0
    dilation_h: int = 1
    dilation_w: int = 1
    groups: int = 1
    has_bias: bool = False
    relu: bool = False
    precision: str = "fp32"

    def params(self) -> Params:
        return Params(self.batch, self.in_channels, self.in_h, self.in_w, self.out_channels, self.kernel_h,
                      self.kernel_w, self.stride_h, self.stride_w, self.pad_h, self.pad_w, self.dilation_h,
                      self.dilation_w, self.groups)

    @property
    def out_h(self) -> int:
        p = self.params()
        return lib().gie_oracle_out_h(ctypes.byref(p))

    @property
    def out_w(self) -> int:
        p = self.params()
        return lib().gie_oracle_out_w(ctypes.byref(p))

    @property
    def gemm_k(self) -> int:
        return self.in_channels * self.kernel_h * self.kernel_w

    def flops(self) -> int:
        return 2 * self.out_channels * self.batch * self.out_h * self.out_w * self.gemm_k

    def x_shape(self):
        return (self.batch, self.in_channels, self.in_h, self.in_w)

    def w_shape(self):
        return (self.out_channels, self.in_channels, self.kernel_h, self.kernel_w)

    def y_shape(self):
        return (self.batch, self.out_channels, self.out_h, self.out_w)


def P(B, C, H, W, O, Kh, Kw, Sh, Sw, Ph, Pw, **kw) -> Conv:
    """tests/shapes.h:20-25 argument order."""
    return Conv(B, C, H, W, O, Kh, Kw, Sh, Sw, Ph, Pw, **kw)


def validate(c: Conv) -> int:
    p = c.params()
    return lib().gie_oracle_validate(ctypes.byref(p))


def conv2d(c: Conv, x: np.ndarray, w: np.ndarray, bias: np.ndarray | None, threads: int = 0):
    """cpu_reference.cpp:13-56 -> (y, scale) float32 NCHW."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty(c.y_shape(), np.float32)
    s = np.empty(c.y_shape(), np.float32)
    b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
    p = c.params()
    rc = lib().gie_oracle_conv2d(ctypes.byref(p), int(c.has_bias), int(c.relu), _f(x), _f(w),
                                 _f(b) if b is not None else None, _f(y), _f(s), threads)
    if rc != OK:
        raise ValueError(f"invalid problem (code {rc})")
    return y, s


def conv2d_points(c: Conv, x: np.ndarray, w: np.ndarray, bias: np.ndarray | None, idx: np.ndarray,
                  threads: int = 0):
    """cpu_reference.cpp:13-56 restricted to the listed flat NCHW output indices -> (y, scale)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    y = np.empty(idx.size, np.float32)
    s = np.empty(idx.size, np.float32)
    b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
    p = c.params()
    rc = lib().gie_oracle_conv2d_points(ctypes.byref(p), int(c.has_bias), int(c.relu), _f(x), _f(w),
                                        _f(b) if b is not None else None,
                                        idx.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), idx.size, _f(y), _f(s),
                                        threads)
    if rc != OK:
        raise ValueError(f"invalid problem or index (code {rc})")
    return y, s


def make_data(c: Conv, seed: int, dist: int = UNIFORM, scaling: int = SCALING_BENCH):
    """testing.cu:75-105 draw order; returns quantized float32 x, w, bias."""
    x = np.empty(c.x_shape(), np.float32)
    w = np.empty(c.w_shape(), np.float32)
    b = np.empty((c.out_channels,), np.float32)
    p = c.params()
    rc = lib().gie_oracle_make_data(ctypes.byref(p), PRECISIONS[c.precision], ctypes.c_uint64(seed), dist, scaling,
                                    _f(x), _f(w), _f(b))
    if rc != OK:
        raise ValueError(f"invalid problem (code {rc})")
    return x, w, b


def quantize(precision: str, a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    lib().gie_oracle_quantize_array(PRECISIONS[precision], _f(a), _f(out), a.size)
    return out


def to_bits(precision: str, a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().gie_oracle_to_bits(PRECISIONS[precision], _f(a), _u16(out), a.size)
    return out


def from_bits(precision: str, a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().gie_oracle_from_bits(PRECISIONS[precision], _u16(a), _f(out), a.size)
    return out


def compare(test: np.ndarray, ref: np.ndarray, scale: np.ndarray, c: Conv, intermediate_rounding: bool = False,
            precision: str | None = None) -> Metrics:
    """reference.cu:139-200 TolerancePolicy::for_problem + compare_outputs (+ relative L2)."""
    t = np.ascontiguousarray(test, dtype=np.float32).ravel()
    r = np.ascontiguousarray(ref, dtype=np.float32).ravel()
    s = np.ascontiguousarray(scale, dtype=np.float32).ravel()
    assert t.size == r.size == s.size
    m = Metrics()
    lib().gie_oracle_compare(_f(t), _f(r), _f(s), t.size, PRECISIONS[precision or c.precision], c.gemm_k,
                             int(intermediate_rounding), ctypes.byref(m))
    return m


def tol(precision: str, k: int, ref: float, scale: float, intermediate_rounding: bool = False) -> float:
    return lib().gie_oracle_tol(PRECISIONS[precision], k, int(intermediate_rounding), ref, scale)


def repack_c_hw(src_bits: np.ndarray, batch: int, C: int, HW: int, C_pad: int | None = None) -> np.ndarray:
    """tensor_core_mma.cu:61-82: dst[b][hw][c] = src[b][c][hw] (16-bit), zero channels up to C_pad."""
    C_pad = C if C_pad is None else C_pad
    src = np.ascontiguousarray(src_bits, dtype=np.uint16).ravel()
    assert src.size == batch * C * HW
    dst = np.empty(batch * HW * C_pad, np.uint16)
    lib().gie_oracle_repack_c_hw(_u16(src), _u16(dst), batch, C, HW, C_pad)
    return dst


def lut(c: Conv) -> np.ndarray:
    """conv_common.cu:22-37 -> int32[C*KH*KW, 4]"""
    p = c.params()
    n = lib().gie_oracle_lut(ctypes.byref(p), None)
    out = np.empty((n, 4), np.int32)
    lib().gie_oracle_lut(ctypes.byref(p), out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)))
    return out


def lut_chunked(c: Conv) -> np.ndarray:
    """conv_common.cu:39-50 -> int32[chunks, 4]"""
    p = c.params()
    n = lib().gie_oracle_lut_chunked(ctypes.byref(p), None)
    if n < 0:
        raise ValueError("needs C % 8 == 0")
    out = np.empty((n, 4), np.int32)
    lib().gie_oracle_lut_chunked(ctypes.byref(p), out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)))
    return out


def splitk_range(ktiles: int, z: int, split: int):
    b, e = ctypes.c_int(), ctypes.c_int()
    lib().gie_oracle_splitk_range(ktiles, z, split, ctypes.byref(b), ctypes.byref(e))
    return b.value, e.value


def splitk_reduce(partial: np.ndarray, bias: np.ndarray | None, total: int, split: int, M: int, HWo: int,
                  relu: bool, precision: str) -> np.ndarray:
    p = np.ascontiguousarray(partial, dtype=np.float32).ravel()
    assert p.size == total * split
    y = np.empty(total, np.float32)
    b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
    lib().gie_oracle_splitk_reduce(_f(p), _f(b) if b is not None else None, _f(y), total, split, M, HWo, int(relu),
                                   PRECISIONS[precision])
    return y


def splitmix64_stream(seed: int, n: int) -> list[int]:
    s = ctypes.c_uint64(seed)
    return [lib().gie_oracle_splitmix64(ctypes.byref(s)) for _ in range(n)]
