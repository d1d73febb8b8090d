"""ctypes binding of the MI355X Conv2D library (lib/libgie.so + lib/libgie_hip.so).

This is host plumbing for tests, the benchmark and Python callers: every call goes through the C-ABI in
include/gie_capi.h (the gie:: plan API) or include/gie_hip.h (the kernels). It has no compute of its own and no
fallback — if the built libraries are missing, importing it raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
LIBGIE = os.path.join(LIB_DIR, "libgie.so")
LIBGIE_HIP = os.path.join(LIB_DIR, "libgie_hip.so")

FP32, FP16, BF16, TF32 = 0, 1, 2, 3
PRECISIONS = {"fp32": FP32, "fp16": FP16, "bf16": BF16, "tf32": TF32}
DTYPE_OF_PRECISION = {FP32: 0, FP16: 1, BF16: 2, TF32: 0}
BACKENDS = {"auto": 0, "cpu_reference": 1, "direct": 2, "im2col_gemm": 3, "simt_tiled": 4, "implicit_gemm": 5,
            "tensor_core": 6}
STATUS = {0: "Ok", 1: "InvalidArgument", 2: "Unsupported", 3: "WorkspaceTooSmall", 4: "HipError", 5: "Internal",
          6: "Io"}
SOURCES = ["forced_kernel", "forced_backend", "tuning_cache", "tuned", "cost_model"]


class GieError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS.get(code, code)}: {message}")
        self.code = code
        self.status = STATUS.get(code, str(code))


class GieProblem(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "batch", "in_channels", "in_h", "in_w", "out_channels", "kernel_h", "kernel_w", "stride_h", "stride_w",
        "pad_h", "pad_w", "dilation_h", "dilation_w", "groups", "precision", "has_bias", "relu")]


class GieOptions(ctypes.Structure):
    _fields_ = [("backend", ctypes.c_int), ("kernel", ctypes.c_char_p), ("autotune", ctypes.c_int),
                ("force_retune", ctypes.c_int), ("cache_path", ctypes.c_char_p)]


class GieTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int), ("n", ctypes.c_int64), ("c", ctypes.c_int64),
                ("h", ctypes.c_int64), ("w", ctypes.c_int64)]


class GieTuneOptions(ctypes.Structure):
    _fields_ = [("warmup", ctypes.c_int), ("samples", ctypes.c_int), ("min_sample_ms", ctypes.c_double),
                ("seed", ctypes.c_uint64), ("validate", ctypes.c_int), ("model_keep", ctypes.c_int),
                ("max_candidates", ctypes.c_int), ("use_cache", ctypes.c_int), ("force_retune", ctypes.c_int),
                ("verbose", ctypes.c_int), ("cache_path", ctypes.c_char_p)]


class GieConvGeom(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "batch", "in_channels", "in_h", "in_w", "out_channels", "kernel_h", "kernel_w", "stride_h", "stride_w",
        "pad_h", "pad_w", "out_h", "out_w", "c_pad", "relu")]


class GieHaloConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("tile_m", "tile_n", "tile_k", "kernel_h", "kernel_w", "threads",
                                            "stages", "version")]


class GieBandConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("tile_m", "tile_n", "tile_k", "kernel_h", "kernel_w", "threads",
                                            "stages", "version")]


class GieSlabConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("tile_m", "rows", "pitch", "tile_k", "stages", "workgroups_per_cu",
                                            "form", "threads", "lds_bytes", "version")]


class GieStackConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("tile_m", "rows", "pitch", "tile_k", "threads", "lds_bytes", "halves",
                                            "version")]


class GieDeviceModel(ctypes.Structure):
    _fields_ = [("cus", ctypes.c_int), ("mfma_tflops", ctypes.c_double), ("fp32_tflops", ctypes.c_double),
                ("hbm_gbs", ctypes.c_double), ("launch_us", ctypes.c_double), ("lds_per_workgroup", ctypes.c_size_t)]


class GieIgemmConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "tile_m", "tile_n", "tile_k", "waves_m", "waves_n", "threads", "lds_bytes", "stages", "version")]


_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i = ctypes.c_int
_cp = ctypes.c_char_p
_dp = ctypes.POINTER(ctypes.c_double)
_ip = ctypes.POINTER(ctypes.c_int)
_PP = ctypes.POINTER(GieProblem)
_TP = ctypes.POINTER(GieTensor)
_OP = ctypes.POINTER(GieOptions)

_CAPI = {
    "gie_last_error": ([], ctypes.c_char_p),
    "gie_status_string": ([_i], ctypes.c_char_p),
    "gie_validate_problem": ([_PP], _i),
    "gie_problem_key": ([_PP, _cp, _sz], _i),
    "gie_conv2d_forward": ([_PP, _TP, _TP, _TP, _TP, _vp, _sz, _vp, _OP], _i),
    "gie_conv2d_forward_n": ([_PP, _TP, _TP, _TP, _TP, _vp, _sz, _vp, _OP, _i], _i),
    "gie_conv2d_forward_n_timed": ([_PP, _TP, _TP, _TP, _TP, _vp, _sz, _vp, _OP, _i, _vp, _vp], _i),
    "gie_conv2d_time_forward": ([_PP, _TP, _TP, _TP, _TP, _vp, _sz, _vp, _OP, _i, _i, ctypes.c_double,
                                 ctypes.POINTER(ctypes.c_double), _ip], _i),
    "gie_conv2d_workspace_size": ([_PP, _OP, ctypes.POINTER(_sz)], _i),
    "gie_make_host_data": ([_PP, ctypes.c_uint64, _i, _i, _vp, _vp, _vp], _i),
    "gie_conv2d_clear_plan_cache": ([], _i),
    "gie_plan_create": ([_PP, _cp, _i, ctypes.POINTER(_vp)], _i),
    "gie_plan_destroy": ([_vp], _i),
    "gie_plan_workspace_bytes": ([_vp, ctypes.POINTER(_sz)], _i),
    "gie_plan_kernel_name": ([_vp, _cp, _sz], _i),
    "gie_plan_lut_bytes": ([_vp, ctypes.POINTER(_sz)], _i),
    "gie_plan_execute_staged": ([_vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, ctypes.POINTER(_vp)], _i),
    "gie_build_conv_lut": ([_PP, _i, ctypes.POINTER(ctypes.c_int32), ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)], _i),
    "gie_plan_execute": ([_vp, _TP, _TP, _TP, _TP, _vp, _sz, _vp], _i),
    "gie_plan_execute_unchecked": ([_vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp], _i),
    "gie_plan_time": ([_vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _i, _i, ctypes.c_double, _dp, _ip], _i),
    "gie_plan_time_stages": ([_vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _i, _dp], _i),
    "gie_registry_count": ([], _i),
    "gie_registry_name": ([_i, _cp, _sz], _i),
    "gie_kernel_describe": ([_cp, _cp, _sz], _i),
    "gie_kernel_supports": ([_cp, _PP, _ip, _cp, _sz], _i),
    "gie_dispatch_select": ([_PP, _OP, _cp, _sz, _ip, _dp], _i),
    "gie_rank_by_model": ([_PP, _cp, _sz, _dp, _i, _ip], _i),
    "gie_tune_options_default": ([ctypes.POINTER(GieTuneOptions)], None),
    "gie_autotune": ([_PP, ctypes.POINTER(GieTuneOptions), _cp, _sz, _dp, _dp, _ip], _i),
    "gie_tune_cache_key": ([_PP, _i, _cp, _sz], _i),
    "gie_tune_cache_size": ([_cp, ctypes.POINTER(_sz)], _i),
    "gie_tune_cache_clear": ([_cp], _i),
    "gie_estimate_kernel": ([_cp, _PP, _dp, _ip], _i),
    "gie_measure_host_cost": ([_PP, ctypes.POINTER(GieOptions), _i, _dp], _i),
    "gie_model_estimate": ([_cp, _PP, ctypes.POINTER(GieDeviceModel), _dp, _ip], _i),
    "gie_model_rank": ([_PP, ctypes.POINTER(GieDeviceModel), ctypes.c_char_p, _sz, _dp, _i, _ip], _i),
    "gie_measure_ceilings": ([_i, _i, _dp, _ip], _i),
    "gie_theoretical_ceilings": ([_i, _dp], _i),
    "gie_gpu_reference": ([_PP, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "gie_cpu_reference": ([_PP, _vp, _vp, _vp, _vp, _vp], _i),
    "gie_device_describe": ([_i, _cp, _sz], _i),
    "gie_device_arch": ([_i, _cp, _sz], _i),
    "gie_device_cu_count": ([_i, _ip], _i),
    "gie_build_fingerprint": ([_cp, _sz], _i),
    "gie_testing_add_faulty_kernels": ([_i], _i),
    "gie_testing_add_lut_probe_kernels": ([], _i),
    "gie_graph_create": ([ctypes.POINTER(_vp)], _i),
    "gie_graph_destroy": ([_vp], _i),
    "gie_graph_capture_chain": ([_vp, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                 ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                 ctypes.POINTER(_sz)], _i),
    "gie_graph_recapture_chain": ([_vp, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                   ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                   ctypes.POINTER(_sz), _ip], _i),
    "gie_graph_launch": ([_vp, _vp], _i),
    "gie_graph_node_count": ([_vp, ctypes.POINTER(_sz)], _i),
    "gie_dev_malloc": ([_sz, ctypes.POINTER(_vp)], _i),
    "gie_dev_free": ([_vp], _i),
    "gie_memcpy_h2d": ([_vp, _vp, _sz], _i),
    "gie_memcpy_d2h": ([_vp, _vp, _sz], _i),
    "gie_memcpy_d2d_async": ([_vp, _vp, _sz, _vp], _i),
    "gie_memset": ([_vp, _i, _sz], _i),
    "gie_device_synchronize": ([], _i),
    "gie_get_device_count": ([_ip], _i),
    "gie_set_device": ([_i], _i),
    "gie_stream_create": ([ctypes.POINTER(_vp)], _i),
    "gie_stream_destroy": ([_vp], _i),
    "gie_stream_synchronize": ([_vp], _i),
    "gie_event_create": ([ctypes.POINTER(_vp)], _i),
    "gie_event_destroy": ([_vp], _i),
    "gie_event_record": ([_vp, _vp], _i),
    "gie_event_synchronize": ([_vp], _i),
    "gie_event_elapsed_ms": ([_vp, _vp, ctypes.POINTER(ctypes.c_float)], _i),
}

_GP = ctypes.POINTER(GieConvGeom)
_HIP = {
    "gie_hip_status_string": ([_i], ctypes.c_char_p),
    "gie_hip_repack_act_nchw_to_nhwc": ([_vp, _vp, _i, _i, _i, _i, _vp], _i),
    "gie_hip_repack_w_oihw_to_orsc": ([_vp, _vp, _i, _i, _i, _i, _vp], _i),
    "gie_hip_repack_act_and_w": ([_vp, _vp, _vp, _vp, _GP, _vp], _i),
    "gie_hip_igemm_config_count": ([], _i),
    "gie_hip_igemm_config_get": ([_i, ctypes.POINTER(GieIgemmConfig)], _i),
    "gie_hip_igemm_occupancy": ([_i, _i, _ip], _i),
    "gie_hip_conv_igemm": ([_i, _i, _GP, _vp, _vp, _vp, _vp, _vp, _i, _vp], _i),
    "gie_hip_repack_blocked": ([_vp, _vp, _vp, _vp, _GP, _vp], _i),
    "gie_hip_halo_config_count": ([], _i),
    "gie_hip_halo_config_get": ([_i, ctypes.POINTER(GieHaloConfig)], _i),
    "gie_hip_halo_check": ([_i, _GP, _ip], _i),
    "gie_hip_conv_halo": ([_i, _i, _GP, _vp, _vp, _vp, _vp, _vp, _i, _vp], _i),
    "gie_hip_repack_w_blocked": ([_vp, _vp, _GP, _vp], _i),
    "gie_hip_band_config_count": ([], _i),
    "gie_hip_band_config_get": ([_i, ctypes.POINTER(GieBandConfig)], _i),
    "gie_hip_band_check": ([_i, _GP, _ip], _i),
    "gie_hip_conv_band": ([_i, _i, _GP, _vp, _vp, _vp, _vp, _vp, _i, _vp], _i),
    "gie_hip_pw_check": ([_GP, _ip], _i),
    "gie_hip_conv_pw": ([_i, _GP, _vp, _vp, _vp, _vp, _vp], _i),
    "gie_hip_splitk_reduce": ([_i, _vp, _vp, _vp, ctypes.c_int64, _i, _i, _i, _i, _vp], _i),
    "gie_hip_splitk_reduce_form": ([_i, ctypes.c_int64, _i, _i, _ip, _ip], _i),
    "gie_hip_bias_act": ([_i, _vp, _vp, ctypes.c_int64, _i, _i, _i, _vp], _i),
    "gie_hip_pws_check": ([_GP, _vp], _i),
    "gie_hip_conv_pws": ([_i, _GP, _vp, _vp, _vp, _vp, _vp], _i),
    "gie_hip_stem_check": ([_GP, _vp], _i),
    "gie_hip_conv_stem": ([_i, _GP, _vp, _vp, _vp, _vp, _vp], _i),
    "gie_hip_narrow_check": ([_GP, _vp], _i),
    "gie_hip_conv_narrow": ([_i, _GP, _vp, _vp, _vp, _vp, _vp], _i),
    "gie_hip_slab_config_count": ([], _i),
    "gie_hip_slab_config_get": ([_i, ctypes.POINTER(GieSlabConfig)], _i),
    "gie_hip_slab_check": ([_i, _GP, _ip], _i),
    "gie_hip_conv_slab": ([_i, _i, _GP, _vp, _vp, _vp, _vp, _vp, _i, _vp], _i),
    "gie_hip_conv_slab_noalloc": ([_i, _i, _GP, _vp, _vp, _vp, _vp, _i, _vp], _i),
    "gie_hip_slab_scratch_floats": ([], ctypes.c_longlong),
    "gie_hip_deep_check": ([_GP, _ip], _i),
    "gie_hip_conv_deep": ([_i, _GP, _vp, _vp, _vp, _vp, _vp], _i),
    "gie_hip_stack_config_count": ([], _i),
    "gie_hip_stack_config_get": ([_i, ctypes.POINTER(GieStackConfig)], _i),
    "gie_hip_stack_check": ([_i, _GP, _ip, _ip], _i),
    "gie_hip_conv_stack": ([_i, _i, _GP, _vp, _vp, _vp, _vp, _vp, _i, _vp], _i),
    "gie_hip_f32_config_count": ([], _i),
    "gie_hip_f32_config_tile_m": ([_i], _i),
    "gie_hip_f32_check": ([_i, _GP, _vp], _i),
    "gie_hip_conv_f32": ([_i, _i, _GP, _vp, _vp, _vp, _vp, _vp, _i, _vp], _i),
    "gie_hip_reference_conv": ([_i, _GP, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "gie_hip_ceiling_mfma": ([_i, _i, _vp, _vp], _i),
    "gie_hip_ceiling_copy": ([_vp, _vp, _sz, _vp], _i),
    "gie_hip_ceiling_stream": ([_vp, _sz, _vp, _sz, _i, _i, _vp], _i),
    "gie_hip_ceiling_empty": ([_vp], _i),
    "gie_hip_ceiling_empty_args": ([_i, _vp], _i),
    "gie_hip_fill_u16": ([_vp, ctypes.c_int64, ctypes.c_uint16, _vp], _i),
}

_libs = None


def libs():
    """(libgie, libgie_hip) — raises if the HIP build is missing; there is no fallback path."""
    global _libs
    if _libs is None:
        for p in (LIBGIE_HIP, LIBGIE):
            if not os.path.exists(p):
                raise ImportError(f"{p} is not built (run __graft_entry__.build() or make -C cuda-inference_amd)")
        hip = ctypes.CDLL(LIBGIE_HIP, mode=ctypes.RTLD_GLOBAL)
        gie = ctypes.CDLL(LIBGIE, mode=ctypes.RTLD_GLOBAL)
        for table, L in ((_CAPI, gie), (_HIP, hip)):
            for name, (args, res) in table.items():
                f = getattr(L, name)
                f.argtypes = args
                f.restype = res
        _libs = (gie, hip)
    return _libs


def capi():
    return libs()[0]


def hip():
    return libs()[1]


def check(rc: int, what: str = ""):
    if rc != 0:
        msg = capi().gie_last_error().decode(errors="replace")
        raise GieError(rc, f"{what}: {msg}" if what else msg)


def check_hip(rc: int, what: str):
    if rc != 0:
        raise GieError(4 if rc > 0 else (1 if rc == -1 else 2),
                       f"{what}: {hip().gie_hip_status_string(rc).decode()} ({rc})")


def _str_out(fn, *args, n=4096) -> str:
    buf = ctypes.create_string_buffer(n)
    check(fn(*args, buf, n))
    return buf.value.decode()


# ------------------------------------------------------------------------------------------------- problems
@dataclass
class Problem:
    """ConvProblem: geometry + precision + fused epilogue (conv2d.h:47-85)."""
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
    precision: str = "fp16"
    has_bias: bool = True
    relu: bool = True

    def c(self) -> GieProblem:
        return GieProblem(self.batch, self.in_channels, self.in_h, self.in_w, self.out_channels, self.kernel_h,
                          self.kernel_w, self.stride_h, self.stride_w, self.pad_h, self.pad_w, self.dilation_h,
                          self.dilation_w, self.groups, PRECISIONS[self.precision], int(self.has_bias),
                          int(self.relu))

    @property
    def out_h(self):
        return (self.in_h + 2 * self.pad_h - self.dilation_h * (self.kernel_h - 1) - 1) // self.stride_h + 1

    @property
    def out_w(self):
        return (self.in_w + 2 * self.pad_w - self.dilation_w * (self.kernel_w - 1) - 1) // self.stride_w + 1

    @property
    def gemm_m(self):
        return self.out_channels

    @property
    def gemm_n(self):
        return self.batch * self.out_h * self.out_w

    @property
    def gemm_k(self):
        return self.in_channels * self.kernel_h * self.kernel_w

    def flops(self) -> int:
        return 2 * self.gemm_m * self.gemm_n * self.gemm_k

    @property
    def dtype(self) -> int:
        return DTYPE_OF_PRECISION[PRECISIONS[self.precision]]

    @property
    def esize(self) -> int:
        return 4 if self.dtype == 0 else 2

    def x_shape(self):
        return (self.batch, self.in_channels, self.in_h, self.in_w)

    def w_shape(self):
        return (self.out_channels, self.in_channels, self.kernel_h, self.kernel_w)

    def y_shape(self):
        return (self.batch, self.out_channels, self.out_h, self.out_w)

    def b_shape(self):
        return (1, self.out_channels, 1, 1)

    def key(self) -> str:
        p = self.c()
        return _str_out(capi().gie_problem_key, ctypes.byref(p))

    def geom(self, c_pad: int | None = None) -> GieConvGeom:
        cp = c_pad if c_pad is not None else (self.in_channels + 7) // 8 * 8
        return GieConvGeom(self.batch, self.in_channels, self.in_h, self.in_w, self.out_channels, self.kernel_h,
                           self.kernel_w, self.stride_h, self.stride_w, self.pad_h, self.pad_w, self.out_h,
                           self.out_w, cp, int(self.relu))


def validate(p: Problem):
    pc = p.c()
    check(capi().gie_validate_problem(ctypes.byref(pc)), "validate_problem")


# ------------------------------------------------------------------------------------------------- memory
class DeviceBuffer:
    """Owning device allocation (gie_dev_malloc / gie_dev_free)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        if self.nbytes > 0:
            check(capi().gie_dev_malloc(self.nbytes, ctypes.byref(self.ptr)), "hipMalloc")

    @property
    def addr(self) -> int:
        return self.ptr.value or 0

    def free(self):
        if self.ptr.value:
            capi().gie_dev_free(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(capi().gie_memcpy_h2d(self.addr + offset, a.ctypes.data, a.nbytes), "upload")

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        check(capi().gie_memcpy_d2h(out.ctypes.data, self.addr + offset, out.nbytes), "download")
        return out

    def fill(self, value: int):
        check(capi().gie_memset(self.addr, value, self.nbytes), "memset")


def to_device(a: np.ndarray, extra: int = 0) -> DeviceBuffer:
    a = np.ascontiguousarray(a)
    b = DeviceBuffer(a.nbytes + extra)
    b.upload(a)
    return b


def synchronize():
    check(capi().gie_device_synchronize(), "hipDeviceSynchronize")


def device_count() -> int:
    n = ctypes.c_int(0)
    check(capi().gie_get_device_count(ctypes.byref(n)), "hipGetDeviceCount")
    return n.value


class Stream:
    def __init__(self):
        self.h = ctypes.c_void_p()
        check(capi().gie_stream_create(ctypes.byref(self.h)), "hipStreamCreate")

    def sync(self):
        check(capi().gie_stream_synchronize(self.h), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.h.value:
                capi().gie_stream_destroy(self.h)
        except Exception:
            pass


class Event:
    def __init__(self):
        self.h = ctypes.c_void_p()
        check(capi().gie_event_create(ctypes.byref(self.h)), "hipEventCreate")

    def record(self, stream=None):
        check(capi().gie_event_record(self.h, stream.h if stream else None), "hipEventRecord")

    def sync(self):
        check(capi().gie_event_synchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float()
        check(capi().gie_event_elapsed_ms(self.h, later.h, ctypes.byref(ms)), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.h.value:
                capi().gie_event_destroy(self.h)
        except Exception:
            pass


def tensor(ptr: int, p: Problem, which: str) -> GieTensor:
    shape = {"x": p.x_shape, "w": p.w_shape, "y": p.y_shape, "b": p.b_shape}[which]()
    return GieTensor(ptr, p.dtype, *shape)


# ------------------------------------------------------------------------------------------------- data
def host_to_storage(values: np.ndarray, precision: str) -> np.ndarray:
    """Storage bits of already-quantized float values (fp16 / bf16) or the float32 array itself."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    if precision == "fp16":
        return v.astype(np.float16).view(np.uint16)
    if precision == "bf16":
        u = v.view(np.uint32)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return v


def storage_to_float(bits: np.ndarray, precision: str) -> np.ndarray:
    if precision == "fp16":
        return bits.view(np.float16).astype(np.float32)
    if precision == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float32)


class ConvTensors:
    """Device copies of x, w, bias (storage dtype) and an output buffer poisoned with NaN bits."""

    def __init__(self, p: Problem, x: np.ndarray, w: np.ndarray, b: np.ndarray | None):
        self.p = p
        self.dx = to_device(host_to_storage(x, p.precision))
        self.dw = to_device(host_to_storage(w, p.precision))
        self.db = to_device(host_to_storage(b, p.precision)) if b is not None else None
        self.ny = int(np.prod(p.y_shape()))
        self.dy = DeviceBuffer(self.ny * p.esize)
        self.poison()

    def poison(self):
        self.dy.fill(0xFF)

    def tensors(self):
        p = self.p
        return (tensor(self.dx.addr, p, "x"), tensor(self.dw.addr, p, "w"),
                tensor(self.db.addr, p, "b") if (self.db is not None and p.has_bias) else None,
                tensor(self.dy.addr, p, "y"))

    def bias_addr(self):
        return self.db.addr if (self.db is not None and self.p.has_bias) else None

    def y(self) -> np.ndarray:
        raw = self.dy.download(np.uint16 if self.p.esize == 2 else np.uint32, self.ny)
        return storage_to_float(raw, self.p.precision).reshape(self.p.y_shape())


# ------------------------------------------------------------------------------------------------- API
def _opts(backend="auto", kernel=None, autotune=False, force_retune=False, cache_path=None) -> GieOptions:
    return GieOptions(BACKENDS[backend], kernel.encode() if kernel else None, int(autotune), int(force_retune),
                      cache_path.encode() if cache_path else None)


def workspace_size(p: Problem, **opt) -> int:
    pc, oc, n = p.c(), _opts(**opt), ctypes.c_size_t()
    check(capi().gie_conv2d_workspace_size(ctypes.byref(pc), ctypes.byref(oc), ctypes.byref(n)), "workspace_size")
    return n.value


def forward(p: Problem, t: ConvTensors, workspace: DeviceBuffer | None, stream: Stream | None = None,
            ws_bytes: int | None = None, **opt):
    """Conv2D::forward (conv2d.h:98-104)."""
    pc, oc = p.c(), _opts(**opt)
    x, w, b, y = t.tensors()
    check(capi().gie_conv2d_forward(ctypes.byref(pc), ctypes.byref(x), ctypes.byref(w),
                                    ctypes.byref(b) if b is not None else None, ctypes.byref(y),
                                    workspace.addr if workspace else None,
                                    ws_bytes if ws_bytes is not None else (workspace.nbytes if workspace else 0),
                                    stream.h if stream else None, ctypes.byref(oc)), "Conv2D::forward")


def forward_n(p: Problem, t: ConvTensors, workspace: DeviceBuffer | None, stream: Stream | None, count: int,
              **opt):
    """`count` Conv2D::forward calls issued from C++ (one timed benchmark step each)."""
    pc, oc = p.c(), _opts(**opt)
    x, w, b, y = t.tensors()
    check(capi().gie_conv2d_forward_n(ctypes.byref(pc), ctypes.byref(x), ctypes.byref(w),
                                      ctypes.byref(b) if b is not None else None, ctypes.byref(y),
                                      workspace.addr if workspace else None, workspace.nbytes if workspace else 0,
                                      stream.h if stream else None, ctypes.byref(oc), count), "Conv2D::forward x n")


def forward_n_timed(p: Problem, t: ConvTensors, workspace: DeviceBuffer | None, stream: Stream | None, count: int,
                    start: "Event", end: "Event", **opt):
    """forward_n with `start` / `end` recorded on the stream by the library right around the calls (the argument
    marshalling here happens before the start event)."""
    pc, oc = p.c(), _opts(**opt)
    x, w, b, y = t.tensors()
    check(capi().gie_conv2d_forward_n_timed(ctypes.byref(pc), ctypes.byref(x), ctypes.byref(w),
                                            ctypes.byref(b) if b is not None else None, ctypes.byref(y),
                                            workspace.addr if workspace else None,
                                            workspace.nbytes if workspace else 0, stream.h if stream else None,
                                            ctypes.byref(oc), count, start.h, end.h), "Conv2D::forward x n (timed)")


def time_forward(p: Problem, t: ConvTensors, workspace: DeviceBuffer | None, stream: Stream | None, warmup=5,
                 samples=30, min_sample_ms=1.0, **opt) -> dict:
    """Conv2D::forward under the library's time_stream_work protocol (warm-up, then `samples` samples of
    back-to-back calls lasting >= min_sample_ms each): per-call microsecond statistics."""
    pc, oc = p.c(), _opts(**opt)
    x, w, b, y = t.tensors()
    st, inner = (ctypes.c_double * 7)(), ctypes.c_int()
    check(capi().gie_conv2d_time_forward(ctypes.byref(pc), ctypes.byref(x), ctypes.byref(w),
                                         ctypes.byref(b) if b is not None else None, ctypes.byref(y),
                                         workspace.addr if workspace else None, workspace.nbytes if workspace else 0,
                                         stream.h if stream else None, ctypes.byref(oc), warmup, samples,
                                         min_sample_ms, st, ctypes.byref(inner)), "Conv2D::forward timing")
    keys = ("median_us", "mean_us", "min_us", "max_us", "p10_us", "p90_us", "stddev_us")
    return dict(zip(keys, list(st)), inner=inner.value, samples=samples, warmup=warmup, min_sample_ms=min_sample_ms)


def measure_host_cost(p: Problem, batch: int = 256, **opt) -> dict:
    """Host wall time per Conv2D::forward call (plan cached) and per bare kernel launch, plus the GPU time per
    forward, over batches of `batch` back-to-back calls (the library's own measurement, from C++)."""
    pc, oc = p.c(), _opts(**opt)
    out = (ctypes.c_double * 3)()
    check(capi().gie_measure_host_cost(ctypes.byref(pc), ctypes.byref(oc), batch, out), "measure_host_cost")
    return {"host_us_per_forward": out[0], "host_us_per_bare_launch": out[1], "device_us_per_forward": out[2]}


DISTRIBUTIONS = {"uniform": 0, "normal": 1, "sparse_signed": 2, "positive": 3}


def make_host_data(p: Problem, seed: int, dist: str = "uniform", scaling: str = "benchmark"):
    """The library's make_conv_data host half: quantized float32 x, w, bias (testing.h)."""
    x = np.empty(p.x_shape(), np.float32)
    w = np.empty(p.w_shape(), np.float32)
    b = np.empty((p.out_channels,), np.float32)
    pc = p.c()
    check(capi().gie_make_host_data(ctypes.byref(pc), seed, DISTRIBUTIONS[dist], 1 if scaling == "benchmark" else 0,
                                    x.ctypes.data, w.ctypes.data, b.ctypes.data), "make_conv_data")
    return x, w, b


def clear_plan_cache():
    check(capi().gie_conv2d_clear_plan_cache(), "clear_plan_cache")


class Plan:
    """ExecutionPlan bound to one registered kernel (execution_plan.h:14-51)."""

    def __init__(self, p: Problem, kernel: str, device: int = -1):
        self.p = p
        pc = p.c()
        self.h = ctypes.c_void_p()
        check(capi().gie_plan_create(ctypes.byref(pc), kernel.encode(), device, ctypes.byref(self.h)),
              f"ExecutionPlan::create({kernel})")

    def __del__(self):
        try:
            if self.h.value:
                capi().gie_plan_destroy(self.h)
        except Exception:
            pass

    @property
    def workspace_bytes(self) -> int:
        n = ctypes.c_size_t()
        check(capi().gie_plan_workspace_bytes(self.h, ctypes.byref(n)))
        return n.value

    @property
    def kernel(self) -> str:
        return _str_out(capi().gie_plan_kernel_name, self.h)

    @property
    def lut_bytes(self) -> int:
        n = ctypes.c_size_t()
        check(capi().gie_plan_lut_bytes(self.h, ctypes.byref(n)))
        return n.value

    def execute(self, t: ConvTensors, ws: DeviceBuffer | None, stream: Stream | None = None, **override):
        x, w, b, y = t.tensors()
        pass_bias = override.pop("bias", True)
        for k, v in override.items():  # e.g. x_data=..., y_c=... patch one field of one tensor descriptor
            setattr({"x": x, "w": w, "b": b, "y": y}[k[0]], k[2:], v)
        check(capi().gie_plan_execute(self.h, ctypes.byref(x), ctypes.byref(w),
                                      ctypes.byref(b) if (b is not None and pass_bias) else None,
                                      ctypes.byref(y), ws.addr if ws else None, ws.nbytes if ws else 0,
                                      stream.h if stream else None), "ExecutionPlan::execute")

    def execute_raw(self, x: int, w: int, b: int | None, y: int, ws: int | None, ws_bytes: int,
                    stream: Stream | None = None):
        check(capi().gie_plan_execute_unchecked(self.h, x, w, b, y, ws, ws_bytes, stream.h if stream else None),
              "ExecutionPlan::execute_unchecked")

    def time(self, t: ConvTensors, ws: DeviceBuffer, stream: Stream, warmup=5, samples=30, min_sample_ms=1.0):
        stats = (ctypes.c_double * 7)()
        inner = ctypes.c_int()
        check(capi().gie_plan_time(self.h, t.dx.addr, t.dw.addr, t.bias_addr(), t.dy.addr,
                                   ws.addr if ws else None, ws.nbytes if ws else 0, stream.h, warmup, samples,
                                   min_sample_ms, stats, ctypes.byref(inner)), "time_stream_work")
        keys = ("median_us", "mean_us", "min_us", "max_us", "p10_us", "p90_us", "stddev_us")
        d = dict(zip(keys, list(stats)))
        d["inner"] = inner.value
        return d

    def time_stages(self, t: ConvTensors, ws: DeviceBuffer, stream: Stream, iters=50):
        us = (ctypes.c_double * 3)()
        check(capi().gie_plan_time_stages(self.h, t.dx.addr, t.dw.addr, t.bias_addr(), t.dy.addr,
                                          ws.addr if ws else None, ws.nbytes if ws else 0, stream.h, iters, us),
              "stage timing")
        return {"repack_us": us[0], "gemm_us": us[1], "reduce_us": us[2]}


def build_conv_lut(p: Problem, chunked: bool = False) -> np.ndarray:
    """build_conv_lut / build_conv_lut_chunked (kernel_registry.h:86-96) -> int32[entries, 4]"""
    pc = p.c()
    n = ctypes.c_int64()
    check(capi().gie_build_conv_lut(ctypes.byref(pc), int(chunked), None, 0, ctypes.byref(n)), "build_conv_lut")
    out = np.empty((n.value, 4), np.int32)
    check(capi().gie_build_conv_lut(ctypes.byref(pc), int(chunked),
                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), n.value, ctypes.byref(n)),
          "build_conv_lut")
    return out


def registry() -> list[str]:
    return [_str_out(capi().gie_registry_name, i, n=256) for i in range(capi().gie_registry_count())]


def kernel_describe(name: str) -> dict:
    s = _str_out(capi().gie_kernel_describe, name.encode())
    out = {}
    for kv in s.split(","):
        k, v = kv.split("=")
        out[k] = int(v) if v.lstrip("-").isdigit() else v
    return out


def kernel_supports(name: str, p: Problem):
    pc, ok = p.c(), ctypes.c_int()
    why = ctypes.create_string_buffer(4096)
    check(capi().gie_kernel_supports(name.encode(), ctypes.byref(pc), ctypes.byref(ok), why, 4096))
    return bool(ok.value), why.value.decode()


def select(p: Problem, **opt):
    pc, oc = p.c(), _opts(**opt)
    buf = ctypes.create_string_buffer(256)
    src, us = ctypes.c_int(), ctypes.c_double()
    check(capi().gie_dispatch_select(ctypes.byref(pc), ctypes.byref(oc), buf, 256, ctypes.byref(src),
                                     ctypes.byref(us)), "Dispatcher::select")
    return buf.value.decode(), SOURCES[src.value], us.value


def rank_by_model(p: Problem):
    pc = p.c()
    buf = ctypes.create_string_buffer(65536)
    us = (ctypes.c_double * 512)()
    n = ctypes.c_int()
    check(capi().gie_rank_by_model(ctypes.byref(pc), buf, 65536, us, 512, ctypes.byref(n)), "rank_by_model")
    names = buf.value.decode().split("\n") if n.value else []
    return list(zip(names, list(us)[:n.value]))


def autotune(p: Problem, cache_path: str | None = None, force_retune=False, validate=True, model_keep=0,
             samples=10, warmup=3, min_sample_ms=0.5, verbose=False, use_cache=True, seed=None):
    o = GieTuneOptions()
    capi().gie_tune_options_default(ctypes.byref(o))
    o.samples, o.warmup, o.min_sample_ms = samples, warmup, min_sample_ms
    o.validate, o.model_keep, o.force_retune, o.verbose, o.use_cache = int(validate), model_keep, int(
        force_retune), int(verbose), int(use_cache)
    if seed is not None:
        o.seed = seed
    keep = cache_path.encode() if cache_path else None
    o.cache_path = keep
    pc = p.c()
    best = ctypes.create_string_buffer(256)
    best_us, secs = ctypes.c_double(), ctypes.c_double()
    counts = (ctypes.c_int * 6)()
    check(capi().gie_autotune(ctypes.byref(pc), ctypes.byref(o), best, 256, ctypes.byref(best_us),
                              ctypes.byref(secs), counts), "Autotuner::tune")
    keys = ("candidates_total", "candidates_measured", "from_cache", "rejected", "failed_validation", "errors")
    d = dict(zip(keys, list(counts)))
    d.update(best_kernel=best.value.decode(), best_us=best_us.value, search_seconds=secs.value)
    return d


def tune_cache_key(p: Problem, scope: str = "auto") -> str:
    pc = p.c()
    return _str_out(capi().gie_tune_cache_key, ctypes.byref(pc), BACKENDS[scope])


def tune_cache_size(path: str) -> int:
    n = ctypes.c_size_t()
    check(capi().gie_tune_cache_size(path.encode(), ctypes.byref(n)))
    return n.value


def tune_cache_clear(path: str):
    check(capi().gie_tune_cache_clear(path.encode()))


def estimate(name: str, p: Problem) -> dict:
    pc = p.c()
    out = (ctypes.c_double * 6)()
    bound = ctypes.c_int()
    check(capi().gie_estimate_kernel(name.encode(), ctypes.byref(pc), out, ctypes.byref(bound)), "estimate_kernel")
    d = dict(zip(("time_us", "compute_us", "memory_us", "launch_us", "tile_efficiency", "wave_efficiency"),
                 list(out)))
    d["bound"] = ("compute", "bandwidth", "launch")[bound.value]
    return d


# MI355X as the cost model describes it without measuring: 256 CUs, dense FP16 MFMA and FP32 vector peaks, HBM3E,
# dispatch gap of back-to-back launches, LDS opt-in limit per workgroup.
MI355X_MODEL = dict(cus=256, mfma_tflops=2516.6, fp32_tflops=157.3, hbm_gbs=8000.0, launch_us=1.5,
                    lds_per_workgroup=160 * 1024)


def _device_model(dev: dict | None) -> GieDeviceModel:
    d = dict(MI355X_MODEL, **(dev or {}))
    return GieDeviceModel(d["cus"], d["mfma_tflops"], d["fp32_tflops"], d["hbm_gbs"], d["launch_us"],
                          d["lds_per_workgroup"])


def model_estimate(name: str, p: Problem, dev: dict | None = None) -> dict:
    """The cost model's estimate for kernel `name` on a described device (MI355X by default); needs no GPU."""
    pc, dm = p.c(), _device_model(dev)
    out = (ctypes.c_double * 6)()
    bound = ctypes.c_int()
    check(capi().gie_model_estimate(name.encode(), ctypes.byref(pc), ctypes.byref(dm), out, ctypes.byref(bound)),
          "model_estimate")
    d = dict(zip(("time_us", "compute_us", "memory_us", "launch_us", "tile_efficiency", "wave_efficiency"),
                 list(out)))
    d["bound"] = ("compute", "bandwidth", "launch")[bound.value]
    return d


def model_rank(p: Problem, dev: dict | None = None):
    """Capable kernels, best first, with the model's estimate on a described device; needs no GPU."""
    pc, dm = p.c(), _device_model(dev)
    buf = ctypes.create_string_buffer(65536)
    us = (ctypes.c_double * 1024)()
    n = ctypes.c_int()
    check(capi().gie_model_rank(ctypes.byref(pc), ctypes.byref(dm), buf, 65536, us, 1024, ctypes.byref(n)),
          "model_rank")
    names = buf.value.decode().split("\n") if n.value else []
    return list(zip(names, list(us)[:n.value]))


def measure_ceilings(device=0, use_cache=False) -> dict:
    out = (ctypes.c_double * 3)()
    measured = ctypes.c_int()
    check(capi().gie_measure_ceilings(device, int(use_cache), out, ctypes.byref(measured)), "measure_ceilings")
    return {"fp16_mfma_tflops": out[0], "bw_gbs": out[1], "launch_overhead_us": out[2], "measured": bool(measured.value)}


def theoretical_ceilings(device=0) -> dict:
    out = (ctypes.c_double * 3)()
    check(capi().gie_theoretical_ceilings(device, out), "theoretical_ceilings")
    return {"fp16_mfma_tflops": out[0], "bw_gbs": out[1], "launch_overhead_us": out[2]}


def gpu_reference(p: Problem, t: ConvTensors):
    """gpu_conv2d_reference (reference.h:36-39) -> host float32 (y, scale)."""
    n = t.ny
    dy, ds = DeviceBuffer(4 * n), DeviceBuffer(4 * n)
    pc = p.c()
    check(capi().gie_gpu_reference(ctypes.byref(pc), t.dx.addr, t.dw.addr, t.bias_addr(), dy.addr, ds.addr, None),
          "gpu_conv2d_reference")
    synchronize()
    return dy.download(np.float32, n).reshape(p.y_shape()), ds.download(np.float32, n).reshape(p.y_shape())


def cpu_reference(p: Problem, x: np.ndarray, w: np.ndarray, b: np.ndarray | None):
    """The library's own cpu_conv2d_reference (reference.h:31-34)."""
    pc = p.c()
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    b = np.ascontiguousarray(b, np.float32) if b is not None else None
    y = np.empty(p.y_shape(), np.float32)
    s = np.empty(p.y_shape(), np.float32)
    check(capi().gie_cpu_reference(ctypes.byref(pc), x.ctypes.data, w.ctypes.data,
                                   b.ctypes.data if b is not None else None, y.ctypes.data, s.ctypes.data),
          "cpu_conv2d_reference")
    return y, s


def device_describe(device=0) -> str:
    return _str_out(capi().gie_device_describe, device)


def device_arch(device=0) -> str:
    return _str_out(capi().gie_device_arch, device)


def device_cu_count(device=0) -> int:
    n = ctypes.c_int()
    check(capi().gie_device_cu_count(device, ctypes.byref(n)))
    return n.value


def build_fingerprint() -> str:
    return _str_out(capi().gie_build_fingerprint)


class Graph:
    """HipGraphExecutor over a chain of plan executions (cuda_graph.h:14-46)."""

    def __init__(self):
        self.h = ctypes.c_void_p()
        check(capi().gie_graph_create(ctypes.byref(self.h)))

    def __del__(self):
        try:
            if self.h.value:
                capi().gie_graph_destroy(self.h)
        except Exception:
            pass

    @staticmethod
    def _arrays(steps):
        n = len(steps)
        V = ctypes.c_void_p * n
        plans = V(*[s[0].h.value for s in steps])
        xs, ws, bs, ys, wss = (V(*[s[i] for s in steps]) for i in range(1, 6))
        wb = (ctypes.c_size_t * n)(*[s[6] for s in steps])
        return n, plans, xs, ws, bs, ys, wss, wb

    def capture(self, steps):
        """steps: list of (plan, x, w, bias, y, workspace, workspace_bytes) with raw device addresses."""
        check(capi().gie_graph_capture_chain(self.h, *self._arrays(steps)), "HipGraphExecutor::capture")

    def recapture_update(self, steps) -> bool:
        up = ctypes.c_int()
        check(capi().gie_graph_recapture_chain(self.h, *self._arrays(steps), ctypes.byref(up)),
              "HipGraphExecutor::recapture_update")
        return bool(up.value)

    def launch(self, stream: Stream | None = None):
        check(capi().gie_graph_launch(self.h, stream.h if stream else None), "HipGraphExecutor::launch")

    @property
    def node_count(self) -> int:
        n = ctypes.c_size_t()
        check(capi().gie_graph_node_count(self.h, ctypes.byref(n)))
        return n.value


# ------------------------------------------------------------------------------------------------- kernels
def halo_configs() -> list[dict]:
    out = []
    for i in range(hip().gie_hip_halo_config_count()):
        c = GieHaloConfig()
        check_hip(hip().gie_hip_halo_config_get(i, ctypes.byref(c)), "halo config")
        out.append({f: getattr(c, f) for f, _ in c._fields_})
    return out


def band_configs() -> list[dict]:
    out = []
    for i in range(hip().gie_hip_band_config_count()):
        c = GieBandConfig()
        check_hip(hip().gie_hip_band_config_get(i, ctypes.byref(c)), "band config")
        out.append({f: getattr(c, f) for f, _ in c._fields_})
    return out


def igemm_configs() -> list[dict]:
    out = []
    for i in range(hip().gie_hip_igemm_config_count()):
        c = GieIgemmConfig()
        check_hip(hip().gie_hip_igemm_config_get(i, ctypes.byref(c)), "config")
        out.append({f: getattr(c, f) for f, _ in c._fields_})
    return out
