"""GPU tests of the plan API around the kernels, restating the properties of the reference's
tests/test_validation.cpp, test_dispatcher.cpp, test_autotuner.cu, test_cuda_graph.cu and
test_runtime_concurrency.cu with this library's MFMA kernel names. Every call goes through the C-ABI
(include/gie_capi.h) into the gie:: C++ runtime."""
import ctypes
import json
import os
import threading

import numpy as np
import pytest

import gie
import oracle as O
from gpu_helpers import Bundle, kernels

pytestmark = pytest.mark.gpu

K16 = "mfma_fp16_64x64x32_w2x2_s4_sk1"
K16_SK4 = "mfma_fp16_64x64x32_w2x2_s4_sk4"
K16_BIG = "mfma_fp16_128x128x32_w2x2_s4_sk1"


def P(B, C, H, W, Oc, Kh, Kw, Sh, Sw, Ph, Pw, precision="fp16", bias=True, relu=True):
    return gie.Problem(B, C, H, W, Oc, Kh, Kw, Sh, Sw, Ph, Pw, precision=precision, has_bias=bias, relu=relu)


def expect_error(status, fn, *a, **kw):
    with pytest.raises(gie.GieError) as e:
        fn(*a, **kw)
    assert e.value.status == status, str(e.value)
    return str(e.value)


def test_registered_names_exist():
    names = gie.registry()
    for k in (K16, K16_SK4, K16_BIG):
        assert k in names


# ------------------------------------------------------------------------ test_validation.cpp
class Fixture:
    def __init__(self, bias=True):
        self.p = P(2, 8, 10, 10, 8, 3, 3, 1, 1, 1, 1, bias=bias, relu=False)
        self.b = Bundle(self.p, 1)
        self.plan = gie.Plan(self.p, K16)
        self.ws = gie.DeviceBuffer(self.plan.workspace_bytes)


def test_valid_call_succeeds_and_is_correct():
    f = Fixture()
    f.plan.execute(f.b.t, f.ws)
    gie.synchronize()
    assert f.b.compare(f.b.t.y()).passed()


def test_rejects_null_pointers_bad_shapes_and_dtypes():
    f = Fixture()
    expect_error("InvalidArgument", f.plan.execute, f.b.t, f.ws, x_data=None)
    expect_error("InvalidArgument", f.plan.execute, f.b.t, f.ws, x_h=11)
    expect_error("InvalidArgument", f.plan.execute, f.b.t, f.ws, w_dtype=0)
    expect_error("InvalidArgument", f.plan.execute, f.b.t, f.ws, y_c=9)


def test_rejects_bias_mismatch():
    f = Fixture()
    expect_error("InvalidArgument", f.plan.execute, f.b.t, f.ws, bias=False)
    nb = Fixture(bias=False)
    x, w, b, y = nb.b.t.tensors()
    bias = gie.tensor(f.b.t.db.addr, f.p, "b")
    import ctypes
    rc = gie.capi().gie_plan_execute(nb.plan.h, ctypes.byref(x), ctypes.byref(w), ctypes.byref(bias), ctypes.byref(y),
                                     nb.ws.addr, nb.ws.nbytes, None)
    assert gie.STATUS[rc] == "InvalidArgument"
    expect_error("InvalidArgument", f.plan.execute, f.b.t, f.ws, b_c=3)


def test_rejects_output_aliasing_inputs():
    f = Fixture()
    expect_error("InvalidArgument", f.plan.execute, f.b.t, f.ws, y_data=f.b.t.dx.addr)
    big = gie.DeviceBuffer(int(np.prod(f.p.y_shape())) * 2 + 4096)
    expect_error("InvalidArgument", f.plan.execute, f.b.t, f.ws, y_data=big.addr, x_data=big.addr + 1024)


def test_rejects_small_missing_or_misaligned_workspace():
    f = Fixture()
    assert f.plan.workspace_bytes > 0
    import ctypes
    x, w, b, y = f.b.t.tensors()
    rc = gie.capi().gie_plan_execute(f.plan.h, ctypes.byref(x), ctypes.byref(w), ctypes.byref(b), ctypes.byref(y),
                                     None, 0, None)
    assert gie.STATUS[rc] == "WorkspaceTooSmall"
    rc = gie.capi().gie_plan_execute(f.plan.h, ctypes.byref(x), ctypes.byref(w), ctypes.byref(b), ctypes.byref(y),
                                     f.ws.addr, f.ws.nbytes - 1, None)
    assert gie.STATUS[rc] == "WorkspaceTooSmall"
    ws2 = gie.DeviceBuffer(f.ws.nbytes + 256)
    rc = gie.capi().gie_plan_execute(f.plan.h, ctypes.byref(x), ctypes.byref(w), ctypes.byref(b), ctypes.byref(y),
                                     ws2.addr + 16, f.ws.nbytes, None)
    assert gie.STATUS[rc] == "InvalidArgument"
    rc = gie.capi().gie_plan_execute(f.plan.h, ctypes.byref(x), ctypes.byref(w), ctypes.byref(b), ctypes.byref(y),
                                     f.b.t.dx.addr, f.ws.nbytes, None)
    assert gie.STATUS[rc] in ("InvalidArgument", "WorkspaceTooSmall")


def test_plan_rejects_unsupported_precision():
    expect_error("Unsupported", gie.Plan, P(1, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1, precision="fp32"), K16)
    expect_error("Unsupported", gie.Plan, P(1, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1, precision="bf16"), K16)


def test_forward_end_to_end_with_workspace_check():
    p = P(2, 8, 10, 10, 8, 3, 3, 1, 1, 1, 1)
    b = Bundle(p, 3, O.NORMAL)
    # a kernel with a workspace (repack buffers) refuses a missing one
    opts = dict(kernel=K16)
    ws = gie.DeviceBuffer(gie.workspace_size(p, **opts))
    expect_error("WorkspaceTooSmall", gie.forward, p, b.t, None, **opts)
    b.t.poison()
    gie.forward(p, b.t, ws, **opts)
    gie.synchronize()
    assert b.compare(b.t.y()).passed()
    # whatever the dispatcher picks runs with exactly workspace_size() bytes (zero for the direct family)
    opts = dict(backend="tensor_core")
    need = gie.workspace_size(p, **opts)
    ws = gie.DeviceBuffer(need) if need else None
    b.t.poison()
    gie.forward(p, b.t, ws, **opts)
    gie.synchronize()
    assert b.compare(b.t.y()).passed()


def test_invalid_problems_rejected_through_the_api():
    expect_error("InvalidArgument", gie.validate, P(0, 1, 5, 5, 1, 3, 3, 1, 1, 0, 0))
    p = P(1, 1, 9, 9, 1, 3, 3, 1, 1, 0, 0)
    p.dilation_h = 2
    expect_error("Unsupported", gie.validate, p)


# ------------------------------------------------------------------------ test_dispatcher.cpp
def test_capability_filter_reports_every_kernel_with_a_reason():
    """tests/test_dispatcher.cpp:9-20: an FP32 problem has candidates, none of them a tensor-core kernel, and
    every other registered kernel is rejected with a reason."""
    p = P(1, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, precision="fp32", bias=False, relu=False)
    names = gie.registry()
    accepted, rejected = [], []
    for n in names:
        ok, why = gie.kernel_supports(n, p)
        (accepted if ok else rejected).append((n, why))
    assert accepted and rejected and len(accepted) + len(rejected) == len(names)
    assert all(gie.kernel_describe(n)["backend"] != "tensor_core" for n, _ in accepted)
    assert all(why for _, why in rejected)
    # forced to the tensor-core backend, the error lists every kernel of that backend with its reason
    msg = expect_error("Unsupported", gie.select, p, backend="tensor_core")
    tc = [n for n in names if gie.kernel_describe(n)["backend"] == "tensor_core"]
    assert tc and all(f"- {n}: " in msg for n in tc)


def test_precision_routes_to_matching_kernels():
    """tests/test_dispatcher.cpp:22-30, every precision of the reference included."""
    for prec in ("fp32", "fp16", "bf16", "tf32"):
        p = P(2, 32, 28, 28, 64, 3, 3, 1, 1, 1, 1, precision=prec)
        ranked = gie.rank_by_model(p)
        assert ranked, prec
        assert all(f"_{prec}_" in n for n, _ in ranked)


def test_cpu_reference_backend_is_not_dispatchable():
    expect_error("Unsupported", gie.select, P(1, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1), backend="cpu_reference")


def test_forced_backend_without_kernels_gives_clear_error():
    msg = expect_error("Unsupported", gie.select, P(1, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1), backend="direct")
    assert "direct" in msg
    msg = expect_error("Unsupported", gie.select, P(1, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1, precision="fp32"),
                       backend="tensor_core")
    assert "mfma_" in msg


def test_explicit_kernel_overrides_everything():
    p = P(1, 64, 8, 8, 8, 3, 3, 1, 1, 1, 1)
    k, src, _ = gie.select(p, kernel=K16_SK4)
    assert k == K16_SK4 and src == "forced_kernel"
    expect_error("InvalidArgument", gie.select, p, kernel="no_such_kernel")
    expect_error("InvalidArgument", gie.select, p, kernel=K16, backend="implicit_gemm")


def test_model_ranking_is_sorted_deterministic_and_positive():
    p = P(8, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1)
    r1, r2 = gie.rank_by_model(p), gie.rank_by_model(p)
    assert r1 and [n for n, _ in r1] == [n for n, _ in r2]
    us = [u for _, u in r1]
    assert us == sorted(us) and all(u > 0 for u in us)


def test_auto_selection_runs_and_matches_reference():
    for prec in ("fp16", "bf16"):
        p = P(2, 24, 21, 19, 40, 3, 3, 2, 2, 1, 1, precision=prec)
        b = Bundle(p, 9, O.NORMAL)
        opts = dict(cache_path="/nonexistent_dir_for_test/none.json")
        ws = gie.DeviceBuffer(gie.workspace_size(p, **opts))
        gie.forward(p, b.t, ws, **opts)
        gie.synchronize()
        assert b.compare(b.t.y()).passed()
        assert gie.select(p, **opts)[1] == "cost_model"


def test_plan_is_reused_across_calls():
    p = P(1, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1)
    b = Bundle(p, 4)
    gie.clear_plan_cache()
    ws = gie.DeviceBuffer(gie.workspace_size(p, kernel=K16))
    for _ in range(3):
        gie.forward(p, b.t, ws, kernel=K16)
    gie.synchronize()
    assert b.compare(b.t.y()).passed()


def test_forward_n_timed_brackets_the_calls_with_its_events():
    """The benchmark's timed step: count forward calls with the start/end events recorded by the library."""
    p = P(1, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1)
    b = Bundle(p, 5)
    ws = gie.DeviceBuffer(gie.workspace_size(p, kernel=K16))
    s = gie.Stream()
    e0, e1 = gie.Event(), gie.Event()
    b.t.poison()
    gie.forward_n_timed(p, b.t, ws, s, 4, e0, e1, kernel=K16)
    e1.sync()
    gie.synchronize()
    assert e0.elapsed_ms(e1) > 0.0
    assert b.compare(b.t.y()).passed()
    x, w, bias, y = b.t.tensors()
    rc = gie.capi().gie_conv2d_forward_n_timed(ctypes.byref(p.c()), ctypes.byref(x), ctypes.byref(w),
                                              ctypes.byref(bias), ctypes.byref(y), ws.addr, ws.nbytes, s.h,
                                              ctypes.byref(gie._opts(kernel=K16)), 1, None, e1.h)
    assert rc != 0 and "null event" in gie.capi().gie_last_error().decode()


def test_cost_model_bounds():
    big = P(32, 256, 28, 28, 256, 3, 3, 1, 1, 1, 1)
    assert gie.estimate(K16_BIG, big)["bound"] == "compute"
    thin = P(32, 8, 224, 224, 8, 1, 1, 1, 1, 0, 0)
    assert gie.estimate(K16, thin)["bound"] == "bandwidth"
    tiny = P(1, 8, 4, 4, 8, 1, 1, 1, 1, 0, 0)
    assert gie.estimate(K16, tiny)["bound"] == "launch"


# ------------------------------------------------------------------------ test_autotuner.cu
def _cache(tmp_path, tag):
    return str(tmp_path / f"tune_{tag}.json")


def test_incorrect_or_failing_candidates_are_never_selected(tmp_path):
    gie.check(gie.capi().gie_testing_add_faulty_kernels(0))
    gie.check(gie.capi().gie_testing_add_faulty_kernels(1))
    p = P(2, 16, 14, 14, 32, 3, 3, 1, 1, 1, 1)
    r = gie.autotune(p, cache_path=_cache(tmp_path, "faulty"), samples=5, warmup=2, min_sample_ms=0.2)
    assert not r["best_kernel"].startswith("test_")
    assert r["failed_validation"] >= 1 and r["errors"] >= 1
    b = Bundle(p, 12, O.NORMAL)
    plan = gie.Plan(p, r["best_kernel"])
    ws = gie.DeviceBuffer(plan.workspace_bytes)
    plan.execute(b.t, ws)
    gie.synchronize()
    assert b.compare(b.t.y()).passed()
    assert r["best_us"] > 0


@pytest.mark.parametrize("precision", ["fp16", "bf16"])
@pytest.mark.parametrize("chunked", [False, True])
def test_plan_uploads_the_gather_table_of_a_needs_lut_kernel(precision, chunked):
    """execution_plan.cpp:69-73,133: a kernel registered with needs_lut gets its gather table built once per plan,
    uploaded to the device and passed as plan_data. The probe kernel copies plan_data into y; the bytes must be the
    oracle's table (conv_common.cu:22-50). Kernels without needs_lut own no table."""
    gie.check(gie.capi().gie_testing_add_lut_probe_kernels())
    p = P(1, 24, 9, 8, 64, 2, 3, 1, 1, 0, 0, precision=precision, bias=False, relu=False)
    name = ("test_lut_chunked_probe_" if chunked else "test_lut_probe_") + precision
    plan = gie.Plan(p, name)
    c = O.P(1, 24, 9, 8, 64, 2, 3, 1, 1, 0, 0)
    want = O.lut_chunked(c) if chunked else O.lut(c)
    assert plan.lut_bytes == want.nbytes
    y = gie.DeviceBuffer(int(np.prod(p.y_shape())) * 2)
    assert y.nbytes >= want.nbytes
    y.fill(0xFF)
    plan.execute_raw(0, 0, None, y.addr, None, 0)
    gie.synchronize()
    got = y.download(np.int32, want.size).reshape(want.shape)
    assert np.array_equal(got, want)
    assert gie.Plan(P(1, 24, 9, 8, 64, 3, 3, 1, 1, 1, 1, precision=precision), K16 if precision == "fp16"
                    else K16.replace("fp16", "bf16")).lut_bytes == 0


@pytest.mark.parametrize("kernel", [K16, "mfma_fp16_64x64x32_w2x2_s4_sk4"])
def test_stage_events_bracket_repack_and_convolution(kernel):
    """execution_plan.cpp:122-136 / im2col.cu:88-114: stage events passed to execute are recorded before the
    repack, after it and after the convolution (before any split-K reduce), on the caller's stream, and the call's
    result is unchanged."""
    p = P(2, 64, 12, 12, 24, 3, 3, 1, 1, 1, 1)  # K = 576: long enough for split 4
    b = Bundle(p, 5)
    plan = gie.Plan(p, kernel)
    ws = gie.DeviceBuffer(plan.workspace_bytes) if plan.workspace_bytes else None
    st = gie.Stream()
    ev = [gie.Event() for _ in range(3)]
    evs = (ctypes.c_void_p * 3)(*[e.h.value for e in ev])
    b.t.poison()
    gie.check(gie.capi().gie_plan_execute_staged(plan.h, b.t.dx.addr, b.t.dw.addr, b.t.bias_addr(), b.t.dy.addr,
                                                   ws.addr if ws else None, ws.nbytes if ws else 0, st.h, evs),
              "execute with stage events")
    st.sync()
    repack_ms, conv_ms = ev[0].elapsed_ms(ev[1]), ev[1].elapsed_ms(ev[2])
    assert repack_ms > 0 and conv_ms > 0, (repack_ms, conv_ms)
    assert b.compare(b.t.y()).passed()


def test_search_space_and_cost_are_reported(tmp_path):
    p = P(2, 32, 14, 14, 32, 3, 3, 1, 1, 1, 1)
    r = gie.autotune(p, cache_path=_cache(tmp_path, "space"), samples=5, warmup=2, min_sample_ms=0.2)
    assert r["candidates_total"] >= 10 and r["candidates_measured"] == r["candidates_total"]
    assert r["search_seconds"] > 0


def test_cache_hit_persists_force_retune_and_clear(tmp_path):
    p = P(1, 16, 12, 12, 16, 3, 3, 1, 1, 1, 1)
    path = _cache(tmp_path, "hit")
    cold = gie.autotune(p, cache_path=path, samples=5, warmup=2, min_sample_ms=0.2)
    assert not cold["from_cache"]
    warm = gie.autotune(p, cache_path=path, samples=5, warmup=2, min_sample_ms=0.2)
    assert warm["from_cache"] and warm["best_kernel"] == cold["best_kernel"]
    k, src, _ = gie.select(p, cache_path=path)
    assert k == cold["best_kernel"] and src == "tuning_cache"
    assert not gie.autotune(p, cache_path=path, force_retune=True, samples=5, warmup=2,
                            min_sample_ms=0.2)["from_cache"]
    gie.tune_cache_clear(path)
    assert gie.tune_cache_size(path) == 0
    assert gie.select(p, cache_path=path)[1] == "cost_model"


def test_cache_key_separates_problems_precisions_and_fusion():
    a = P(1, 16, 12, 12, 16, 3, 3, 1, 1, 1, 1, bias=False, relu=False)
    variants = [P(1, 16, 12, 12, 16, 3, 3, 1, 1, 1, 1, precision="bf16", bias=False, relu=False),
                P(1, 16, 12, 12, 16, 3, 3, 1, 1, 1, 1, bias=True, relu=False),
                P(2, 16, 12, 12, 16, 3, 3, 1, 1, 1, 1, bias=False, relu=False)]
    ka = gie.tune_cache_key(a)
    for v in variants:
        assert gie.tune_cache_key(v) != ka
    assert gie.device_arch(0) in ka and "|hip" in ka and "|src" in ka
    assert gie.tune_cache_key(a, "tensor_core") != ka


def test_stale_and_corrupt_entries_are_rejected(tmp_path):
    p = P(1, 16, 12, 12, 16, 3, 3, 1, 1, 1, 1)
    path = _cache(tmp_path, "stale")
    gie.autotune(p, cache_path=path, samples=5, warmup=2, min_sample_ms=0.2)
    assert gie.select(p, cache_path=path)[1] == "tuning_cache"
    root = json.load(open(path))
    for e in root["entries"].values():
        e["kernel_version"] = 999
    json.dump(root, open(path, "w"))
    assert gie.select(p, cache_path=path)[1] == "cost_model"
    for e in root["entries"].values():
        e["kernel_version"] = 1
        e["kernel"] = "deleted_kernel"
    json.dump(root, open(path, "w"))
    assert gie.select(p, cache_path=path)[1] == "cost_model"
    with open(path, "w") as f:
        f.write("{ this is not json")
    assert gie.select(p, cache_path=path)[1] == "cost_model"
    again = gie.autotune(p, cache_path=path, samples=5, warmup=2, min_sample_ms=0.2)
    assert not again["from_cache"]
    assert gie.select(p, cache_path=path)[1] == "tuning_cache"


def test_model_pruning_limits_search(tmp_path):
    p = P(4, 64, 28, 28, 64, 3, 3, 1, 1, 1, 1)
    r = gie.autotune(p, cache_path=_cache(tmp_path, "prune"), use_cache=False, model_keep=4, samples=5, warmup=2,
                     min_sample_ms=0.2)
    assert r["candidates_measured"] == 4


def test_tuning_validation_is_reproducible(tmp_path):
    p = P(2, 8, 10, 10, 8, 3, 3, 1, 1, 1, 1)
    a = gie.autotune(p, use_cache=False, samples=3, warmup=1, min_sample_ms=0.1)
    b = gie.autotune(p, use_cache=False, samples=3, warmup=1, min_sample_ms=0.1)
    assert (a["candidates_total"], a["failed_validation"], a["errors"]) == \
        (b["candidates_total"], b["failed_validation"], b["errors"])


# ------------------------------------------------------------------------ test_cuda_graph.cu
def _copy_inputs(dst: Bundle, src: Bundle, stream):
    for d, s in ((dst.t.dx, src.t.dx), (dst.t.dw, src.t.dw), (dst.t.db, src.t.db)):
        gie.check(gie.capi().gie_memcpy_d2d_async(d.addr, s.addr, s.nbytes, stream.h))


def _poison_async(b: Bundle, stream):
    gie.check_hip(gie.hip().gie_hip_fill_u16(b.t.dy.addr, b.t.ny, 0xFFFF, stream.h), "fill")


@pytest.mark.parametrize("kernel", [K16, K16_SK4, "mfma_bf16_64x64x32_w2x2_s4_sk2", "band_fp16_3x3_32x224x32_s4_sk1",
                                    "band_bf16_3x3_32x224x32_s4_sk2"])
def test_graph_replay_with_changing_inputs(kernel):
    prec = "bf16" if "bf16" in kernel else "fp16"
    c = 128 if kernel.startswith("band_") else 32  # four 32-channel slices: enough K for the band kernel's split
    p = P(2, c, 14, 14, 48, 3, 3, 1, 1, 1, 1, precision=prec)
    plan = gie.Plan(p, kernel)  # plans exist before capture
    ws = gie.DeviceBuffer(plan.workspace_bytes)
    bufs = Bundle(p, 1)
    data = [Bundle(p, 50 + i, O.SPARSE if i == 1 else O.NORMAL) for i in range(3)]
    g = gie.Graph()
    g.capture([(plan, bufs.t.dx.addr, bufs.t.dw.addr, bufs.t.db.addr, bufs.t.dy.addr, ws.addr, ws.nbytes)])
    assert g.node_count >= (2 if kernel.endswith("sk1") else 3)
    s1, s2 = gie.Stream(), gie.Stream()
    for rep in range(6):
        st = s2 if rep % 2 else s1
        src = data[rep % 3]
        _copy_inputs(bufs, src, st)
        _poison_async(bufs, st)
        g.launch(st)
        st.sync()
        m = src.compare(bufs.t.y())
        assert m.passed(), f"{kernel} replay {rep}: {m.summary()}"


def test_graph_recapture_update_switches_buffers_in_place():
    p = P(1, 16, 12, 12, 16, 3, 3, 1, 1, 1, 1)
    plan = gie.Plan(p, K16)
    ws = gie.DeviceBuffer(plan.workspace_bytes)
    b1, b2 = Bundle(p, 5, O.NORMAL), Bundle(p, 6)
    step = lambda b: [(plan, b.t.dx.addr, b.t.dw.addr, b.t.db.addr, b.t.dy.addr, ws.addr, ws.nbytes)]
    g = gie.Graph()
    g.capture(step(b1))
    st = gie.Stream()
    g.launch(st)
    st.sync()
    assert b1.compare(b1.t.y()).passed()
    assert g.recapture_update(step(b2))
    b2.t.poison()
    g.launch(st)
    st.sync()
    assert b2.compare(b2.t.y()).passed()


def test_graph_chain_of_layers_equals_eager_chain():
    p = P(1, 32, 12, 12, 32, 3, 3, 1, 1, 1, 1)
    plan = gie.Plan(p, K16_SK4)
    b = Bundle(p, 9, O.NORMAL)
    n = int(np.prod(p.x_shape())) * 2
    a_buf, b_buf = gie.DeviceBuffer(n), gie.DeviceBuffer(n)
    ws = gie.DeviceBuffer(plan.workspace_bytes)
    steps = []
    src, dst = a_buf, b_buf
    for _ in range(4):
        steps.append((plan, src.addr, b.t.dw.addr, b.t.db.addr, dst.addr, ws.addr, ws.nbytes))
        src, dst = dst, src
    x_bits = gie.host_to_storage(b.x, "fp16")
    st = gie.Stream()
    a_buf.upload(x_bits)
    for s in steps:
        plan.execute_raw(*s[1:], stream=st)
    st.sync()
    eager = a_buf.download(np.uint16, n // 2)
    g = gie.Graph()
    g.capture(steps)
    for _ in range(3):
        a_buf.upload(x_bits)
        g.launch(st)
        st.sync()
        assert np.array_equal(a_buf.download(np.uint16, n // 2), eager)


# ------------------------------------------------------------------------ test_runtime_concurrency.cu
def test_create_then_use_on_fresh_streams():
    cases = []
    for k in (K16, K16_SK4, "mfma_fp16_128x64x64_w2x2_s3_sk1"):
        for v in range(2):
            p = P(2, 32 + 8 * v, 9 + v, 11, 24, 3, 3, 1, 1, 1, 1)
            cases.append((k, p, Bundle(p, 1000 + v, O.NORMAL)))
    bad = 0
    for it in range(36):
        k, p, b = cases[it % len(cases)]
        plan = gie.Plan(p, k)
        ws = gie.DeviceBuffer(plan.workspace_bytes)
        st = gie.Stream()
        _poison_async(b, st)
        plan.execute_raw(b.t.dx.addr, b.t.dw.addr, b.t.db.addr, b.t.dy.addr, ws.addr, ws.nbytes, st)
        st.sync()
        bad += not b.compare(b.t.y()).passed()
    assert bad == 0


@pytest.mark.parametrize("kernel", [K16, K16_SK4])
def test_one_plan_concurrent_streams_changing_inputs(kernel):
    p = P(2, 32, 10, 10, 32, 3, 3, 1, 1, 1, 1)
    plan = gie.Plan(p, kernel)
    S = 4
    streams = [gie.Stream() for _ in range(S)]
    bufs = [Bundle(p, 1 + s) for s in range(S)]
    even = [Bundle(p, 11 + s, O.NORMAL) for s in range(S)]
    odd = [Bundle(p, 91 + s, O.SPARSE) for s in range(S)]
    wss = [gie.DeviceBuffer(plan.workspace_bytes) for _ in range(S)]
    for rnd in range(6):
        for s in range(S):
            _copy_inputs(bufs[s], (odd if rnd % 2 else even)[s], streams[s])
            _poison_async(bufs[s], streams[s])
        for s in range(S):
            d = bufs[s]
            plan.execute_raw(d.t.dx.addr, d.t.dw.addr, d.t.db.addr, d.t.dy.addr, wss[s].addr, wss[s].nbytes,
                             streams[s])
        for s in range(S):
            streams[s].sync()
        for s in range(S):
            m = (odd if rnd % 2 else even)[s].compare(bufs[s].t.y())
            assert m.passed(), f"{kernel} stream {s} round {rnd}: {m.summary()}"


def test_one_plan_shared_by_host_threads():
    p = P(2, 32, 10, 10, 32, 3, 3, 1, 1, 1, 1)
    plan = gie.Plan(p, K16)
    T = 4
    bundles = [Bundle(p, 300 + t, O.NORMAL) for t in range(T)]
    wss = [gie.DeviceBuffer(plan.workspace_bytes) for _ in range(T)]
    errors = []

    def worker(t):
        try:
            gie.check(gie.capi().gie_set_device(0))
            st = gie.Stream()
            d = bundles[t]
            for _ in range(10):
                _poison_async(d, st)
                plan.execute_raw(d.t.dx.addr, d.t.dw.addr, d.t.db.addr, d.t.dy.addr, wss[t].addr, wss[t].nbytes, st)
                st.sync()
                if not d.compare(d.t.y()).passed():
                    errors.append(t)
        except Exception as e:  # noqa: BLE001
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(T)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors


@pytest.mark.parametrize("kernel", [K16, K16_SK4, K16_BIG])
def test_unaligned_user_pointers_are_correct(kernel):
    p = P(2, 32, 10, 10, 32, 3, 3, 1, 1, 1, 1)
    b = Bundle(p, 77, O.NORMAL)
    plan = gie.Plan(p, kernel)
    ws = gie.DeviceBuffer(plan.workspace_bytes)
    nx, ny = int(np.prod(p.x_shape())), int(np.prod(p.y_shape()))
    xb, yb, wb = gie.DeviceBuffer(nx * 2 + 64), gie.DeviceBuffer(ny * 2 + 64), gie.DeviceBuffer(
        int(np.prod(p.w_shape())) * 2 + 64)
    xb.upload(gie.host_to_storage(b.x, "fp16"), offset=2)
    wb.upload(gie.host_to_storage(b.w, "fp16"), offset=2)
    yb.fill(0xFF)
    plan.execute_raw(xb.addr + 2, wb.addr + 2, b.t.db.addr, yb.addr + 2, ws.addr, ws.nbytes)
    gie.synchronize()
    raw = np.frombuffer(yb.download(np.uint8, ny * 2 + 2)[2:].tobytes(), np.uint16)
    y = gie.storage_to_float(raw, "fp16")
    m = b.compare(y)
    assert m.passed(), m.summary()


def test_grid_limit_capability_checks():
    p = P(1, 8, 1, 1, 9_000_000, 1, 1, 1, 1, 0, 0)
    ok, why = gie.kernel_supports(K16, p)
    assert not ok and "grid.y" in why
