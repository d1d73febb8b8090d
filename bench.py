"""Benchmark of the fused Conv2D hot path on one MI355X (BASELINE.json metric: fused FP16 conv TFLOP/s and % of
the MFMA peak per config; us/call next to the host CPU reference).

A step is one Conv2D::forward call through the unchanged plan API (plan-cache lookup, argument validation,
fused repack dispatch, MFMA implicit GEMM with the bias+ReLU epilogue, split-K reduce when the selected
kernel splits), issued back-to-back from C++ on one stream with inputs already resident in HBM. `value` is
config 2 (FP16 3x3, N=32 C=256 14x14 K=256): TFLOP/s = 2*M*N*K / (time per step).
The other GPU configs (1x1, 7x7 stem, BF16 split-K) are reported under "configs" with the same protocol.

roofline: the dominant kernel (the MFMA implicit GEMM) launched alone back to back on the bench stream between two
HIP events (on a workspace one full call has filled); algorithmic FLOPs per launch / average launch duration
against the dense FP16 MFMA peak.
cpu_baseline: the oracle's C restatement of the reference's cpu_conv2d_reference (OpenMP, double accumulation)
on the same quantized inputs, timed on this host.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cuda-inference_amd"))

PEAK_FP16_TFLOPS = 2516.6  # MI355X dense FP16/BF16 MFMA (256 CUs x 4096 FLOP/clk x 2.4 GHz)
PEAK_HBM_GBS = 8000.0
SEED = 0x1234ABCD

CONFIGS = {
    "c2_fp16_3x3": dict(batch=32, in_channels=256, in_h=14, in_w=14, out_channels=256, kernel_h=3, kernel_w=3,
                        stride_h=1, stride_w=1, pad_h=1, pad_w=1, precision="fp16"),
    "c3_fp16_1x1": dict(batch=64, in_channels=256, in_h=28, in_w=28, out_channels=1024, kernel_h=1, kernel_w=1,
                        stride_h=1, stride_w=1, pad_h=0, pad_w=0, precision="fp16"),
    "c4_fp16_7x7s2_stem": dict(batch=64, in_channels=3, in_h=224, in_w=224, out_channels=64, kernel_h=7, kernel_w=7,
                               stride_h=2, stride_w=2, pad_h=3, pad_w=3, precision="fp16"),
    "c5_bf16_3x3_splitk": dict(batch=8, in_channels=512, in_h=7, in_w=7, out_channels=512, kernel_h=3, kernel_w=3,
                               stride_h=1, stride_w=1, pad_h=1, pad_w=1, precision="bf16"),
}
HEADLINE = "c2_fp16_3x3"
# the reference's CPU-runnable FP32 case (timed on the host only)
C1 = dict(batch=1, in_channels=64, in_h=56, in_w=56, out_channels=64, kernel_h=3, kernel_w=3, stride_h=1, stride_w=1,
          pad_h=1, pad_w=1, precision="fp32")
SPLITK = "c5_bf16_3x3_splitk"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def compulsory_bytes(p) -> float:
    e = p.esize
    return float((np.prod(p.x_shape()) + np.prod(p.w_shape()) + np.prod(p.y_shape()) + p.out_channels) * e)


def run_config(gie, name, cfg, steps, warmup, stream, tune_cache, kernel=None):
    p = gie.Problem(**cfg, has_bias=True, relu=True)
    x, w, b = gie.make_host_data(p, SEED, "uniform", "benchmark")
    t = gie.ConvTensors(p, x, w, b)
    # pick the kernel: autotuned (validated against the GPU double reference, cached), or forced by name
    opts = dict(kernel=kernel) if kernel else dict(autotune=True, cache_path=tune_cache)
    kernel, source, _ = gie.select(p, **opts)
    ws = gie.DeviceBuffer(gie.workspace_size(p, **opts))
    # timed region: `warmup` untimed calls, then exactly `steps` forward calls between two events on the stream.
    # The output of the last timed call is what the correctness check below reads; the check (an FP64 reference
    # convolution on the GPU plus host-side comparison) runs after the timing so it does not sit in front of it.
    t.poison()
    gie.forward_n(p, t, ws, stream, warmup, **opts)
    stream.sync()
    e0, e1 = gie.Event(), gie.Event()
    gie.synchronize()
    # the library records e0 right before the first call and e1 right after the last (no Python work inside)
    gie.forward_n_timed(p, t, ws, stream, steps, e0, e1, **opts)
    e1.sync()
    gie.synchronize()
    ms = e0.elapsed_ms(e1)
    us_call = ms * 1e3 / steps
    flops = p.flops()
    tflops = flops / (us_call * 1e-6) / 1e12
    # correctness of the timed calls' output, against the library's GPU double reference
    y = t.y().astype(np.float64)
    ref, _ = gie.gpu_reference(p, t)
    ref = ref.astype(np.float64)
    if p.precision == "bf16":
        ref_r = (gie.storage_to_float(gie.host_to_storage(ref.astype(np.float32), "bf16"), "bf16")).astype(np.float64)
    else:
        ref_r = ref
    rel_l2 = float(np.linalg.norm(y - ref_r) / np.linalg.norm(ref_r))
    max_abs = float(np.abs(y - ref).max())
    # the reference harness's protocol (benchmark_main.cpp:55-56, timing.cpp:42-83): warm-up 5, then 30 samples of
    # back-to-back forward calls lasting >= 1 ms each, median per call
    med = gie.time_forward(p, t, ws, stream, warmup=5, samples=30, min_sample_ms=1.0, **opts)
    # per-stage device time (events on the launch stream around each kernel), same plan and buffers
    plan = gie.Plan(p, kernel)
    stages = plan.time_stages(t, ws, stream, iters=max(50, min(steps, 400)))
    gemm_tflops = flops / (stages["gemm_us"] * 1e-6) / 1e12
    cb = compulsory_bytes(p)
    ai = flops / cb
    roof_tflops = min(PEAK_FP16_TFLOPS, ai * PEAK_HBM_GBS / 1e3)
    desc = gie.kernel_describe(kernel)
    split = desc.get("split_k", 1)
    rp_bytes = repack_bytes(kernel, p)
    rd_bytes = reduce_bytes(split, p)
    out = {
        "kernel": kernel, "selection": source, "gemm_view": {"M": p.gemm_m, "N": p.gemm_n, "K": p.gemm_k},
        "gflop": flops / 1e9, "us_per_call": us_call, "tflops": tflops,
        "median_protocol": {"us_per_call": med["median_us"], "tflops": flops / (med["median_us"] * 1e-6) / 1e12,
                            "p10_us": med["p10_us"], "p90_us": med["p90_us"], "calls_per_sample": med["inner"],
                            "samples": med["samples"], "warmup": med["warmup"],
                            "min_sample_ms": med["min_sample_ms"]},
        "pct_of_fp16_peak": 100.0 * tflops / PEAK_FP16_TFLOPS,
        "roofline_tflops": roof_tflops, "roofline_fraction": tflops / roof_tflops,
        "bound": "mfma" if ai * PEAK_HBM_GBS / 1e3 >= PEAK_FP16_TFLOPS else "hbm",
        "compulsory_mb": cb / 1e6, "arith_intensity": ai,
        "stage_us": stages, "gemm_kernel_tflops": gemm_tflops,
        "repack_bytes": rp_bytes, "reduce_bytes": rd_bytes,
        "repack_gbs": rp_bytes / (stages["repack_us"] * 1e-6) / 1e9 if rp_bytes else None,
        "reduce_gbs": rd_bytes / (stages["reduce_us"] * 1e-6) / 1e9 if rd_bytes else None,
        "split_k": split, "rel_l2": rel_l2, "max_abs": max_abs,
        "parity_ok": bool(rel_l2 <= 1e-3 and max_abs <= 2e-2),
    }
    return p, t, out


def repack_bytes(kernel: str, p):
    """HBM bytes the kernel's repack launch moves (reads of x/w plus writes of the repacked copies), or None for a
    family that has no repack launch (slab, stack, pw, stem and narrow read NCHW x and OIHW w directly)."""
    e = p.esize
    nx, nw = float(np.prod(p.x_shape())), float(np.prod(p.w_shape()))
    taps = p.kernel_h * p.kernel_w
    if kernel.startswith("band_"):  # weights only: OIHW -> 32-channel blocks
        cp = (p.in_channels + 31) // 32 * 32
        return (nw + p.out_channels * taps * cp) * e
    if kernel.startswith("halo_") or kernel.startswith("mfma_"):  # x -> NHWC, w -> O x taps x C, channels padded
        cp = (p.in_channels + 31) // 32 * 32 if kernel.startswith("halo_") else (p.in_channels + 7) // 8 * 8
        return (nx + nw + (p.batch * p.in_h * p.in_w + p.out_channels * taps) * cp) * e
    return None


def reduce_bytes(split: int, p):
    """HBM bytes of the split-K reduce (FP32 partials read, bias read, output written), None without split-K."""
    if split <= 1:
        return None
    ny = float(np.prod(p.y_shape()))
    return split * ny * 4 + ny * p.esize + p.out_channels * p.esize


def repack_rates(gie, cfg, stream, launches: int = 200):
    """Achieved HBM rate of the repack kernels on one config's tensors: the NCHW -> NHWC activation repack, the
    OIHW -> O.RS.C weight repack (channels padded to a multiple of 8, as the implicit-GEMM entries use them) and the
    two in one dispatch, each launched `launches` times back to back between two events on the bench stream.
    Bytes = elements read (unpadded) + elements written (padded), 2 bytes each."""
    p = gie.Problem(**cfg, has_bias=True, relu=True)
    x, w, b = gie.make_host_data(p, SEED, "uniform", "benchmark")
    cp = (p.in_channels + 7) // 8 * 8
    hw, rs = p.in_h * p.in_w, p.kernel_h * p.kernel_w
    nx, nw = p.batch * p.in_channels * hw, p.out_channels * p.in_channels * rs
    nxp, nwp = p.batch * hw * cp, p.out_channels * rs * cp
    dx, dw = gie.to_device(gie.host_to_storage(x, p.precision)), gie.to_device(gie.host_to_storage(w, p.precision))
    dxn, dwk = gie.DeviceBuffer(2 * nxp + 256), gie.DeviceBuffer(2 * nwp + 256)
    g = p.geom(cp)
    H = gie.hip()
    kernels = {
        "act_nchw_to_nhwc": (lambda: H.gie_hip_repack_act_nchw_to_nhwc(dx.addr, dxn.addr, p.batch, p.in_channels, hw,
                                                                       cp, stream.h), 2 * (nx + nxp)),
        "w_oihw_to_orsc": (lambda: H.gie_hip_repack_w_oihw_to_orsc(dw.addr, dwk.addr, p.out_channels, p.in_channels,
                                                                   rs, cp, stream.h), 2 * (nw + nwp)),
        "act_and_w_one_dispatch": (lambda: H.gie_hip_repack_act_and_w(dx.addr, dxn.addr, dw.addr, dwk.addr,
                                                                      ctypes.byref(g), stream.h),
                                   2 * (nx + nxp + nw + nwp)),
    }
    out = {}
    for name, (launch, nbytes) in kernels.items():
        for _ in range(20):
            gie.check_hip(launch(), name)
        e0, e1 = gie.Event(), gie.Event()
        e0.record(stream)
        for _ in range(launches):
            gie.check_hip(launch(), name)
        e1.record(stream)
        e1.sync()
        us = e0.elapsed_ms(e1) * 1e3 / launches
        out[name] = {"us_per_launch": us, "bytes": nbytes, "gbs": nbytes / (us * 1e-6) / 1e9}
    return out


def fastest_split_entry(gie, cfg, stream):
    """Among the registry entries with split_k > 1 that can run cfg, the fastest by a short plan timing."""
    p = gie.Problem(**cfg, has_bias=True, relu=True)
    x, w, b = gie.make_host_data(p, SEED, "uniform", "benchmark")
    t = gie.ConvTensors(p, x, w, b)
    best, best_us = None, float("inf")
    for name in gie.registry():
        if gie.kernel_describe(name).get("split_k", 1) <= 1 or not gie.kernel_supports(name, p)[0]:
            continue
        plan = gie.Plan(p, name)
        ws = gie.DeviceBuffer(plan.workspace_bytes)
        us = plan.time(t, ws, stream, warmup=3, samples=5, min_sample_ms=0.3)["median_us"]
        if us < best_us:
            best, best_us = name, us
    return best


def cpu_time(c, x, w, b, cores: int, min_runs: int, budget_s: float):
    """Median wall time of the oracle on (c, x, w, b): at least min_runs runs, more while within budget_s."""
    import oracle as O
    times = []
    t_end = time.time() + budget_s
    while len(times) < min_runs or (time.time() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        O.conv2d(c, x, w, b, threads=cores)
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_configs(budget_s: float):
    """The oracle on BASELINE configs 1 (FP32, N=1 C=64 56x56 K=64 3x3) and 3-5, full workloads, median of >= 5
    (config 1) or >= 3 runs, on this host's cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    cores = len(os.sched_getaffinity(0))
    out = {}
    for name, cfg, runs in (("c1_fp32_3x3", C1, 5), ("c3_fp16_1x1", CONFIGS["c3_fp16_1x1"], 3),
                            ("c4_fp16_7x7s2_stem", CONFIGS["c4_fp16_7x7s2_stem"], 3),
                            ("c5_bf16_3x3_splitk", CONFIGS["c5_bf16_3x3_splitk"], 3)):
        c = O.Conv(cfg["batch"], cfg["in_channels"], cfg["in_h"], cfg["in_w"], cfg["out_channels"], cfg["kernel_h"],
                   cfg["kernel_w"], cfg["stride_h"], cfg["stride_w"], cfg["pad_h"], cfg["pad_w"], has_bias=True,
                   relu=True, precision=cfg["precision"])
        x, w, b = O.make_data(c, SEED, O.UNIFORM, O.SCALING_BENCH)
        med, n = cpu_time(c, x, w, b, cores, runs, budget_s)
        flops = 2.0 * cfg["batch"] * cfg["out_channels"] * c.out_h * c.out_w * cfg["in_channels"] * cfg["kernel_h"] * \
            cfg["kernel_w"]
        out[name] = {"us_per_call": med * 1e6, "tflops": flops / med / 1e12, "runs": n, "cores": cores,
                     "precision": cfg["precision"]}
        log(f"[bench] cpu {name}: {med * 1e3:.2f} ms/call ({n} runs, {cores} threads)")
    return out


def cpu_baseline(p, t, budget_s: float):
    """Oracle CPU reference (C, OpenMP, double accumulation) on the same quantized inputs, bounded in time."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    c = O.Conv(p.batch, p.in_channels, p.in_h, p.in_w, p.out_channels, p.kernel_h, p.kernel_w, p.stride_h,
               p.stride_w, p.pad_h, p.pad_w, has_bias=True, relu=True, precision=p.precision)
    x, w, b = O.make_data(c, SEED, O.UNIFORM, O.SCALING_BENCH)
    cores = len(os.sched_getaffinity(0))
    med, n = cpu_time(c, x, w, b, cores, 5, budget_s)
    return {"value": p.flops() / med / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "us_per_call": med * 1e6,
            "sample": f"full config-2 workload ({p.flops() / 1e9:.2f} GFLOP) x {n} runs, median; "
                      f"oracle/gie_oracle.c cpu_conv2d_reference restatement, {cores} OpenMP threads",
            "cpu_model": _cpu_model()}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_traffic(kernel_name: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary (FETCH_SIZE and
    WRITE_SIZE scaled by a plain copy's counters), when that summary covers the same registry kernel (else None:
    counters of another tiling say nothing about this one)."""
    path = os.path.join(ROOT, "profiles", "traffic_c2_fp16_3x3.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None
    k = d.get("kernels", {}).get(kernel_name)
    return k.get("bytes_per_launch") if k else None


def dominant_kernel(registry_name: str) -> str:
    """The device function that does the multiply-accumulate work for a registry kernel (the rocprof kernel name)."""
    if registry_name.startswith("slab_") and "_l_" in registry_name:
        return "slab_lean_kernel (3x3 MFMA convolution straight from NCHW / OIHW, lean form, conv_slab.hip)"
    if registry_name.startswith("slab_") and "_ld_" in registry_name:
        return ("slab_split_kernel (3x3 MFMA convolution straight from NCHW / OIHW, split form: loader waves beside "
                "the multiplying waves, conv_slab.hip)")
    if registry_name.startswith("deep_"):
        return ("deep_kernel (3x3 MFMA convolution of small images, whole reduction per workgroup, loader waves, "
                "conv_deep.hip)")
    if registry_name.startswith("slab_") and "_p_" in registry_name:
        return "slab_pipe_kernel (3x3 MFMA convolution straight from NCHW / OIHW, pipelined form, conv_slab.hip)"
    stems = [("slab_", "slab_kernel (3x3 MFMA convolution straight from NCHW / OIHW, conv_slab.hip)"),
             ("band_", "band_kernel (band MFMA convolution straight from NCHW, conv_band.hip)"),
             ("halo_", "halo_kernel (halo-tiled MFMA implicit GEMM, conv_halo.hip)"),
             ("stem_", "stem_kernel (7x7 stride-2 stem straight from NCHW, conv_stem.hip)"),
             ("narrow_", "narrow_kernel (3x3, whole reduction per workgroup, conv_narrow.hip)"),
             ("stack_", "stack_kernel (3x3 MFMA convolution of small images stacked per workgroup, conv_stack.hip)"),
             ("implicit_gemm_fp32_", "f32_kernel (FP32 MFMA convolution, conv_f32.hip)"),
             ("mfma_tf32_", "f32_kernel (TF32 MFMA convolution, conv_f32.hip)")]
    for stem, fn in stems:
        if registry_name.startswith(stem):
            return fn
    if registry_name.startswith("pw_"):
        if registry_name.endswith("_wreg"):
            return "pws_kernel (weight-stationary streaming pointwise, conv_pw.hip)"
        return "pw_kernel (pointwise MFMA convolution straight from NCHW, conv_pw.hip)"
    return "igemm_kernel (MFMA implicit GEMM, conv_mfma.hip)"


def copy_probe(gie, mib: int, reps: int):
    """A plain device copy of known size (`reps` launches of gie_hip_ceiling_copy over `mib` MiB): run under
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE it gives the counters' scale factor on this machine."""
    n = mib << 20
    src, dst = gie.DeviceBuffer(n), gie.DeviceBuffer(n)
    src.fill(0x3C)
    for _ in range(reps):
        gie.check_hip(gie.hip().gie_hip_ceiling_copy(src.addr, dst.addr, n, None), "ceiling_copy")
    gie.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n, "copy_probe_bytes_written": n, "launches": reps}), flush=True)


def stream_probe(gie, reps: int = 30, workgroups: int = 256):
    """HBM streaming ceilings at the benchmark outputs' byte counts (gie_hip_ceiling_stream: one contiguous chunk
    per workgroup, 16-byte accesses): writes of config 4's Y and the stem's and the pointwise kernel's read+write
    mixes, per store policy; microseconds per launch from events around `reps` launches after 5 untimed ones."""
    y4 = 64 * 64 * 112 * 112 * 2
    cases = [("write c4 Y", 0, y4, (0, 1, 2)),
             ("stem mix: read x, write Y (c4)", 64 * 3 * 224 * 224 * 2, y4, (0, 1)),
             ("pointwise mix: c3's counted bytes", 32899072, 116391936, (0, 1)),
             ("copy-like 64 MiB + 64 MiB", 64 << 20, 64 << 20, (0, 1))]
    big = max(max(r, w) for _, r, w, _ in cases)
    src, dst = gie.DeviceBuffer(big), gie.DeviceBuffer(big)
    src.fill(0x3C)
    dst.fill(0)
    s = gie.Stream()
    e0, e1 = gie.Event(), gie.Event()
    names = {0: "write-back", 1: "device scope (sc1)", 2: "non-temporal"}
    out = []
    for name, rb, wb, pols in cases:
        for pol in pols:
            launch = lambda: gie.check_hip(gie.hip().gie_hip_ceiling_stream(src.addr if rb else None, rb, dst.addr, wb,
                                                                              pol, workgroups, s.h), "ceiling_stream")
            for _ in range(5):
                launch()
            e0.record(s)
            for _ in range(reps):
                launch()
            e1.record(s)
            e1.sync()
            us = e0.elapsed_ms(e1) * 1e3 / reps
            out.append({"case": name, "stores": names[pol], "read_bytes": rb, "write_bytes": wb, "us": us,
                        "tb_per_s": (rb + wb) / us / 1e6})
            log(f"stream probe: {name}, {names[pol]}: {us:.2f} us, {(rb + wb) / us / 1e6:.2f} TB/s")
    print(json.dumps({"stream_probe": out, "workgroups": workgroups, "threads": 512, "launches": reps}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--configs", default="all", help="'all' or a comma list of config names")
    ap.add_argument("--cpu-budget-s", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--tune-cache", default=os.path.join(ROOT, "gpurun_out", "bench_tune_cache.json"))
    ap.add_argument("--kernel", default=None,
                    help="force this registry kernel (no autotune) on a single --configs entry; for a config other "
                         "than the headline only that config runs and its result dict is printed (profiling runs)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain copy of this many MiB (counter calibration) and exit")
    ap.add_argument("--stream-probe", action="store_true",
                    help="only run the HBM streaming ceilings (write / read / read+write per store policy) and exit")
    args = ap.parse_args()
    if args.steps < 1 or args.warmup < 0:
        ap.error("--steps must be >= 1 and --warmup >= 0")
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the Conv2D library is a "
              "single-GPU operator; across GPUs each rank would run its own share of the batch with the same "
              "weights, no collective in the forward pass).", file=sys.stderr)
        sys.exit(2)

    import gie
    gie.check(gie.capi().gie_set_device(0), "hipSetDevice")
    os.makedirs(os.path.dirname(args.tune_cache), exist_ok=True)
    if args.stream_probe:
        stream_probe(gie)
        return
    if args.copy_probe_mib > 0:
        copy_probe(gie, args.copy_probe_mib, 5)
        return
    stream = gie.Stream()
    names = list(CONFIGS) if args.configs == "all" else args.configs.split(",")
    if args.kernel and len(names) != 1:
        ap.error("--kernel applies to a single --configs entry")
    if args.kernel and names[0] != HEADLINE:
        name = names[0]
        _, _, r = run_config(gie, name, CONFIGS[name], args.steps, args.warmup, stream, args.tune_cache, args.kernel)
        log(f"[bench] {name}: {r['kernel']} {r['us_per_call']:.2f} us/call (kernel {r['stage_us']['gemm_us']:.2f} us)")
        print(json.dumps({"config": name, "result": r}), flush=True)
        return
    if HEADLINE not in names:
        names.insert(0, HEADLINE)
    results = {}
    head = None
    for name in names:
        log(f"[bench] {name}: tuning + timing")
        # every config under the same protocol: --warmup untimed calls, then exactly --steps timed calls
        p, t, r = run_config(gie, name, CONFIGS[name], args.steps, args.warmup, stream, args.tune_cache,
                             args.kernel if name == HEADLINE else None)
        log(f"[bench] {name}: {r['kernel']} {r['us_per_call']:.2f} us/call {r['tflops']:.1f} TFLOP/s "
            f"(median protocol {r['median_protocol']['us_per_call']:.2f} us; gemm {r['stage_us']['gemm_us']:.2f} us, "
            f"repack {r['stage_us']['repack_us']:.2f} us) rel_l2={r['rel_l2']:.2e}")
        results[name] = r
        if name == HEADLINE:
            head = (p, t)
    if SPLITK in names and not args.kernel:
        # BASELINE config 5 is the split-K config: whatever the autotuner picked, also bench the fastest entry that
        # splits the reduction, so the reduce kernel's time and GB/s are measured on the real shape
        best = fastest_split_entry(gie, CONFIGS[SPLITK], stream)
        if best:
            log(f"[bench] {SPLITK}: forced split-K entry {best}")
            _, _, r = run_config(gie, SPLITK, CONFIGS[SPLITK], args.steps, args.warmup, stream, args.tune_cache, best)
            r["selection"] = "forced: fastest split_k > 1 entry by a short plan timing"
            log(f"[bench] {SPLITK} split-K: {r['kernel']} {r['us_per_call']:.2f} us/call, reduce "
                f"{r['stage_us']['reduce_us']:.2f} us = {r['reduce_gbs'] or 0:.0f} GB/s")
            results[SPLITK + "_forced_splitk"] = r
    repack = {}
    if not args.kernel:
        # the repack kernels of the implicit-GEMM path, on the configs whose tensors they would move
        for name in names:
            repack[name] = repack_rates(gie, CONFIGS[name], stream)
            r = repack[name]
            log(f"[bench] {name} repack: activations {r['act_nchw_to_nhwc']['gbs']:.0f} GB/s "
                f"({r['act_nchw_to_nhwc']['us_per_launch']:.2f} us), weights {r['w_oihw_to_orsc']['gbs']:.0f} GB/s "
                f"({r['w_oihw_to_orsc']['us_per_launch']:.2f} us), both in one dispatch "
                f"{r['act_and_w_one_dispatch']['gbs']:.0f} GB/s")
    hr = results[HEADLINE]
    p, t = head
    cpu = None
    cpu_other = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (oracle) on the host")
        cpu = cpu_baseline(p, t, args.cpu_budget_s)
        cpu_other = cpu_configs(min(args.cpu_budget_s, 5.0))
        cpu["other_configs"] = cpu_other
    host = gie.measure_host_cost(gie.Problem(1, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1, precision="fp16"), 256)
    log(f"[bench] host cost per Conv2D::forward (plan cached, 1x8x8x8 -> 8 3x3): {host['host_us_per_forward']:.2f} "
        f"us vs {host['host_us_per_bare_launch']:.2f} us per bare kernel launch")
    gemm_us = hr["stage_us"]["gemm_us"]
    achieved = p.flops() / (gemm_us * 1e-6) / 1e12
    line = {
        "metric": "fused FP16 conv TFLOP/s (conv+bias+ReLU through Conv2D::forward, incl. repack)",
        "value": hr["tflops"], "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": hr["us_per_call"] / 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (SplitMix64 seed 0x1234ABCD; x U[-1,1], w U[-1,1]/sqrt(K), b U[-0.1,0.1])",
        "config": {"workload": "BASELINE configs[1]: FP16 NCHW 3x3 conv N=32 C=256 H=W=14 K=256 s1 p1 + bias + ReLU",
                   "gemm_view": hr["gemm_view"], "kernel": hr["kernel"], "selection": hr["selection"],
                   "pct_of_fp16_peak": hr["pct_of_fp16_peak"], "us_per_call": hr["us_per_call"],
                   "median_protocol_us_per_call": hr["median_protocol"]["us_per_call"],
                   "median_protocol_tflops": hr["median_protocol"]["tflops"]},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_FP16_TFLOPS, "traffic": load_traffic(hr["kernel"]),
                     "kernel": dominant_kernel(hr["kernel"]), "avg_launch_us": gemm_us,
                     "flop_per_launch": p.flops()},
        "cpu_baseline": cpu,
        "host_cost": host,
        "parity": {"rel_l2": hr["rel_l2"], "max_abs": hr["max_abs"], "ok": hr["parity_ok"],
                   "against": "library GPU double reference on the timed call's inputs"},
        "configs": results,
        "repack_kernels": repack,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
