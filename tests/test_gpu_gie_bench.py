"""The gie_bench harness on the GPU: every row type of the reference's benchmarks/benchmark_main.cpp flow.

Two small workloads (a 3x3 and a 1x1 layer) at fp16, bf16 and fp32 through tensor_core and implicit_gemm (fixed
and tuned configurations), the dispatcher, a kernel named on the command line, the CPU reference and the copy
rows, fused and unfused. Checks that each GPU row validated against the double reference before it was timed and
carries positive timings, that the unfused rows (convolution + stand-alone bias and ReLU passes) validate under
the two-rounding tolerance, that a precision a backend has no kernel for gives an 'unsupported' row (tensor_core
is FP16/BF16/TF32, implicit_gemm FP32), and that the dispatcher row records its selection and the warm host
overhead.
"""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "cuda-inference_amd", "lib", "gie_bench")

pytestmark = pytest.mark.gpu


def test_gie_bench_rows_on_gpu(tmp_path):
    doc = {"split": "gpu_test", "workloads": [
        {"name": "l3x3", "category": "t", "B": 2, "C": 64, "H": 14, "O": 64, "K": 3, "P": 1},
        {"name": "l1x1", "category": "t", "B": 2, "C": 64, "H": 16, "O": 96, "K": 1, "relu": False},
    ]}
    wl = tmp_path / "w.json"
    wl.write_text(json.dumps(doc))
    out = tmp_path / "res"
    named = "mfma_fp16_64x64x64_w2x2_s4_sk1"
    cmd = [BIN, "--workloads", str(wl), "--backends", "tensor_core,implicit_gemm,dispatcher,cpu_reference,simt_tiled",
           "--precisions", "fp16,bf16,fp32", "--mode", "both", "--fusion", "both", "--kernels", named,
           "--warmup", "1", "--samples", "3", "--min-sample-ms", "0.2", "--tune-samples", "2", "--model-keep", "3",
           "--cache", str(tmp_path / "tune.json"), "--e2e", "--out", str(out), "--tag", "gpu"]
    print(" ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    print(p.stderr[-3000:], flush=True)
    assert p.returncode == 0, p.stderr[-2000:]
    rows = [json.loads(line) for line in open(out / "results.jsonl")]
    by = {}
    for r in rows:
        by.setdefault((r["workload"], r["precision"], r["backend"], r["fusion"], r["mode"]), []).append(r)

    for w in ("l3x3", "l1x1"):
        for prec in ("fp16", "bf16"):
            for mode in ("fixed", "tuned"):
                for fusion in ("fused", "unfused"):
                    (r,) = by[(w, prec, "tensor_core", fusion, mode)]
                    assert r["status"] == "ok", r
                    assert r["validated"] is True and r["nan_count"] == 0 and r["frac_over_tol"] == 0
                    assert r["median_us"] > 0 and r["tflops"] > 0 and r["samples"] == 3
                    if mode == "fixed":
                        assert r["kernel"].startswith(f"mfma_{prec}_128x128x64_w4x2_s3_sk1"), r["kernel"]
                    assert ("+bias+relu(unfused)" in r["kernel"]) == (fusion == "unfused")
                    assert r["host_sync_latency_us"] > 0
            (t,) = by[(w, prec, "tensor_core", "fused", "tuned")]
            assert "tuning_seconds" in t and "tuning_cache_hit" in t
            (d,) = by[(w, prec, "dispatcher", "fused", "auto")]
            assert d["status"] == "ok", d
            assert d["config"].startswith("selected ") and d["warm_dispatch_overhead_us"] == pytest.approx(
                d["dispatch_api_host_us"] - d["raw_launch_host_us"])
            (k,) = by[(w, prec, "kernel", "fused", "named")]
            if prec == "fp16":
                assert k["status"] == "ok" and k["kernel"] == named, k
            else:
                assert k["status"] == "unsupported" and "fp16" in k["reason"], k
            (c,) = by[(w, prec, "cpu_reference", "fused", "host")]
            assert c["status"] == "ok" and c["max_abs_err"] < 1e-5, c
            (s,) = by[(w, prec, "simt_tiled", "fused", "n/a")]
            assert s["status"] == "unsupported"
            (m,) = by[(w, prec, "memcpy", "n/a", "pinned")]
            assert m["status"] == "ok" and m["h2d_us"] > 0 and m["d2h_us"] > 0
        for mode in ("fixed", "tuned"):
            (f,) = by[(w, "fp32", "tensor_core", "fused", mode)]
            assert f["status"] == "unsupported", f
            for fusion in ("fused", "unfused"):
                (g,) = by[(w, "fp32", "implicit_gemm", fusion, mode)]
                assert g["status"] == "ok" and g["validated"] is True and g["tflops"] > 0, g
                assert g["kernel"].startswith("implicit_gemm_fp32_"), g
            for prec in ("fp16", "bf16"):
                (u,) = by[(w, prec, "implicit_gemm", "fused", mode)]
                assert u["status"] == "unsupported", u
        (fd,) = by[(w, "fp32", "dispatcher", "fused", "auto")]
        assert fd["status"] == "ok" and fd["config"].startswith("selected implicit_gemm_fp32_"), fd
    # the 3x3 fixed configuration is a two-launch kernel (repack + convolution): both stages are timed
    (r,) = by[("l3x3", "fp16", "tensor_core", "fused", "fixed")]
    assert r["stage_repack_us"] > 0 and r["stage_conv_us"] > 0 and "stage_reduce_us" not in r
    meta = json.load(open(out / "meta.json"))
    assert "gfx950" in meta["arch"] and meta["cu_count"] > 0


GRAPH_BIN = os.path.join(ROOT, "cuda-inference_amd", "lib", "gie_graph_bench")


@pytest.mark.parametrize("precision", ["fp16", "bf16"])
def test_graph_bench_chain_records(tmp_path, precision):
    """gie_graph_bench (the reference's benchmarks/graph_bench.cpp measurements): for the first chain case at two
    depths, the graph replays reproduce the eager chain bit for bit, the graph holds one node per layer launch, and
    every timing is positive; the stream-concurrency rows cover 2, 4 and 8 independent convolutions."""
    cmd = [GRAPH_BIN, "--out", str(tmp_path), "--precision", precision, "--cases", "1", "--depths", "1,4"]
    print(" ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    print(p.stdout[-2000:], p.stderr[-2000:], flush=True)
    assert p.returncode == 0, p.stderr[-2000:]
    rows = [json.loads(line) for line in open(tmp_path / "graphs.jsonl")]
    chains = [r for r in rows if r["experiment"] == "F_hip_graphs"]
    assert [r["layers"] for r in chains] == [1, 4]
    for r in chains:
        assert r["case"] == "b1_c32_14x14_k3" and r["precision"] == precision
        assert r["bitwise_identical_replays"] is True
        assert r["graph_nodes"] >= r["layers"]
        for k in ("capture_us", "instantiate_us", "eager_device_us", "graph_device_us", "eager_host_launch_us",
                  "graph_host_launch_us"):
            assert r[k] > 0, (k, r)
    conc = [r for r in rows if r["experiment"] == "F_stream_concurrency"]
    assert [r["independent_convs"] for r in conc] == [2, 4, 8]
    assert all(r["one_stream_us"] > 0 and r["multi_stream_us"] > 0 for r in conc)
