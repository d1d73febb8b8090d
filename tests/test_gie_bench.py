"""The gie_bench harness on the CPU: workload-file loading, selection flags and the result-file schema.

* the workload schema of the reference's benchmarks/benchmark_main.cpp:148-181 — W defaults to H, O to C,
  Kh/Kw to K (3), Sh/Sw to S (1), Ph/Pw to P (0), bias/relu to true; explicit Kh/Kw/Sh/Sw/Ph/Pw win over K/S/P;
  --filter (substring of the name), --category (exact) and --max-workloads;
* results.csv carries exactly the reference's column list (benchmark_main.cpp:183-192) in that order, with
  booleans as 1/0, absent fields empty and RFC 4180 quoting; results.jsonl holds one JSON object per row;
* a cpu_reference-only run needs no GPU, and every requested backend gets a row (the reference's backends that
  have no MI355X counterpart as 'unsupported' with a reason);
* command-line errors exit with status 1.
"""
import csv
import io
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cuda-inference_amd")
BIN = os.path.join(PKG, "lib", "gie_bench")
WORKLOADS = os.path.join(PKG, "examples", "workloads.json")

# benchmarks/benchmark_main.cpp:183-192
REFERENCE_COLUMNS = (
    "tag,gpu,cc,workload,category,split,B,C,H,W,O,Kh,Kw,Sh,Sw,Ph,Pw,precision,bias,relu,fusion,backend,mode,kernel,"
    "status,reason,median_us,mean_us,min_us,p10_us,p90_us,p99_us,stddev_us,samples,inner_iters,images_per_s,tflops,"
    "workspace_bytes,persistent_bytes,tuning_seconds,tuning_cache_hit,setup_seconds,max_abs_err,frac_over_tol,"
    "worst_tol_ratio,flops,compulsory_bytes,arithmetic_intensity,model_pred_us,roofline_bound,conv_only_us,"
    "layout_inclusive_us,src_fp,warmup,layout,stage_im2col_us,stage_gemm_us,host_sync_latency_us,flush_l2,config"
).split(",")

pytestmark = pytest.mark.skipif(not os.path.exists(BIN), reason="gie_bench not built (run __graft_entry__.build())")


def run(*args, check=True):
    # the harness must not need a GPU for these runs
    env = dict(os.environ, HIP_VISIBLE_DEVICES="")
    p = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=300, env=env)
    if check:
        assert p.returncode == 0, p.stderr
    return p


def listed(path, *flags):
    out = run("--workloads", path, "--list", *flags).stdout
    return [line.split("\t") for line in out.splitlines()]


def test_committed_workloads_hold_the_baseline_configs():
    rows = listed(WORKLOADS, "--category", "baseline")
    assert [r[2] for r in rows] == [
        "B1_C64_56x56_O64_K3x3_s1x1_p1x1_d1x1_g1",
        "B32_C256_14x14_O256_K3x3_s1x1_p1x1_d1x1_g1",
        "B64_C256_28x28_O1024_K1x1_s1x1_p0x0_d1x1_g1",
        "B64_C3_224x224_O64_K7x7_s2x2_p3x3_d1x1_g1",
        "B8_C512_7x7_O512_K3x3_s1x1_p1x1_d1x1_g1",
    ]
    with open(WORKLOADS) as f:
        doc = json.load(f)
    assert len(listed(WORKLOADS)) == len(doc["workloads"])


def test_workload_defaults_and_overrides(tmp_path):
    doc = {"split": "dev", "workloads": [
        {"name": "only_h", "B": 2, "C": 5, "H": 9},                                   # W=H, O=C, 3x3 s1 p0
        {"name": "k_s_p", "C": 4, "H": 10, "W": 12, "O": 6, "K": 5, "S": 2, "P": 2, "category": "x"},
        {"name": "explicit", "C": 4, "H": 10, "K": 5, "Kh": 1, "Kw": 7, "S": 2, "Sw": 1, "P": 1, "Pw": 3},
        {"category": "x", "C": 8, "H": 4, "K": 1},                                    # unnamed
    ]}
    path = tmp_path / "w.json"
    path.write_text(json.dumps(doc))
    rows = listed(str(path))
    assert rows == [
        ["only_h", "uncategorized", "B2_C5_9x9_O5_K3x3_s1x1_p0x0_d1x1_g1"],
        ["k_s_p", "x", "B1_C4_10x12_O6_K5x5_s2x2_p2x2_d1x1_g1"],
        ["explicit", "uncategorized", "B1_C4_10x10_O4_K1x7_s2x1_p1x3_d1x1_g1"],
        ["unnamed", "x", "B1_C8_4x4_O8_K1x1_s1x1_p0x0_d1x1_g1"],
    ]
    assert [r[0] for r in listed(str(path), "--category", "x")] == ["k_s_p", "unnamed"]
    assert [r[0] for r in listed(str(path), "--filter", "_")] == ["only_h", "k_s_p"]
    assert [r[0] for r in listed(str(path), "--max-workloads", "1", "--filter", "e")] == ["explicit"]


def _read(out):
    with open(os.path.join(out, "results.csv"), newline="") as f:
        text = f.read()
    rows = list(csv.reader(io.StringIO(text)))
    with open(os.path.join(out, "results.jsonl")) as f:
        jl = [json.loads(line) for line in f]
    return text, rows, jl


def test_cpu_only_run_writes_the_reference_schema(tmp_path):
    doc = {"split": "unit", "workloads": [
        {"name": "tiny_a", "category": "t", "B": 1, "C": 3, "H": 6, "O": 4, "K": 3, "P": 1},
        {"name": "tiny_b", "category": "t", "B": 2, "C": 2, "H": 5, "W": 4, "O": 3, "K": 1, "bias": False},
        {"name": "big", "category": "t", "B": 8, "C": 256, "H": 56, "O": 256, "K": 3, "P": 1},
    ]}
    path = tmp_path / "w.json"
    path.write_text(json.dumps(doc))
    out = str(tmp_path / "res")
    p = run("--workloads", str(path), "--backends", "cpu_reference,direct,cudnn", "--precisions", "fp32,fp16",
            "--out", out, "--tag", "unit", "--seed", "7")
    assert "3 workloads" in p.stderr
    text, rows, jl = _read(out)
    assert rows[0] == REFERENCE_COLUMNS
    body = rows[1:]
    assert len(body) == len(jl) == 3 * 2 * 3  # workloads x precisions x backends, nothing dropped
    col = {c: i for i, c in enumerate(REFERENCE_COLUMNS)}
    for r, j in zip(body, jl):
        assert len(r) == len(REFERENCE_COLUMNS)
        assert r[col["tag"]] == "unit" and r[col["split"]] == "unit" and r[col["gpu"]] == "none"
        assert r[col["workload"]] == j["workload"] and r[col["backend"]] == j["backend"]
        assert r[col["bias"]] == ("1" if j["bias"] else "0") and r[col["flush_l2"]] == "0"
        assert float(r[col["flops"]]) == j["flops"] > 0
        if j["backend"] == "cpu_reference" and j["workload"] != "big":
            assert j["status"] == "ok", j
            assert j["kernel"] == "cpu_reference(double accum, OpenMP)"
            assert r[col["kernel"]] == j["kernel"]  # the comma forces quoting; csv reads it back whole
            assert j["median_us"] > 0 and j["samples"] == 1 and j["tflops"] > 0
        elif j["backend"] == "cpu_reference":
            assert j["status"] == "unsupported" and "--cpu-max-gflop" in j["reason"]
        else:
            assert j["status"] == "unsupported" and j["reason"].startswith(j["backend"] + ":")
            assert r[col["median_us"]] == "" and r[col["kernel"]] == ""
    assert '"cpu_reference(double accum, OpenMP)"' in text
    b = [j for j in jl if j["workload"] == "tiny_b"][0]
    assert (b["B"], b["C"], b["H"], b["W"], b["O"], b["Kh"], b["Kw"], b["Ph"], b["bias"], b["relu"]) == \
        (2, 2, 5, 4, 3, 1, 1, 0, False, True)
    meta = json.load(open(os.path.join(out, "meta.json")))
    assert meta["gpu"] == "none" and meta["seed"] == 7 and meta["precisions"] == ["fp32", "fp16"]

    # a second run appends rows under the same single header
    run("--workloads", str(path), "--backends", "cpu_reference", "--precisions", "fp16", "--filter", "tiny_a",
        "--out", out)
    _, rows2, jl2 = _read(out)
    assert rows2[0] == REFERENCE_COLUMNS and len(rows2) == len(rows) + 1 and len(jl2) == len(jl) + 1
    assert sum(1 for r in rows2 if r == REFERENCE_COLUMNS) == 1


@pytest.mark.parametrize("args", [["--bogus"], ["--mode", "sometimes"], ["--fusion", "half"], ["--samples"],
                                  ["--precisions", "fp8"], ["--scaling", "huge"]])
def test_bad_command_lines_exit_1(args):
    p = run("--workloads", WORKLOADS, "--list", *args, check=False)
    assert p.returncode == 1 and "fatal:" in p.stderr


def test_workload_file_without_a_list_is_an_error(tmp_path):
    path = tmp_path / "bad.json"
    path.write_text(json.dumps({"version": 1}))
    p = run("--workloads", str(path), "--list", check=False)
    assert p.returncode == 1 and "workloads" in p.stderr
