"""The cost model on a described MI355X (no GPU needed): it must route each benchmark layer to the kernel family
measured fastest there, classify the reference's bound cases (tests/test_perf_model.cpp's compute / bandwidth /
launch examples) the same way, rank deterministically, and count workgroup waves per XCD.

The family efficiencies and per-wave costs inside the model were fitted to MI355X per-call times of these layers;
these tests pin the resulting choices so a change to the model or to a family's registration that flips a routing
decision is caught here rather than in the benchmark.
"""
import math

import pytest

import gie

P = gie.Problem

BENCH = {
    # layer: (problem, family the model must pick, family measured fastest on the MI355X)
    "c2_fp16_3x3": (P(32, 256, 14, 14, 256, 3, 3, 1, 1, 1, 1, precision="fp16", has_bias=True, relu=True), "slab_"),
    "c3_fp16_1x1": (P(64, 256, 28, 28, 1024, 1, 1, 1, 1, 0, 0, precision="fp16", has_bias=True, relu=True), "pw_"),
    "c4_fp16_7x7s2": (P(64, 3, 224, 224, 64, 7, 7, 2, 2, 3, 3, precision="fp16", has_bias=True, relu=True), "stem_"),
    "c5_bf16_3x3": (P(8, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1, precision="bf16", has_bias=True, relu=True), "deep_"),
}


@pytest.mark.parametrize("layer", list(BENCH))
def test_model_routes_benchmark_layers_to_the_measured_fastest_family(layer):
    p, family = BENCH[layer]
    ranked = gie.model_rank(p)
    assert ranked, layer
    assert ranked[0][0].startswith(family), (layer, ranked[:3])
    prec = p.precision
    assert all(f"_{prec}_" in n for n, _ in ranked)


def test_model_bound_classification():
    k16, k16_big = "mfma_fp16_64x64x32_w2x2_s4_sk1", "mfma_fp16_128x128x64_w4x2_s3_sk1"
    assert gie.model_estimate(k16_big, P(32, 256, 28, 28, 256, 3, 3, 1, 1, 1, 1))["bound"] == "compute"
    assert gie.model_estimate(k16, P(32, 8, 224, 224, 8, 1, 1, 1, 1, 0, 0))["bound"] == "bandwidth"
    assert gie.model_estimate(k16, P(1, 8, 4, 4, 8, 1, 1, 1, 1, 0, 0))["bound"] == "launch"


def test_model_ranking_is_sorted_and_deterministic():
    p = P(8, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1)
    a, b = gie.model_rank(p), gie.model_rank(p)
    assert a == b and len(a) > 10
    us = [u for _, u in a]
    assert us == sorted(us) and all(u > 0 for u in us)


def test_model_counts_waves_per_xcd():
    # slab entries: one workgroup per (image, 32-filter block) slab; 33 images x 8 blocks = 264 workgroups deal 33
    # to each XCD, whose 32 CUs take them in two waves: efficiency 264 / (2 x 32 x 8)
    p = P(33, 256, 14, 14, 256, 3, 3, 1, 1, 1, 1)
    e = gie.model_estimate("slab_fp16_3x3_32x14r16_k32_s3_sk1", p)
    assert math.isclose(e["wave_efficiency"], 264 / 512, rel_tol=1e-12)
    full = gie.model_estimate("slab_fp16_3x3_32x14r16_k32_s3_sk1", P(32, 256, 14, 14, 256, 3, 3, 1, 1, 1, 1))
    assert full["wave_efficiency"] == 1.0
    # 14x14 images in 14-row x 16-pitch slabs: 196 of 224 positions are output pixels
    assert math.isclose(full["tile_efficiency"], 196 / 224, rel_tol=1e-12)
    # half the part (CUs and every ceiling halved): the same launch runs in two waves, and its compute time doubles
    half = gie.model_estimate("slab_fp16_3x3_32x14r16_k32_s3_sk1", P(32, 256, 14, 14, 256, 3, 3, 1, 1, 1, 1),
                              dict(cus=128, mfma_tflops=2516.6 / 2, fp32_tflops=157.3 / 2, hbm_gbs=4000.0))
    assert half["wave_efficiency"] == 1.0
    assert math.isclose(half["compute_us"], 2 * full["compute_us"], rel_tol=1e-12)


def test_model_rejects_a_bad_device_description():
    with pytest.raises(gie.GieError):
        gie.model_rank(P(1, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1), dict(cus=0))
