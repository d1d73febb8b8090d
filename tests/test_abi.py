"""C-ABI checks that need no GPU: both libraries load, every function the public headers declare is exported
and bound by the Python layer, and the host-side logic behind the boundary (problem validation, problem keys,
the library's CPU reference, the seeded data generator, the tile table) agrees with the oracle.

Reference behaviour followed: conv2d.cpp:77-109 (key and validation), cpu_reference.cpp:13-56,
testing.cu:75-105 (data generator), tensor_core_mma.cu:370-388 (tile table)."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

import gie
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = {"gie_capi.h": gie.LIBGIE, "gie_hip.h": gie.LIBGIE_HIP}


def declared(header: str) -> list[str]:
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(gie_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_every_declared_symbol_is_exported(header):
    names = declared(header)
    assert len(names) > 10
    lib = ctypes.CDLL(HEADERS[header], mode=ctypes.RTLD_GLOBAL)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_headers():
    bound = set(gie._CAPI) | set(gie._HIP)
    for header in HEADERS:
        missing = [n for n in declared(header) if n not in bound]
        assert not missing, (header, missing)
    gie.libs()  # argtypes/restype applied to every bound symbol


def _problems(rng, n):
    """Random problems around the validation boundaries (zero, negative, oversize padding, dilation, groups)."""
    good = ((1, 4), (1, 9), (1, 12), (1, 12), (1, 9), (1, 6), (1, 6), (1, 4), (1, 4), (0, 5), (0, 5), (1, 2),
            (1, 2), (1, 2))
    bad = ((-1, 1), (-1, 1), (-1, 1), (-1, 1), (-1, 1), (-1, 1), (-1, 1), (-1, 1), (-1, 1), (-2, 0), (-2, 0),
           (0, 4), (0, 4), (0, 4))
    out = []
    for _ in range(n):
        v = [int(rng.integers(*g)) for g in good]
        for f in rng.choice(len(v), size=int(rng.integers(0, 3)), replace=False):
            v[f] = int(rng.integers(*bad[f]))
        out.append(v)
    return out


def test_validation_matches_oracle():
    rng = np.random.default_rng(7)
    seen = {0: 0, 1: 0, 2: 0}
    for v in _problems(rng, 3000):
        c = O.Conv(*v)
        expect = O.validate(c)
        p = gie.Problem(*v)
        pc = p.c()
        got = gie.capi().gie_validate_problem(ctypes.byref(pc))
        assert got == expect, (v, got, expect)
        seen[expect] += 1
    assert min(seen.values()) > 20, seen  # every outcome exercised


def test_problem_key_is_injective_on_geometry_and_flags():
    base = dict(batch=2, in_channels=8, in_h=9, in_w=10, out_channels=4, kernel_h=3, kernel_w=3, stride_h=1,
                stride_w=1, pad_h=1, pad_w=1)
    keys = {gie.Problem(**base).key()}
    for f in base:
        d = dict(base)
        d[f] += 1
        keys.add(gie.Problem(**d).key())
    keys.add(gie.Problem(**base, precision="bf16").key())
    keys.add(gie.Problem(**base, has_bias=False).key())
    keys.add(gie.Problem(**base, relu=False).key())
    assert len(keys) == len(base) + 4


@pytest.mark.parametrize("shape", [(1, 3, 8, 8, 4, 3, 3, 1, 1, 1, 1), (2, 7, 11, 13, 9, 3, 3, 2, 2, 0, 0),
                                   (1, 4, 12, 12, 6, 1, 3, 1, 1, 0, 1), (2, 5, 9, 7, 3, 5, 5, 2, 1, 2, 2)])
@pytest.mark.parametrize("bias,relu", [(True, True), (False, False)])
def test_library_cpu_reference_matches_oracle(shape, bias, relu):
    c = O.P(*shape, has_bias=bias, relu=relu, precision="fp32")
    x, w, b = O.make_data(c, 11, O.NORMAL)
    yo, so = O.conv2d(c, x, w, b if bias else None)
    p = gie.Problem(*shape, precision="fp32", has_bias=bias, relu=relu)
    yl, sl = gie.cpu_reference(p, x, w, b if bias else None)
    np.testing.assert_allclose(yl, yo, rtol=0, atol=1e-5 * max(1.0, float(np.abs(so).max())))
    np.testing.assert_allclose(sl, so, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("precision", ["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("dist", [O.UNIFORM, O.NORMAL, O.SPARSE, O.POSITIVE])
def test_host_data_generator_matches_oracle_bit_exact(precision, dist):
    shape = (2, 5, 6, 7, 3, 3, 3, 1, 1, 1, 1)
    c = O.P(*shape, precision=precision)
    xo, wo, bo = O.make_data(c, 0xBEEF, dist, O.SCALING_BENCH)
    p = gie.Problem(*shape, precision=precision)
    xl, wl, bl = gie.make_host_data(p, 0xBEEF, dist=["uniform", "normal", "sparse_signed", "positive"][dist],
                                    scaling="benchmark")
    for a, b_ in ((xl, xo), (wl, wo), (bl.reshape(-1), bo)):
        assert np.array_equal(a.reshape(-1).view(np.uint32), b_.reshape(-1).view(np.uint32))


def test_tile_table_is_consistent():
    cfgs = gie.igemm_configs()
    assert len(cfgs) >= 8
    for c in cfgs:
        assert c["threads"] == 64 * c["waves_m"] * c["waves_n"]
        assert c["tile_k"] % 32 == 0
        assert c["tile_m"] % (16 * c["waves_m"]) == 0 and c["tile_n"] % (16 * c["waves_n"]) == 0
        assert 0 < c["lds_bytes"] <= 160 * 1024


def test_status_strings_and_fingerprint():
    for rc in (0, -1, -2):
        assert gie.hip().gie_hip_status_string(rc)
    for rc in range(7):
        assert gie.capi().gie_status_string(rc)
    assert len(gie.build_fingerprint()) > 8


def test_stem_geometry_check_on_host():
    """gie_hip_stem_check is host arithmetic: every shape the GPU stem tests launch qualifies within the LDS limit,
    and the geometries the kernel cannot run are refused."""
    ok = [(2, 3, 32, 32, 64), (1, 1, 16, 16, 20), (3, 2, 17, 32, 70), (2, 4, 40, 48, 128), (1, 3, 9, 16, 64),
          (1, 4, 6, 304, 64), (1, 4, 6, 464, 64), (2, 4, 9, 464, 64), (1, 3, 4, 512, 64), (4, 3, 64, 64, 32),
          (2, 3, 30, 48, 64), (64, 3, 224, 224, 64)]
    for B, C, H, W, K in ok:
        p = gie.Problem(B, C, H, W, K, 7, 7, 2, 2, 3, 3, precision="fp16")
        lds = ctypes.c_int(0)
        assert gie.hip().gie_hip_stem_check(ctypes.byref(p.geom(C)), ctypes.byref(lds)) == 0, (B, C, H, W, K)
        assert 0 < lds.value <= 160 * 1024
    for p in (gie.Problem(2, 3, 32, 32, 64, 5, 5, 2, 2, 2, 2, precision="fp16"),
              gie.Problem(2, 3, 32, 32, 64, 7, 7, 1, 1, 3, 3, precision="fp16"),
              gie.Problem(2, 5, 32, 32, 64, 7, 7, 2, 2, 3, 3, precision="fp16"),
              gie.Problem(2, 3, 32, 40, 64, 7, 7, 2, 2, 3, 3, precision="fp16"),
              gie.Problem(1, 4, 6, 480, 64, 7, 7, 2, 2, 3, 3, precision="fp16"),
              gie.Problem(1, 3, 6, 528, 64, 7, 7, 2, 2, 3, 3, precision="fp16")):
        assert gie.hip().gie_hip_stem_check(ctypes.byref(p.geom(p.in_channels)), None) != 0


def test_narrow_geometry_check_on_host():
    """gie_hip_narrow_check is host arithmetic: the GPU narrow tests' shapes qualify within the LDS limit."""
    for B, C, H, W, K in [(2, 128, 5, 5, 40), (3, 256, 4, 4, 64), (1, 128, 14, 14, 96), (40, 128, 1, 1, 20),
                          (8, 512, 7, 7, 512), (2, 384, 6, 6, 33)]:
        p = gie.Problem(B, C, H, W, K, 3, 3, 1, 1, 1, 1, precision="bf16")
        lds = ctypes.c_int(0)
        assert gie.hip().gie_hip_narrow_check(ctypes.byref(p.geom(C)), ctypes.byref(lds)) == 0, (B, C, H, W, K)
        assert 0 < lds.value <= 160 * 1024
    p = gie.Problem(2, 1024, 56, 56, 64, 3, 3, 1, 1, 1, 1, precision="fp16")
    assert gie.hip().gie_hip_narrow_check(ctypes.byref(p.geom(1024)), None) != 0


def test_slab_configuration_table_on_host():
    """Every slab configuration answers its table query (the registry builds its entries from it) with a
    consistent shape, and the slab registry entries exist for both precisions and every split factor."""
    h = gie.hip()
    n = h.gie_hip_slab_config_count()
    assert n >= 4
    for i in range(n):
        c = gie.GieSlabConfig()
        assert h.gie_hip_slab_config_get(i, ctypes.byref(c)) == 0, i
        assert c.tile_m == 32 and c.tile_k == 32 and c.pitch in (8, 16, 32) and 2 <= c.stages <= 4
        # four multiplying waves; the split form (3) adds one loader wave per SIMD
        assert c.threads == (512 if c.form == 3 else 256)
        assert (c.rows // 2) * c.pitch % 16 == 0
        assert 0 < c.lds_bytes <= 160 * 1024
    assert h.gie_hip_slab_config_get(n, ctypes.byref(gie.GieSlabConfig())) != 0
    names = gie.registry()
    for prec in ("fp16", "bf16"):
        for sk in (1, 2, 4, 8):
            assert any(k.startswith(f"slab_{prec}_3x3_") and k.endswith(f"_sk{sk}") for k in names), (prec, sk)


def test_slab_geometry_check_on_host():
    """gie_hip_slab_check is host arithmetic: the GPU slab tests' shapes qualify for some configuration, and the
    geometries the kernel cannot run are refused by all."""
    h = gie.hip()
    n = h.gie_hip_slab_config_count()
    for B, C, H, W, K in [(2, 64, 14, 14, 32), (3, 128, 14, 14, 40), (2, 72, 13, 10, 20), (2, 72, 13, 7, 20),
                          (1, 64, 29, 14, 32), (2, 64, 7, 6, 32), (8, 512, 7, 7, 64), (2, 64, 28, 28, 48),
                          (1, 32, 5, 3, 8), (2, 8, 6, 6, 5), (32, 256, 14, 14, 256), (8, 512, 7, 7, 512)]:
        p = gie.Problem(B, C, H, W, K, 3, 3, 1, 1, 1, 1, precision="fp16")
        ok = 0
        for i in range(n):
            lds = ctypes.c_int(0)
            if h.gie_hip_slab_check(i, ctypes.byref(p.geom(C)), ctypes.byref(lds)) == 0:
                assert 0 < lds.value <= 160 * 1024
                ok += 1
        assert ok > 0, (B, C, H, W, K)
    for p in (gie.Problem(2, 64, 7, 7, 64, 5, 5, 1, 1, 2, 2, precision="fp16"),
              gie.Problem(2, 64, 7, 7, 64, 3, 3, 2, 2, 1, 1, precision="fp16"),
              gie.Problem(2, 132, 7, 7, 64, 3, 3, 1, 1, 1, 1, precision="fp16"),
              gie.Problem(1, 64, 8, 40, 32, 3, 3, 1, 1, 1, 1, precision="fp16")):
        for i in range(n):
            assert h.gie_hip_slab_check(i, ctypes.byref(p.geom(p.in_channels)), None) != 0


def test_stack_configuration_table_and_geometry_on_host():
    """The stack configurations answer their table query consistently, their registry entries exist for both
    precisions and every split factor, gie_hip_stack_check (host arithmetic) accepts the GPU stack tests' shapes with
    the images per unit the stack holds, and refuses what the kernel cannot run."""
    h = gie.hip()
    n = h.gie_hip_stack_config_count()
    assert n >= 1
    for i in range(n):
        c = gie.GieStackConfig()
        assert h.gie_hip_stack_config_get(i, ctypes.byref(c)) == 0, i
        assert c.tile_m == 32 and c.tile_k == 32 and c.pitch == 8 and c.halves in (1, 2) and c.threads == 256 * c.halves
        assert (c.rows // 2) * c.pitch % 16 == 0 and 0 < c.lds_bytes <= 160 * 1024
    assert h.gie_hip_stack_config_get(n, ctypes.byref(gie.GieStackConfig())) != 0
    names = gie.registry()
    for prec in ("fp16", "bf16"):
        for sk in (1, 2, 4, 8):
            assert any(k.startswith(f"stack_{prec}_3x3_") and k.endswith(f"_sk{sk}") for k in names), (prec, sk)
    rows = []
    for i in range(n):
        c = gie.GieStackConfig()
        h.gie_hip_stack_config_get(i, ctypes.byref(c))
        rows.append(c.rows)
    for B, C, H, W, K in [(8, 512, 7, 7, 64), (3, 64, 7, 7, 40), (5, 96, 6, 5, 20), (2, 32, 4, 4, 8),
                          (16, 64, 3, 7, 32), (4, 128, 7, 1, 16), (2, 64, 15, 7, 32), (6, 160, 5, 6, 48),
                          (1, 96, 2, 3, 33), (8, 512, 7, 7, 512)]:
        p = gie.Problem(B, C, H, W, K, 3, 3, 1, 1, 1, 1, precision="bf16")
        ok = 0
        for i in range(n):
            lds, ni = ctypes.c_int(0), ctypes.c_int(0)
            if h.gie_hip_stack_check(i, ctypes.byref(p.geom(C)), ctypes.byref(lds), ctypes.byref(ni)) == 0:
                assert ni.value == min(rows[i] // (H + 1), B), (i, B, H)
                ok += 1
        assert ok > 0, (B, C, H, W, K)
    for p in (gie.Problem(2, 64, 7, 7, 64, 5, 5, 1, 1, 2, 2, precision="fp16"),   # 5x5
              gie.Problem(2, 64, 7, 7, 64, 3, 3, 2, 2, 1, 1, precision="fp16"),   # stride 2
              gie.Problem(2, 72, 7, 7, 64, 3, 3, 1, 1, 1, 1, precision="fp16"),   # C % 32 != 0
              gie.Problem(2, 64, 7, 8, 64, 3, 3, 1, 1, 1, 1, precision="fp16"),   # rows wider than the pitch allows
              gie.Problem(1, 64, 40, 7, 32, 3, 3, 1, 1, 1, 1, precision="fp16")):  # images taller than every stack
        for i in range(n):
            assert h.gie_hip_stack_check(i, ctypes.byref(p.geom(p.in_channels)), None, None) != 0


@pytest.mark.parametrize("shape", [(1, 24, 9, 9, 4, 3, 3, 1, 1, 1, 1, 1), (2, 16, 7, 5, 8, 2, 3, 1, 1, 0, 0, 2),
                                   (1, 64, 14, 14, 32, 1, 1, 1, 1, 0, 0, 1), (1, 8, 30, 30, 4, 7, 7, 2, 2, 3, 3, 1)])
def test_gather_table_builders_match_oracle(shape):
    """build_conv_lut / build_conv_lut_chunked (kernel_registry.h:86-96) against the oracle's restatement of
    conv_common.cu:22-50, bit for bit, with and without dilation; the chunked form rejects C % 8 != 0."""
    B, C, H, W, Oc, Kh, Kw, Sh, Sw, Ph, Pw, dil = shape
    p = gie.Problem(B, C, H, W, Oc, Kh, Kw, Sh, Sw, Ph, Pw, precision="fp16", has_bias=False, relu=False)
    p.dilation_h = p.dilation_w = dil
    c = O.P(B, C, H, W, Oc, Kh, Kw, Sh, Sw, Ph, Pw, dilation_h=dil, dilation_w=dil)
    assert np.array_equal(gie.build_conv_lut(p), O.lut(c))
    assert np.array_equal(gie.build_conv_lut(p, chunked=True), O.lut_chunked(c))
    odd = gie.Problem(1, 12, 5, 5, 4, 3, 3, 1, 1, 1, 1, precision="fp16", has_bias=False, relu=False)
    with pytest.raises(gie.GieError):
        gie.build_conv_lut(odd, chunked=True)
    assert gie.build_conv_lut(odd).shape == (12 * 9, 4)


def test_splitk_reduce_form_keeps_partial_offsets_in_range():
    """The 32-bit reduce form indexes partial[z * total + i]: it may be chosen only while (total + 4) * split stays
    below 2^31 (a split-8 reduce over 300M outputs must take the 64-bit form). No launch: the host-side choice."""
    def form(total, split, vec=1, dtype=gie.PRECISIONS["fp16"]):
        bits, unrolled = ctypes.c_int(), ctypes.c_int()
        assert gie.hip().gie_hip_splitk_reduce_form(dtype, total, split, vec, ctypes.byref(bits),
                                                    ctypes.byref(unrolled)) == 0
        return bits.value, unrolled.value

    assert form(200_704, 2) == (32, 2)             # config 5 at split 2
    assert form(200_704, 3) == (32, 0)             # any other split: the run-time slice loop
    assert form(200_703, 4, vec=0) == (32, 0)      # unaligned: the scalar form
    for split in (2, 4, 8):
        limit = (1 << 31) // split - 4             # largest total whose offsets all fit an int
        assert form(limit - 1, split)[0] == 32
        assert form(limit, split)[0] == 64
        assert form(limit + 1000, split)[0] == 64
    assert form(307_000_000, 8)[0] == 64           # split 8 x 307M outputs: 2.46e9 > 2^31 - 1
    assert form(716_000_000, 4)[0] == 64
    assert form((1 << 30) - 4, 1)[0] == 64         # the magic-number divisions need n < 2^30
    assert form(1000, 4, dtype=gie.PRECISIONS["fp32"]) == (64, 0)
    bits = ctypes.c_int()
    assert gie.hip().gie_hip_splitk_reduce_form(gie.PRECISIONS["fp16"], 0, 2, 1, ctypes.byref(bits),
                                                ctypes.byref(bits)) != 0
