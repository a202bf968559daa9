"""C-ABI and host-logic checks that need no GPU.

The library must load and export every entry point declared in
include/lighthouse_hip.h; host-side geometry and argument validation run
without launching anything; the Python API exposes the names the reference's
model wiring imports (lighthouse-attention.patch:591-598).
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from oracle import lh_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lighthouse_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    for n in ["lh_pyramid_fwd", "lh_select_topk", "lh_attn_fwd", "lh_attn_bwd", "lh_scatter_fwd",
              "lh_scatter_bwd", "lh_pyramid_bwd", "lh_dilated_scores", "lh_select_geometry"]:
        assert n in names


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg._native.lib()
    for n in _declared():
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert set(_declared()) == set(pkg._native.EXPORTED)


def test_abi_version_matches_header(pkg):
    """The header's LH_ABI_VERSION is what the built library reports, so a C
    caller can compare the two at start-up."""
    with open(HEADER) as f:
        m = re.search(r"#define\s+LH_ABI_VERSION\s+(\d+)", f.read())
    assert m, "LH_ABI_VERSION is not defined in the header"
    assert pkg._native.lib().lh_abi_version() == int(m.group(1))


def test_attention_schedule_switch(pkg):
    """Host-only: the schedule flags round-trip, unknown bits are refused and
    leave the setting alone, and the default is restored."""
    lib = pkg._native.lib()
    prev = ctypes.c_int(-1)
    assert lib.lh_attn_set_schedule(3, ctypes.byref(prev)) == 0
    assert prev.value == 0
    assert lib.lh_attn_set_schedule(4, ctypes.byref(prev)) == 1  # LH_ERR_INVALID_ARG
    assert lib.lh_attn_set_schedule(1, ctypes.byref(prev)) == 0
    assert prev.value == 3
    assert pkg._native.set_attention_schedule() == (False, True)
    assert pkg._native.set_attention_schedule() == (True, True)


def test_gla_workspace_geometry(pkg):
    """Host-only size query of the segmented GLA walk: one segment needs no
    workspace; otherwise (P - 1) fp32 128 x 128 states plus one decay per
    (b, virtual head, direction); invalid geometry gives -1."""
    f = pkg._native.lib().lh_gla_workspace_bytes
    units = 1 * 4 * 8 * 2  # cfg2 with dilation 4: B * dilation * H * 2
    assert f(1, 32768, 8, 128, 4, 0) == units * 3 * (128 * 128 + 1) * 4  # 4 segments of 32 chunks
    assert f(1, 32768, 8, 128, 4, 1) == 0
    assert f(1, 32768, 8, 128, 4, 6) == units * 5 * (128 * 128 + 1) * 4  # 128 chunks: 22 per segment, 6 segments
    assert f(1, 32768, 8, 128, 4, 100000) == units * 127 * (128 * 128 + 1) * 4  # clamped to one chunk each
    assert f(1, 1024, 2, 128, 4, 0) == 0  # 4 chunks: one walk
    assert f(1, 8188 * 4, 2, 128, 4, 0) == (1 * 4 * 2 * 2) * 3 * (128 * 128 + 1) * 4  # 128 chunks, last ragged: 4
    assert f(64, 32768, 8, 128, 4, 0) == 64 * units * 3 * (128 * 128 + 1) * 4  # per-sequence rule: 4 segments
    assert f(1, 1000, 1, 128, 3, 0) == -1  # S not a multiple of the dilation
    assert f(1, 1024, 1, 64, 4, 0) == -1  # D != 128
    assert f(0, 1024, 1, 128, 4, 0) == -1


def test_strerror(pkg):
    lib = pkg._native.lib()
    for rc in range(6):
        assert b"unknown" not in lib.lh_strerror(rc)
    assert b"unknown" in lib.lh_strerror(99)


@pytest.mark.parametrize("geo", [(32768, 3, 4, 2048), (4096, 3, 4, 256), (4096, 3, 4, 1536), (65536, 3, 4, 1536),
                                 (65536, 3, 4, 3072), (65536, 3, 4, 6144), (131072, 5, 2, 1536),
                                 (32768, 3, 4, 1536), (5000, 3, 4, 256), (2048, 2, 2, 128), (98304, 3, 4, 4096)])
def test_geometry_matches_oracle(pkg, geo):
    S, L, p, k = geo
    g = O.tile_geometry(S, L, p, k)
    T, NCC, per_tile, S_sel = pkg._native.geometry(S, L, p, k, strict=False)
    assert (T, NCC, per_tile, S_sel) == (g.T, g.NCC, g.per_tile, g.S_sel)
    if g.strict_ok:
        assert pkg._native.geometry(S, L, p, k, strict=True)[3] == g.S_sel
        assert g.S_sel == pkg.compute_output_indices_selection(S, L, p, k)
    else:
        with pytest.raises(AssertionError):
            pkg._native.geometry(S, L, p, k, strict=True)


def test_host_validation_rejects_before_launch(pkg):
    lib = pkg._native.lib()
    null = ctypes.c_void_p(0)
    # unsupported head dim, null pointers, bad tie mode: all refused on the host
    assert lib.lh_attn_fwd(null, null, null, 0, 0, 0, null, null, null, 0, 0, 0, 0, null,
                           1, 1, 128, 64, ctypes.c_float(0.1), null, null, 0, null) == 4
    assert lib.lh_attn_fwd(null, null, null, 0, 0, 0, null, null, null, 0, 0, 0, 0, null,
                           1, 1, 128, 128, ctypes.c_float(0.1), null, null, 0, null) == 1
    assert lib.lh_select_topk(null, null, null, null, 1, 1, 4096, 3, 4, 256, 0, 1, null) == 1
    assert lib.lh_pyramid_fwd(null, null, null, 0, 0, 0, null, null, null, 0, 0, 0, null, null,
                              1, 1024, 1, 128, 3, 4, 0, 0, null) == 1
    assert lib.lh_scatter_fwd(null, null, null, 0, 0, 0, 1, 1, 1024, 1024, 10, 64, 3, 4, 0, null) == 4
    assert lib.lh_pyramid_bwd(null, null, null, 0, 0, 0, null, null, null, null, 1, 1024, 1, 128, 3, 3,
                              0, null) == 1
    # an element type other than LH_DTYPE_BF16 (0) / LH_DTYPE_F16 (1) is refused
    fake = ctypes.c_void_p(64)  # never dereferenced: every call below is refused first
    assert lib.lh_scatter_fwd(fake, fake, fake, 128, 128, 128, 1, 1, 1024, 1024, 10, 128, 3, 4, 2, null) == 1
    assert lib.lh_scatter_bwd(fake, 128, 128, 128, fake, null, fake, null, 1, 1, 1024, 1024, 10, 128, 3, 4, 7,
                              null) == 1
    assert lib.lh_pyramid_fwd(fake, fake, fake, 128, 128, 128, fake, fake, fake, 128, 128, 128, fake, fake,
                              1, 1024, 1, 128, 3, 4, 0, 2, null) == 1
    assert lib.lh_pyramid_bwd(fake, null, null, 128, 128, 128, null, fake, null, null, 1, 1024, 1, 128, 3, 4,
                              -1, null) == 1
    assert lib.lh_dilated_scores(fake, fake, fake, fake, fake, 1, 1024, 1, 128, 4, 1024, ctypes.c_float(0.1), 3,
                                 null) == 1
    assert lib.lh_select_geometry(4096, 3, 4, 1536, 1, None, None, None, None) == 2
    assert lib.lh_select_geometry(4096, 1, 4, 256, 0, None, None, None, None) == 1
    # transformer-block kernels
    assert lib.lh_rope_qkv_fwd(null, 3072, null, null, null, null, 1, 16, 8, 8, 128, null) == 1
    assert lib.lh_rope_pyramid_fwd(null, null, null, 0, 0, 0, null, null, null, 0, 0, 0, null, null, null,
                                   0, 0, 0, null, null, 1, 1024, 1, 128, 3, 4, null) == 1
    assert lib.lh_rope_pyramid_fwd(null, null, null, 0, 0, 0, fake, null, null, 0, 0, 0, null, null, null,
                                   0, 0, 0, null, null, 1, 1024, 1, 128, 3, 4, null) == 1
    assert lib.lh_rope_pyramid_fwd(fake, fake, fake, 384, 384, 128, fake, null, fake, 384, 384, 128, fake, fake,
                                   fake, 128, 128, 128, fake, fake, 1, 1024, 1, 128, 3, 4, null) == 1  # rq null
    assert lib.lh_pyramid_rope_bwd(null, null, null, 0, 0, 0, null, null, null, null, null, 0, 0, 0,
                                   1, 1024, 1, 128, 3, 4, null) == 1  # freqs null
    assert lib.lh_pyramid_rope_bwd(fake, null, null, 8, 8, 8, null, fake, null, null, null, 8, 8, 8,
                                   1, 1024, 1, 128, 3, 4, null) == 1  # grad without output
    assert lib.lh_rope_qkv_bwd(null, null, null, null, null, null, 3072, 1, 16, 8, 8, 128, null) == 1
    assert lib.lh_rmsnorm_fwd(null, null, null, null, 16, 1024, ctypes.c_float(1e-5), null) == 1
    assert lib.lh_rmsnorm_bwd(null, null, null, null, null, null, null, null, 4, 16, 1024, null) == 1
    assert lib.lh_add_rmsnorm_fwd(null, null, null, null, null, null, 16, 1024, ctypes.c_float(1e-5), null) == 1
    assert lib.lh_swiglu_fwd(null, null, 16, 1024, null) == 1
    assert lib.lh_swiglu_bwd(null, null, null, 16, 1000, null) == 1
    assert lib.lh_splitk_sum(null, null, 4, 1024, null) == 1
    # a row too long for one wave's registers is refused as unsupported
    x = (ctypes.c_uint16 * 1024)()
    r = (ctypes.c_float * 4)()
    ptr = ctypes.cast(x, ctypes.c_void_p)
    assert lib.lh_rmsnorm_fwd(ptr, ptr, ptr, ctypes.cast(r, ctypes.c_void_p), 1, 8192,
                              ctypes.c_float(1e-5), null) in (1, 4)


def test_no_cpu_fallback(pkg):
    x = torch.zeros(1, 256, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(pkg._native.LighthouseHipError):
        pkg._native.pyramid_fwd(x, x, x, 2, 2)
    with pytest.raises(pkg._native.LighthouseHipError):
        pkg.lighthouse_layer(x, x, x, num_levels=2, pooling_factor=2, topk=128)


def test_product_code_does_not_import_the_oracle():
    pkg_dir = os.path.join(ROOT, "lighthouse-attention_amd")
    for dirpath, _, files in os.walk(pkg_dir):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle", text, flags=re.M), f
                assert "select_ref" not in text and "lh_oracle" not in text, f


def test_reference_import_names_and_constructors(pkg):
    for name in ["DilatedLighthouseScorer", "DialatedLighthouseNormScorer", "DilatedLighthouseGLAScorer",
                 "LighthouseLocal", "DialatedLighthouseNormScorerCP", "LighthouseCP"]:
        assert hasattr(pkg, name)
    norm = pkg.DialatedLighthouseNormScorer(pooling_factor=4, levels=3)
    dil = pkg.DilatedLighthouseScorer(head_dim=128, dilation=4, pooling_factor=4, levels=3)
    assert dil.attention is None and dil.dilation == 4
    layer = pkg.LighthouseLocal(scorer=norm, num_levels=3, pooling_factor=4, topk=2048, attention=None)
    assert layer.topk == 2048 and layer.tie_break == "reference" and layer.strict
    gla = pkg.DilatedLighthouseGLAScorer(head_dim=128)
    assert gla.dilation == 4 and abs(gla.scaling - 128 ** -0.5) < 1e-12
    x = torch.zeros(1, 64, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(pkg._native.LighthouseHipError):  # no CPU path
        gla(x, x, x, torch.zeros(1, 64, 2))
    with pytest.raises(ValueError, match="gate"):  # the GLA scorer needs its gate
        pkg.LighthouseLocal(scorer=gla, num_levels=3, pooling_factor=4, topk=128, attention=None)(x, x, x)
    cp = pkg.LighthouseCP(attention=None, scorer=pkg.DialatedLighthouseNormScorerCP())
    cp.set_cp_info(0, 2, None)
    with pytest.raises(NotImplementedError):
        cp(None, None, None)
    assert pkg.compute_output_indices_selection(32768, 3, 4, 2048) == 18432
    assert pkg.LighthouseSelectionQkKqChunkedTopkNvrtc is pkg.LighthouseSelectionQkKqChunkedTopkHip


def test_selection_class_asserts_like_reference(pkg):
    s = torch.zeros(1, 1, 5376)
    with pytest.raises(AssertionError):  # not on a GPU
        pkg.LighthouseSelectionQkKqChunkedTopkNvrtc.forward(s, s, 3, 4, 256, 4096)
    with pytest.raises(AssertionError):
        pkg.LighthouseSelectionQkKqChunkedTopkNvrtc.forward(s, s[..., :10], 3, 4, 256, 4096)


def test_check_indices_host_validation(pkg):
    lib = pkg._native.lib()
    null = ctypes.c_void_p(0)
    assert lib.lh_check_indices(null, 1, 1, 8, 0, 10, null, null, null) == 1
    assert lib.lh_check_indices(ctypes.c_void_p(16), 1, 1, 8, 5, 5, null, ctypes.c_void_p(16), null) == 1


def test_row_kernels_refuse_non_bf16(pkg):
    """The kernels read and write bf16 rows: other dtypes raise TypeError on the
    host before any device work (CPU tensors suffice to reach the check)."""
    N = pkg._native
    x32 = torch.zeros(1, 2, 16, 128)
    idx = torch.zeros(1, 2, 16, dtype=torch.int32)
    with pytest.raises(TypeError):
        N.scatter_fwd(x32, idx, 16, 16, 2, 2)
    with pytest.raises(TypeError):
        N.scatter_bwd(x32, idx, None, 16, 2, 2)
    with pytest.raises(TypeError):
        N.Rows(x32, x32, x32, (0, 0, 0))
    with pytest.raises(TypeError):
        N.pyramid_bwd(x32, x32, x32, None, 1, 16, 2, 2, 2)
    with pytest.raises(TypeError):
        pkg.scatter_to_base_sequence(x32, idx, None, 16, 16, 2, 2)
    xb = torch.zeros(1, 2, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(TypeError):  # int64 indices where the kernels read int32
        N.attn_fwd(N.Rows(xb, xb, xb, (0, 0, 0)), idx.long(), 1, 2, 16)
    with pytest.raises(ValueError):  # head dimension not contiguous
        N.Rows(xb.transpose(-1, -2), xb, xb, (0, 0, 0))


def test_layer_refuses_float32_and_mixed_dtypes(pkg):
    """Float32 inputs are refused rather than silently downcast, and so are
    inputs of different dtypes, before any device work."""
    x = torch.zeros(1, 512, 2, 128)
    with pytest.raises(TypeError, match="bfloat16 or float16"):
        pkg.lighthouse_layer(x, x, x, num_levels=3, pooling_factor=4, topk=128)
    h = x.half()
    with pytest.raises(TypeError, match="share a dtype"):
        pkg.lighthouse_layer(h, h.bfloat16(), h, num_levels=3, pooling_factor=4, topk=128)
    with pytest.raises(TypeError, match="bfloat16 or float16"):
        pkg.lighthouse_layer(x, x, x, num_levels=3, pooling_factor=4, topk=128, dilation=4,
                             gk=torch.zeros(1, 512, 2))
