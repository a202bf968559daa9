"""Pins of the CPU oracle (runs without a GPU).

Each oracle function is checked against something other than itself:

geometry            the reference formula and the published size table; the
                    reference kernel's closed-form level offset
bitonic_sort128     sortedness + permutation on distinct keys, the 0-1 principle,
                    identity on all-equal keys, planted mistakes that must fail
select (structural) brute-force top-64(qk) + top-64(kq of the rest) per tile and
                    level on distinct scores; brute-force (score, lower index)
                    order in lower_index mode; the slot-literal C restatement
                    (oracle/select_ref.c) for both tie modes, strict and
                    generalized; a hand-built post-order on tiny trees
norm / dilated      per-token loops
sdpa_causal         torch's F.scaled_dot_product_attention and a naive loop; the
                    chunked form (long sequences) against the explicit form,
                    values and autograd gradients
scatter fwd / bwd   per-entry loops; the adjoint identity
layer backward      central finite differences in float64
golden fixtures     committed vectors (tests/golden/) for cfg1 and a tie-heavy case
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import lh_oracle as O
from oracle import select_ref as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

# Selected lengths of the benchmark geometries: (S, L, p, k) -> (S_sel by the reference formula,
# src/lighthouse_selection_cuda.py:346-357, S_sel generalized)
TABLE = {
    (4096, 3, 4, 1536): (12544, 5292),
    (32768, 3, 4, 2048): (18432, 18432),
    (65536, 3, 4, 1536): (16384, 16380),
    (65536, 3, 4, 3072): (28672, 28656),
    (65536, 3, 4, 6144): (53248, 44976),
    (131072, 5, 2, 1536): (20480, 20472),
    (32768, 3, 4, 1536): (14336, 14328),
}


# ----------------------------------------------------------------------------- geometry
@pytest.mark.parametrize("geo", sorted(TABLE))
def test_geometry_table(geo):
    S, L, p, k = geo
    ref, gen = TABLE[geo]
    assert O.compute_output_indices_selection(S, L, p, k) == ref
    g = O.tile_geometry(S, L, p, k)
    assert g.S_sel == gen
    assert g.strict_ok == (geo == (32768, 3, 4, 2048))
    if g.strict_ok:
        assert g.S_sel == ref


@pytest.mark.parametrize("S,L,p", [(4096, 3, 4), (32768, 3, 4), (65536, 3, 4), (131072, 5, 2), (2048, 2, 2),
                                   (98304, 3, 4), (98304, 5, 2), (98304, 3, 8)])
def test_level_offsets_closed_form(S, L, p):
    offs = O.level_offsets(S, L, p)
    for lvl in range(1, L + 1):
        assert offs[lvl - 1] == O.closed_form_offset(S, lvl, p)


def test_geometry_rejects_like_reference():
    with pytest.raises(AssertionError):
        O.tile_geometry(4096, 3, 4, 100)
    with pytest.raises(AssertionError):
        O.tile_geometry(4096, 3, 3, 256)
    with pytest.raises(AssertionError):
        O.select_indices(np.zeros((1, 1, 5376), np.float32), np.zeros((1, 1, 5376), np.float32), 3, 4, 1536, 4096)


# ----------------------------------------------------------------------------- network
def _rows(n, rng, kind):
    if kind == "distinct":
        return np.stack([rng.permutation(1000)[:128].astype(np.float32) for _ in range(n)])
    if kind == "01":
        return rng.integers(0, 2, (n, 128)).astype(np.float32)
    raise ValueError(kind)


@pytest.mark.parametrize("tie", ["reference", "lower_index"])
def test_bitonic_sorts_distinct(tie):
    rng = np.random.default_rng(0)
    s = _rows(200, rng, "distinct")
    ids = np.tile(np.arange(128), (200, 1))
    out_s, out_x = O.bitonic_sort128(s, ids, tie)
    assert np.array_equal(out_s, -np.sort(-s, axis=1))
    assert np.array_equal(np.take_along_axis(s, out_x, 1), out_s)


def test_bitonic_zero_one_principle():
    rng = np.random.default_rng(1)
    s = _rows(500, rng, "01")
    out_s, out_x = O.bitonic_sort128(s, np.tile(np.arange(128), (500, 1)))
    assert np.array_equal(out_s, -np.sort(-s, axis=1))
    assert all(sorted(r) == list(range(128)) for r in out_x)


def test_bitonic_all_equal_is_identity():
    s = np.full((3, 128), 2.5, np.float32)
    ids = np.tile(np.arange(128), (3, 1))
    _, out_x = O.bitonic_sort128(s, ids)
    assert np.array_equal(out_x, ids)


def test_planted_network_mistakes_are_caught():
    """Mutations of the network that the pins above must reject."""
    def sort_with(swap_rule):
        def f(scores, ids):
            s = scores.astype(np.float32).copy()
            x = ids.copy()
            for k, j in O._STAGES:
                lo = O._POS[(O._POS & j) == 0]
                hi = lo | j
                desc = (lo & k) == 0
                a, b = s[..., lo], s[..., hi]
                sw = swap_rule(a, b, desc)
                s[..., lo], s[..., hi] = np.where(sw, b, a), np.where(sw, a, b)
                xa, xb = x[..., lo], x[..., hi]
                x[..., lo], x[..., hi] = np.where(sw, xb, xa), np.where(sw, xa, xb)
            return s, x
        return f

    ids = np.tile(np.arange(128), (3, 1))
    equal = np.full((3, 128), 1.0, np.float32)
    # swapping on ties too ("<=") moves tied payloads
    le = sort_with(lambda a, b, d: np.where(d, a <= b, a >= b))
    assert not np.array_equal(le(equal, ids)[1], ids)
    # inverted direction rule no longer sorts descending
    rng = np.random.default_rng(2)
    s = _rows(20, rng, "distinct")
    inv = sort_with(lambda a, b, d: np.where(~d, a < b, a > b))
    assert not np.array_equal(inv(s, np.tile(np.arange(128), (20, 1)))[0], -np.sort(-s, 1))


# ----------------------------------------------------------------------------- selection
def _scores(B, H, S, L, p, rng, kind):
    S_tot = sum(O.level_lengths(S, L, p))
    if kind == "distinct":
        x = np.stack([rng.permutation(B * H * S_tot * 4)[:S_tot] for _ in range(B * H)]).astype(np.float32)
        return x.reshape(B, H, S_tot) / 7.0
    x = rng.standard_normal((B, H, S_tot)).astype(np.float32)
    if kind == "bf16":
        return torch.tensor(np.abs(x) * 4 + 8).bfloat16().float().numpy()
    if kind == "coarse":
        return np.floor(np.abs(x) * 2).clip(max=7).astype(np.float32)
    return x


@pytest.mark.parametrize("geo", [(2048, 3, 4, 128), (4096, 3, 4, 256), (8192, 4, 2, 256), (4096, 3, 4, 1536),
                                 (2048, 2, 2, 128)])
@pytest.mark.parametrize("tie", ["reference", "lower_index"])
def test_selection_bruteforce_per_tile(geo, tie):
    """On distinct scores (both modes) and on tie-heavy scores (lower_index), the selected set
    of every (tile, level) is top-64 by qk plus top-64 by kq among the remaining candidates."""
    S, L, p, k = geo
    rng = np.random.default_rng(sum(geo))
    kinds = ["distinct"] + (["coarse", "bf16"] if tie == "lower_index" else [])
    for kind in kinds:
        a = _scores(1, 2, S, L, p, rng, kind)
        b = _scores(1, 2, S, L, p, rng, kind)
        g, levels = O.select_tiles(a, b, L, p, k, S, tie)
        offs = O.level_offsets(S, L, p)
        for lvl in range(L, 1, -1):
            cand, sel = levels[lvl]
            for row in range(cand.shape[0]):
                bh = row // g.T
                c = [int(i) for i in cand[row] if i >= 0]
                key_q = lambda i: (-a.reshape(-1, a.shape[-1])[bh, offs[lvl - 1] + i], i)
                key_k = lambda i: (-b.reshape(-1, b.shape[-1])[bh, offs[lvl - 1] + i], i)
                top_q = sorted(c, key=key_q)[:64]
                rest = [i for i in c if i not in set(top_q)]
                top_k = sorted(rest, key=key_k)[:64]
                got = [int(i) for i in sel[row] if i >= 0]
                assert sorted(got) == sorted(top_q + top_k), (lvl, row, kind)
                # the [TQ | TK] halves are the two ranked lists, in order
                assert [int(i) for i in sel[row][:64] if i >= 0] == top_q
                assert [int(i) for i in sel[row][64:] if i >= 0] == top_k
            # children of this level's selected parents are the next level's candidates
            child, _ = levels[lvl - 1]
            for row in range(cand.shape[0]):
                want = sorted(int(s_) * p + j for s_ in sel[row] if s_ >= 0 for j in range(p))
                assert sorted(int(i) for i in child[row] if i >= 0) == want


def test_reference_ties_differ_from_lower_index():
    """The reference network does not break ties by lower index (bf16 scores), but both
    orders agree on distinct fp32 scores."""
    rng = np.random.default_rng(5)
    S, L, p, k = 4096, 3, 4, 256
    differ = 0
    for _ in range(5):
        a = _scores(1, 2, S, L, p, rng, "bf16")
        b = _scores(1, 2, S, L, p, rng, "bf16")
        differ += not np.array_equal(O.select_indices(a, b, L, p, k, S),
                                     O.select_indices(a, b, L, p, k, S, tie="lower_index"))
        a = _scores(1, 2, S, L, p, rng, "distinct")
        b = _scores(1, 2, S, L, p, rng, "distinct")
        assert np.array_equal(O.select_indices(a, b, L, p, k, S),
                              O.select_indices(a, b, L, p, k, S, tie="lower_index"))
    assert differ >= 4


@pytest.mark.parametrize("geo", [(2048, 3, 4, 128), (4096, 3, 4, 256), (2048, 2, 2, 128), (8192, 4, 2, 256),
                                 (32768, 3, 4, 2048), (4096, 3, 4, 1536), (65536, 3, 4, 1536),
                                 (65536, 3, 4, 6144), (131072, 5, 2, 1536), (5000, 3, 4, 256)])
@pytest.mark.parametrize("tie", ["reference", "lower_index"])
def test_structural_equals_slot_literal(geo, tie):
    """Every-candidate emission (numpy) == the reference's slot-by-slot emission + key sort (C)."""
    S, L, p, k = geo
    g = O.tile_geometry(S, L, p, k)
    rng = np.random.default_rng(S + k)
    for kind in ("bf16", "coarse", "fp32"):
        a = _scores(1, 2, S, L, p, rng, kind)
        b = _scores(1, 2, S, L, p, rng, kind)
        ref = O.select_indices(a, b, L, p, k, S, tie=tie, strict=False)
        assert np.array_equal(ref, R.select_indices_c(a, b, L, p, k, S, g.S_sel, tie=tie, strict=False))
        if g.strict_ok:
            assert np.array_equal(ref, R.select_indices_c(a, b, L, p, k, S, g.S_sel, tie=tie, strict=True))


def _postorder(levels, L, p, S):
    """Expected output of one tile built directly from the tree: for each coarsest
    node in order, if selected its children (recursively) then itself, else itself."""
    offs = O.level_offsets(S, L, p)
    selected = {lvl: set(int(i) for i in levels[lvl][1][0] if i >= 0) for lvl in range(2, L + 1)}

    def visit(lvl, i):
        if lvl >= 2 and i in selected[lvl]:
            out = []
            for c in range(i * p, i * p + p):
                out += visit(lvl - 1, c)
            return out + [offs[lvl - 1] + i]
        return [offs[lvl - 1] + i]

    return [r for i in levels[L][0][0] for r in visit(L, int(i))]


@pytest.mark.parametrize("geo", [(256, 2, 2, 128), (2048, 3, 4, 128), (1024, 4, 2, 128), (768, 2, 2, 128)])
def test_causal_order_is_post_order(geo):
    S, L, p, k = geo
    rng = np.random.default_rng(3)
    a = _scores(1, 1, S, L, p, rng, "bf16")
    b = _scores(1, 1, S, L, p, rng, "bf16")
    g, levels = O.select_tiles(a, b, L, p, k, S)
    got = O.select_indices(a, b, L, p, k, S, strict=False)[0, 0]
    assert list(got) == _postorder(levels, L, p, S)
    if (S, L, p) == (256, 2, 2):  # every node selected: children 2i, 2i+1, then node i
        assert list(got[:6]) == [0, 1, 256, 2, 3, 257]


def test_selection_output_invariants():
    rng = np.random.default_rng(9)
    S, L, p, k = 32768, 3, 4, 2048
    a = _scores(1, 2, S, L, p, rng, "bf16")
    b = _scores(1, 2, S, L, p, rng, "bf16")
    idx = O.select_indices(a, b, L, p, k, S)
    S_tot = a.shape[-1]
    offs = O.level_offsets(S, L, p)
    assert idx.shape == (1, 2, 18432)
    for row in idx.reshape(-1, idx.shape[-1]):
        assert len(set(row.tolist())) == len(row) and row.min() >= 0 and row.max() < S_tot
        # every coarsest node is present (NCC = 128: the coarsest level is fully selected)
        assert set(range(offs[2], S_tot)) <= set(row.tolist())


# ----------------------------------------------------------------------------- fp oracle
def test_norm_scorer_bruteforce():
    torch.manual_seed(0)
    b, s, h, d, p, L = 1, 37, 2, 4, 2, 3
    xs = [torch.randn(b, s, h, d, dtype=torch.float64) for _ in range(3)]
    sqk, skq, qc, kc, vc = O.norm_scorer(*xs, p, L)
    offs = O.level_offsets(s, L, p)
    lens = O.level_lengths(s, L, p)
    for hh in range(h):
        for lvl in range(1, L + 1):
            c = p ** (lvl - 1)
            for i in range(lens[lvl - 1]):
                span = range(i * c, i * c + c)
                r = offs[lvl - 1] + i
                for x, cat in zip(xs, (qc, kc, vc)):
                    m = sum(x[0, t, hh] for t in span) / c
                    assert torch.allclose(cat[0, hh, r], m)
                nq = max(float(torch.sqrt((xs[0][0, t, hh] ** 2).sum())) for t in span)
                nk = max(float(torch.sqrt((xs[1][0, t, hh] ** 2).sum())) for t in span)
                assert abs(float(sqk[0, hh, r]) - nq) < 1e-12 and abs(float(skq[0, hh, r]) - nk) < 1e-12


def test_sdpa_causal_vs_library_and_loop():
    torch.manual_seed(1)
    q, k, v = (torch.randn(2, 3, 17, 8, dtype=torch.float64) for _ in range(3))
    out = O.sdpa_causal(q, k, v)
    lib = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.allclose(out, lib, atol=1e-12)
    i = 11
    w = torch.softmax((q[0, 1, i] @ k[0, 1, :i + 1].T) / 8 ** 0.5, -1)
    assert torch.allclose(out[0, 1, i], w @ v[0, 1, :i + 1], atol=1e-12)


@pytest.mark.parametrize("chunk", [1, 5, 16])
def test_sdpa_chunked_matches_explicit(chunk):
    torch.manual_seed(5)
    q, k, v = (torch.randn(2, 3, 17, 8, dtype=torch.float64, requires_grad=True) for _ in range(3))
    ref = O.sdpa_causal(q, k, v, chunk=17)   # explicit form, torch autograd
    w = torch.randn_like(ref)
    gref = torch.autograd.grad((ref * w).sum(), (q, k, v))
    out = O.sdpa_causal(q, k, v, chunk=chunk)
    assert torch.allclose(out, ref, atol=1e-12)
    got = torch.autograd.grad((out * w).sum(), (q, k, v))
    for a, r in zip(got, gref):
        assert torch.allclose(a, r, atol=1e-12)


def test_dilated_scorer_bruteforce():
    torch.manual_seed(2)
    b, s, h, d, dil = 1, 16, 2, 4, 4
    xs = [torch.randn(b, s, h, d, dtype=torch.float64) for _ in range(3)]
    sqk, skq, *_ = O.dilated_scorer(*xs, dilation=dil, pooling_factor=2, levels=2)
    xq, xk, xv = xs
    for t in range(s):
        for hh in range(h):
            ph = t % dil  # phase: tokens t' = t mod dil share a virtual head
            ts = [u for u in range(s) if u % dil == ph and u <= t]
            for src, dst, score in ((xq, xk, sqk), (xk, xq, skq)):
                logits = torch.stack([(src[0, t, hh] * dst[0, u, hh]).sum() for u in ts]) / d ** 0.5
                o = (torch.softmax(logits, 0)[:, None] * torch.stack([xv[0, u, hh] for u in ts])).sum(0)
                assert abs(float(score[0, hh, t]) - float(o.norm())) < 1e-10


def _idx_small(S, L, p, k, H, seed):
    rng = np.random.default_rng(seed)
    a = _scores(1, H, S, L, p, rng, "bf16")
    b = _scores(1, H, S, L, p, rng, "bf16")
    return O.select_indices(a, b, L, p, k, S, strict=False)


def test_scatter_bruteforce_and_adjoint():
    S, L, p, k = 2048, 3, 4, 128
    idx = _idx_small(S, L, p, k, 1, 4)
    n = idx.shape[-1]
    torch.manual_seed(3)
    attn = torch.randn(1, 1, n, 4, dtype=torch.float64)
    out = O.scatter_fwd(attn, torch.from_numpy(idx), S, L, p)
    offs = O.level_offsets(S, L, p)
    lens = O.level_lengths(S, L, p)
    ref = torch.zeros(1, 1, S, 4, dtype=torch.float64)
    for s_, r in enumerate(idx[0, 0]):
        lvl = max(l for l in range(1, L + 1) if r >= offs[l - 1])
        c, i = p ** (lvl - 1), int(r) - offs[lvl - 1]
        assert i < lens[lvl - 1]
        for t in range((i + 1) * c - 1, (i + 2) * c - 1):
            if t < S:
                ref[0, 0, t] += attn[0, 0, s_]
    assert torch.allclose(out, ref)
    y = torch.randn(1, 1, S, 4, dtype=torch.float64)
    lhs = (O.scatter_fwd(attn, torch.from_numpy(idx), S, L, p) * y).sum()
    rhs = (attn * O.scatter_bwd(y, torch.from_numpy(idx), S, L, p)).sum()
    assert torch.allclose(lhs, rhs)


def test_layer_backward_finite_differences():
    torch.manual_seed(4)
    S, L, p, k, H, d = 256, 2, 2, 128, 1, 4
    xs = [torch.randn(1, S, H, d, dtype=torch.float64) for _ in range(3)]
    _, idx = O.lighthouse_layer(*[x.float() for x in xs], L, p, k, indices=None, strict=False)
    xr = [x.clone().requires_grad_() for x in xs]
    w = torch.randn(1, H, S, d, dtype=torch.float64)
    out, _ = O.lighthouse_layer(*xr, L, p, k, indices=idx)
    (out * w).sum().backward()
    eps = 1e-6
    rng = np.random.default_rng(0)
    for which in range(3):
        for _ in range(6):
            t, e = int(rng.integers(S)), int(rng.integers(d))
            xp = [x.clone() for x in xs]
            xm = [x.clone() for x in xs]
            xp[which][0, t, 0, e] += eps
            xm[which][0, t, 0, e] -= eps
            fp = (O.lighthouse_layer(*xp, L, p, k, indices=idx)[0] * w).sum()
            fm = (O.lighthouse_layer(*xm, L, p, k, indices=idx)[0] * w).sum()
            num = float((fp - fm) / (2 * eps))
            assert abs(num - float(xr[which].grad[0, t, 0, e])) < 1e-6 * max(1.0, abs(num))


# ----------------------------------------------------------------------------- golden fixtures
def _load_golden(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.skip(f"{name} missing")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", ["cfg1_selection.npz", "ties_4096_k256.npz"])
def test_golden_selection(name):
    g = _load_golden(name)
    meta = json.load(open(os.path.join(GOLDEN, "manifest.json")))[name]
    S, L, p, k = meta["S"], meta["L"], meta["p"], meta["topk"]
    for tie in ("reference", "lower_index"):
        got = O.select_indices(g["scores_qk"], g["scores_kq"], L, p, k, S, tie=tie, strict=meta["strict"])
        assert np.array_equal(got, g[f"indices_{tie}"])
        assert hashlib.sha256(got.tobytes()).hexdigest() == meta[f"sha256_{tie}"]


# ----------------------------------------------------------------------------- sanitizer build
SAN_GEOS = [  # (S, L, p, k, strict)
    (2048, 3, 4, 128, True),
    (8192, 4, 2, 256, True),
    (4096, 3, 4, 1536, False),   # cfg1 geometry (NCC < 128)
    (5000, 3, 4, 256, False),    # S not a multiple of p^(L-1)
    (16384, 5, 2, 256, False),
]


@pytest.fixture(scope="module")
def asan_driver():
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    subprocess.run(["make", "-s", "-C", os.path.join(O.__file__.rsplit(os.sep, 1)[0]), "asan"], check=True)
    path = os.path.join(os.path.dirname(O.__file__), "_build", "select_ref_asan")
    libs = subprocess.run(["ldd", path], capture_output=True, text=True).stdout
    assert "libasan" in libs and "libubsan" in libs, "driver is not built with the sanitizers"
    return path


@pytest.mark.parametrize("tie", ["reference", "lower_index"])
@pytest.mark.parametrize("geo", SAN_GEOS)
def test_select_ref_under_sanitizers(asan_driver, tmp_path, geo, tie):
    """oracle/select_ref.c run under AddressSanitizer + UBSan (any out-of-bounds
    slot write, overflow or invalid shift aborts the driver), on strict and
    generalized geometries with tie-heavy scores; the result equals the
    regular build's."""
    import subprocess
    S, L, p, k, strict = geo
    H = 2
    S_tot = sum(O.level_lengths(S, L, p))
    g = torch.Generator().manual_seed(S + L)
    a = ((torch.randn(1, H, S_tot, generator=g).abs() * 4 + 8).bfloat16().float()).numpy()
    b = ((torch.randn(1, H, S_tot, generator=g).abs() * 4 + 8).bfloat16().float()).numpy()
    n = O.tile_geometry(S, L, p, k).S_sel
    expect = R.select_indices_c(a, b, L, p, k, S, n, tie=tie, strict=strict)
    fa, fb, fo = tmp_path / "qk.f32", tmp_path / "kq.f32", tmp_path / "out.i32"
    a.astype(np.float32).tofile(fa)
    b.astype(np.float32).tofile(fb)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([asan_driver, str(H), str(S_tot), str(S), str(L), str(p), str(k),
                        str(int(tie == "lower_index")), "0" if strict else "1", str(n), str(fa), str(fb), str(fo)],
                       capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, f"sanitized driver failed ({r.returncode}): {r.stderr[-2000:]}"
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-2000:]
    got = np.fromfile(fo, dtype=np.int32).reshape(1, H, n)
    assert np.array_equal(got, expect)


# ----------------------------------------------------------------------------- GLA scorer
@pytest.mark.parametrize("seed,gscale", [(0, 1.0), (1, 0.05), (2, 8.0)])
def test_simple_gla_matches_recurrence(seed, gscale):
    """Quadratic form == token-by-token recurrence h_t = e^{g_t} h_{t-1} + k_t^T v_t."""
    g0 = torch.Generator().manual_seed(seed)
    B, T, H, D = 2, 13, 3, 5
    q, k, v = (torch.randn(B, T, H, D, generator=g0) for _ in range(3))
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=g0) * gscale)
    a = O.simple_gla(q, k, v, g, 0.37)
    r = O.simple_gla_recurrent(q, k, v, g, 0.37)
    assert torch.allclose(a, r, rtol=1e-10, atol=1e-12)


def test_simple_gla_limits():
    """g = 0: causal linear attention, o_t = scale q_t sum_{s<=t} k_s^T v_s (prefix sum
    of outer products); g -> -inf: only the diagonal survives, o_t = scale (q_t.k_t) v_t."""
    g0 = torch.Generator().manual_seed(5)
    B, T, H, D = 1, 17, 2, 6
    q, k, v = (torch.randn(B, T, H, D, generator=g0, dtype=torch.float64) for _ in range(3))
    kv = torch.cumsum(k[..., :, None] * v[..., None, :], dim=1)          # [B, T, H, D, D]
    want = 0.5 * torch.einsum("bthi,bthij->bthj", q, kv)
    assert torch.allclose(O.simple_gla(q, k, v, torch.zeros(B, T, H), 0.5), want, rtol=1e-10, atol=1e-10)
    diag = 0.5 * (q * k).sum(-1, keepdim=True) * v
    assert torch.allclose(O.simple_gla(q, k, v, torch.full((B, T, H), -1e4), 0.5), diag, rtol=1e-10, atol=1e-10)


def test_gla_scorer_virtual_heads():
    """Base scores: token t of head h belongs to the sequence x[:, t % dil :: dil, h]
    (virtual head (t % dil) * H + h), built here by slicing, not by the reshape."""
    g0 = torch.Generator().manual_seed(7)
    B, S, H, D, dil = 2, 48, 3, 8, 4
    xq, xk, xv = (torch.randn(B, S, H, D, generator=g0) for _ in range(3))
    gk = torch.nn.functional.logsigmoid(torch.randn(B, S, H, generator=g0)) / 16
    sqk, skq, *_ = O.gla_scorer(xq, xk, xv, gk, dil, 2, 3)
    for r in range(dil):
        for h in range(H):
            sl = lambda x: x[:, r::dil, h:h + 1]  # noqa: E731
            oq = O.simple_gla_recurrent(sl(xq), sl(xk), sl(xv), sl(gk), D ** -0.5)
            ok = O.simple_gla_recurrent(sl(xk), sl(xq), sl(xv), sl(gk), D ** -0.5)
            assert torch.allclose(sqk[:, h, r:S:dil], oq.norm(dim=-1)[..., 0].float(), rtol=1e-5, atol=1e-6)
            assert torch.allclose(skq[:, h, r:S:dil], ok.norm(dim=-1)[..., 0].float(), rtol=1e-5, atol=1e-6)
    # pooled levels: max of the base scores over each span, as the norm scorer's
    assert torch.equal(sqk[:, :, S:S + S // 2], sqk[:, :, :S].reshape(B, H, S // 2, 2).amax(-1))


# ----------------------------------------------------------------------------- property tests
try:
    from hypothesis import given, settings, strategies as st
    HAVE_HYPOTHESIS = True
except Exception:  # pragma: no cover
    HAVE_HYPOTHESIS = False


def _check_selection_properties(a, b, S, L, p, k, tie):
    """Invariants every selection must satisfy, whatever the scores: the structural
    and slot-literal restatements agree, and per (b, h) the indices are unique and
    in range, and every entry below the coarsest level has its parent selected at
    the next level."""
    g = O.tile_geometry(S, L, p, k)
    idx = O.select_indices(a, b, L, p, k, S, tie=tie, strict=False)
    ref = R.select_indices_c(a, b, L, p, k, S, g.S_sel, tie=tie, strict=False)
    assert np.array_equal(idx, ref)
    offs = O.level_offsets(S, L, p)
    lens = O.level_lengths(S, L, p)
    S_tot = sum(lens)
    for row in idx.reshape(-1, idx.shape[-1]):
        assert len(set(row.tolist())) == len(row) and row.min() >= 0 and row.max() < S_tot
        lvl = np.searchsorted(np.asarray(offs), row, side="right")  # 1-based level of each entry
        loc = row - np.asarray(offs)[lvl - 1]
        present = set(row.tolist())
        for lv, i in zip(lvl.tolist(), loc.tolist()):
            if lv < L:
                parent = offs[lv] + i // p
                if i // p < lens[lv]:
                    assert parent in present, "an entry whose parent was not selected"


if HAVE_HYPOTHESIS:
    @settings(max_examples=40, deadline=None)
    @given(L=st.integers(2, 4), p=st.sampled_from([2, 4]), kk=st.sampled_from([128, 256]),
           mult=st.integers(1, 6), extra=st.integers(0, 37), kind=st.sampled_from(["bf16", "fp32", "coarse"]),
           tie=st.sampled_from(["reference", "lower_index"]), seed=st.integers(0, 2 ** 31 - 1))
    def test_selection_properties_random_geometries(L, p, kk, mult, extra, kind, tie, seed):
        S = kk * p ** (L - 1) * mult + extra  # ragged lengths, at least one tile
        rng = np.random.default_rng(seed)
        a = _scores(1, 2, S, L, p, rng, kind)
        b = _scores(1, 2, S, L, p, rng, kind)
        _check_selection_properties(a, b, S, L, p, kk, tie)
