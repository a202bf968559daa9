"""GPU parity of the top-k selection kernel against the oracle (bit-exact).

The reference kernel is src/lighthouse_selection_cuda.py:114-331 (+ :425-427
for the ordering); the oracle restates it twice (numpy structural form and the
slot-literal C form, both checked against each other in test_oracle.py).
"""
import numpy as np
import pytest
import torch

from oracle import lh_oracle as O
from oracle import select_ref as R

pytestmark = pytest.mark.gpu

STRICT = [  # (S, L, p, topk)
    (2048, 3, 4, 128),
    (4096, 3, 4, 256),
    (8192, 4, 2, 256),
    (2048, 2, 2, 128),
    (32768, 3, 4, 2048),  # north-star geometry
]
GENERALIZED = [
    (4096, 3, 4, 1536),    # cfg1 (NCC = 21 < 128)
    (65536, 3, 4, 1536),   # cfg3 k=1536 (NCC = 341)
    (65536, 3, 4, 3072),   # cfg3 k=3072
    (65536, 3, 4, 6144),   # cfg3 k=6144 (NCC = 85)
    (32768, 3, 4, 1536),   # cfg5 layer geometry
    (131072, 5, 2, 1536),  # cfg4 geometry
    (5000, 3, 4, 256),     # S not a multiple of p^(L-1)
]


def _scores(S, L, p, H, kind, seed):
    g = torch.Generator().manual_seed(seed)
    S_tot = sum(O.level_lengths(S, L, p))
    x = torch.randn(1, H, S_tot, generator=g)
    if kind == "bf16":   # heavy ties: a few hundred distinct values
        x = (x.abs() * 4 + 8).bfloat16().float()
    elif kind == "coarse":  # very heavy ties: 8 distinct values
        x = torch.floor(x.abs() * 2).clamp(max=7)
    return x.numpy().astype(np.float32)


def _run(pkg, dev, a, b, S, L, p, k, tie, strict):
    sqk = torch.from_numpy(a).to(dev)
    skq = torch.from_numpy(b).to(dev)
    idx, inv = pkg._native.select_topk(sqk, skq, S, L, p, k, tie=tie, strict=strict)
    torch.cuda.synchronize()
    return idx.cpu().numpy(), inv.cpu().numpy()


@pytest.mark.parametrize("tie", ["reference", "lower_index"])
@pytest.mark.parametrize("kind", ["bf16", "fp32", "coarse"])
@pytest.mark.parametrize("geo", STRICT)
def test_select_strict_bit_exact(pkg, dev, geo, kind, tie):
    S, L, p, k = geo
    H = 2
    a = _scores(S, L, p, H, kind, 1)
    b = _scores(S, L, p, H, kind, 2)
    print(f"select strict S={S} L={L} p={p} k={k} kind={kind} tie={tie}", flush=True)
    g = O.tile_geometry(S, L, p, k)
    ref = R.select_indices_c(a, b, L, p, k, S, g.S_sel, tie=tie, strict=True)
    got, inv = _run(pkg, dev, a, b, S, L, p, k, tie, True)
    assert got.shape == ref.shape
    assert np.array_equal(got, ref), f"{(got != ref).sum()} of {ref.size} indices differ"
    assert np.array_equal(inv, O.inverse_map(ref, a.shape[-1]))


@pytest.mark.parametrize("tie", ["reference", "lower_index"])
@pytest.mark.parametrize("geo", GENERALIZED)
def test_select_generalized_bit_exact(pkg, dev, geo, tie):
    S, L, p, k = geo
    H = 2
    a = _scores(S, L, p, H, "bf16", 3)
    b = _scores(S, L, p, H, "bf16", 4)
    print(f"select generalized S={S} L={L} p={p} k={k} tie={tie}", flush=True)
    g = O.tile_geometry(S, L, p, k)
    ref = R.select_indices_c(a, b, L, p, k, S, g.S_sel, tie=tie, strict=False)
    got, inv = _run(pkg, dev, a, b, S, L, p, k, tie, False)
    assert np.array_equal(got, ref), f"{(got != ref).sum()} of {ref.size} indices differ"
    assert np.array_equal(inv, O.inverse_map(ref, a.shape[-1]))


def test_select_north_star_on_real_norms(pkg, dev):
    """cfg2 shape (H=8) with scores from the native norm scorer on N(0,1) bf16 data."""
    torch.manual_seed(0)
    S, L, p, k, H = 32768, 3, 4, 2048, 8
    xs = [torch.randn(1, S, H, 128, device=dev).bfloat16() for _ in range(3)]
    _, _, _, sqk, skq = pkg._native.pyramid_fwd(*xs, L, p)
    idx, inv = pkg._native.select_topk(sqk, skq, S, L, p, k)
    a, b = sqk.cpu().numpy(), skq.cpu().numpy()
    ref = R.select_indices_c(a, b, L, p, k, S, 18432, strict=True)
    assert np.array_equal(idx.cpu().numpy(), ref)
    assert np.array_equal(inv.cpu().numpy(), O.inverse_map(ref, a.shape[-1]))
    # the default (reference) tie mode differs from lower-index on these tie-heavy scores
    alt = R.select_indices_c(a, b, L, p, k, S, 18432, tie="lower_index", strict=True)
    assert not np.array_equal(ref, alt)


def test_select_strict_rejects_out_of_domain(pkg, dev):
    a = _scores(4096, 3, 4, 1, "fp32", 0)
    with pytest.raises(AssertionError):
        _run(pkg, dev, a, a, 4096, 3, 4, 1536, "reference", True)


def test_api_selection_class(pkg, dev):
    S, L, p, k = 4096, 3, 4, 256
    a = _scores(S, L, p, 3, "bf16", 5)
    b = _scores(S, L, p, 3, "bf16", 6)
    out = pkg.LighthouseSelectionQkKqChunkedTopkNvrtc.forward(
        torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), L, p, k, S)
    ref = R.select_indices_c(a, b, L, p, k, S, pkg.compute_output_indices_selection(S, L, p, k))
    assert out.dtype == torch.int32
    assert np.array_equal(out.cpu().numpy(), ref)
