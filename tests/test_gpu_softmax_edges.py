"""Online-softmax edge cases of the attention kernels.

The forward keeps a running row maximum m and rescales its accumulators only
when a tile's maximum passes m by more than 8 (log2 units); the backward
kernels recompute P = exp2(S scale log2 e - lse) from the forward's lse.
These cases drive that logic away from the N(0, 1) inputs of the other tests:
  rising   - scores grow along the key axis (about 70 log2 units from the
             first key to the last), so most tiles raise m;
  falling  - scores shrink along the key axis, so later tiles' probabilities
             are tiny or underflow against the first tile's maximum;
  large    - inputs x16 (scores of +-2000 log2 units): everything but the keys
             near each row's maximum underflows, nothing may overflow.
Dense rows (identity map), ragged n.

O and lse are checked against fp32 SDPA (the oracle's sdpa_causal).  The
gradients take P (dV) and dS (dQ, dK) in bf16, as flash-style bf16 backward
passes do, and with a 64-sized key component shared by most keys (rising,
falling) sum_t dS[i, t] = 0 cancels in fp32 but not after the rounding of each
dS; and delta = rowsum(dO o O) is formed from the bf16 O, so it is off by up
to a bf16 half-ulp of rowsum(|dO| |O|), which matters where dP - delta nearly
cancels (the one-hot rows of the large case).  The standard max-abs bound does not hold
there.  Each gradient element must instead lie within four bf16 half-ulps of
the terms that make it,
    |dQ - dQ_ref| <= 4 * 2^-9 * scale * (e |K|),  e = |dS| + P (|dP| + rowsum(|dO| |O|))
(dK alike with e^T |Q|; dV: 4 * 2^-9 * P^T |dO|), plus 1e-3 of the largest
reference value, with rel-L2 <= 3e-2 overall; an error in the rescaling would
break this by orders of magnitude.
"""
import pytest
import torch

from conftest import assert_close
from oracle import lh_oracle as O

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _inputs(kind, n, H, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, n, H, 128, generator=g) for _ in range(3))
    t = torch.arange(n, dtype=torch.float32)[None, :, None] / n
    if kind == "rising":
        q[..., 0] = 8.0
        k[..., 0] = 64.0 * t
    elif kind == "falling":
        q[..., 0] = 8.0
        k[..., 0] = 64.0 * (1.0 - t)
    elif kind == "large":
        q, k = 16.0 * q, 16.0 * k
    return [x.bfloat16() for x in (q, k, v)]


def _error_bounds(q, k, v, do, delta, o):
    """Per-element bounds for dQ, dK, dV: four bf16 half-ulps (2^-9 relative)
    of the magnitudes of the terms summed into each element ([B, H, n, D]),
    with the dS terms widened by P (|dP| + rowsum(|dO| |O|))."""
    n = q.shape[2]
    s = (q @ k.transpose(-1, -2)) * SCALE
    s = s.masked_fill(torch.ones(n, n, dtype=torch.bool).triu(1), float("-inf"))
    p = torch.softmax(s, -1)
    dp = do @ v.transpose(-1, -2)
    e = (p * (dp - delta[..., None])).abs() + p * (dp.abs() + (do.abs() * o.abs()).sum(-1)[..., None])
    u = 4 * 2.0 ** -9
    return (u * SCALE * e @ k.abs(), u * SCALE * e.transpose(-1, -2) @ q.abs(),
            u * p.transpose(-1, -2) @ do.abs())


@pytest.mark.parametrize("kind,n", [("rising", 1500), ("falling", 1500), ("large", 1100)])
def test_softmax_edges(pkg, dev, kind, n):
    H = 2
    print(f"softmax edges {kind} n={n}", flush=True)
    N = pkg._native
    cpu = _inputs(kind, n, H, 7)
    gpu = [c.to(dev) for c in cpu]
    x = gpu[0]
    rows = N.Rows(*gpu, (x.stride(0), x.stride(1), x.stride(2)))
    o, lse = N.attn_fwd(rows, None, 1, H, n)
    q, k, v = [c.float().transpose(1, 2).clone().requires_grad_() for c in cpu]
    ref = O.sdpa_causal(q, k, v)
    assert_close(o, ref, f"{kind} out")
    # lse in log2 units against the fp32 log-sum-exp of the scaled scores
    s = (q.detach() @ k.detach().transpose(-1, -2)) * SCALE
    s = s.masked_fill(torch.ones(n, n, dtype=torch.bool).triu(1), float("-inf"))
    ref_lse = torch.logsumexp(s, -1) / torch.log(torch.tensor(2.0))
    assert torch.isfinite(lse).all(), f"{kind} lse: non-finite values"
    err = (lse.cpu() - ref_lse).abs().max().item()
    assert err <= 1e-2 * max(1.0, ref_lse.abs().max().item()), f"{kind} lse: max-abs {err:.3e}"

    g = torch.Generator().manual_seed(8)
    do = torch.randn(1, H, n, 128, generator=g).bfloat16()
    ref.backward(do.float())
    delta = (do.float() * o.float().cpu()).sum(-1)
    dq, dk, dv = N.attn_bwd(rows, None, 1, H, n, do.to(dev), lse, delta.to(dev))
    bounds = _error_bounds(q.detach(), k.detach(), v.detach(), do.float(), delta, ref.detach())
    for name, got, r, b in zip(("dq", "dk", "dv"), (dq, dk, dv), (q.grad, k.grad, v.grad), bounds):
        got = got.float().cpu()
        assert torch.isfinite(got).all(), f"{kind} {name}: non-finite values"
        excess = ((got - r).abs() - b - 1e-3 * r.abs().max()).max().item()
        assert excess <= 0, f"{kind} {name}: beyond the rounding bound by {excess:.3e}"
        assert_close(got, r, f"{kind} {name}", max_abs=float("inf"), rel_l2=3e-2)
