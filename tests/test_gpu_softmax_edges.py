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
passes do.  With a large key component shared by the keys, sum_t dS[i, t] = 0
cancels in fp32 but not after the rounding of each dS, and delta =
rowsum(dO o O), formed from the bf16 O, errs along the same direction; the dQ
kernel subtracts r_i c (r_i the row sum of the bf16 dS, c a mean of the block's
keys) where the keys' mean is large against their spread (key_centres), so its
rounding errors multiply k_t - c instead of k_t.  That makes a component
constant over the keys exact:
  shared   - four channels of every key set to 32 (trained models' keys often
             have such channels): every output and gradient within the
             standard tolerance, at n = 1500 and through the whole layer at
             the cfg2 size.
In the rising and falling cases the shared component is a ramp, so no single
c removes it, and in the large case delta's rounding matters where dP - delta
nearly cancels (its one-hot rows).  Each gradient element must lie within four
bf16 half-ulps of the terms that make it,
    |dQ - dQ_ref| <= 4 * 2^-9 * scale * (e |K|),  e = |dS| + P (|dP| + rowsum(|dO| |O|))
(dK alike with e^T |Q|; dV: 4 * 2^-9 * P^T |dO|), plus 1e-3 of the largest
reference value; an error in the rescaling would break this by orders of
magnitude.  On top of that every output and gradient meets the standard
tolerance, except dQ of the falling ramp, whose max-abs may reach 1.25 times
the standard bound (measured 1.14 times; rel-L2 5.2e-3, within the standard
1e-2).
"""
import pytest
import torch

from conftest import assert_close
from oracle import lh_oracle as O

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _inputs(kind, n, H, seed, dt=torch.bfloat16):
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
    elif kind == "shared":
        k[..., :4] = 32.0
    return [x.to(dt) for x in (q, k, v)]


BLOCK_Q = 256  # queries per block of the dQ kernel


def key_centres(k):
    """The dQ kernel's centre for each query ([B, H, n, D]): the fp32 mean c of
    the 64 keys (s kend) / 64, s < 64, of the query's block, kend the block's
    causal key range (identity row map), where the block centres, i.e. where
    |c|^2 > E|k - c|^2 / 16 over those keys; zero elsewhere."""
    n = k.shape[2]
    c = torch.zeros_like(k)
    for q0 in range(0, n, BLOCK_Q):
        kend = min(q0 + BLOCK_Q, n)
        pos = (torch.arange(64) * kend) // 64
        ks = k[:, :, pos]
        cm = ks.mean(2, keepdim=True)
        cc = (cm * cm).sum(-1, keepdim=True)
        kk = (ks * ks).sum(-1).mean(-1)[..., None, None]
        c[:, :, q0:kend] = torch.where(17 * cc > kk, cm, torch.zeros_like(cm))
    return c


def _error_bounds(q, k, v, do, delta, o):
    """Per-element bounds for dQ, dK, dV: four bf16 half-ulps (2^-9 relative)
    of the magnitudes of the terms summed into each element ([B, H, n, D]),
    with the dS terms widened by P (|dP| + rowsum(|dO| |O|)).  The dQ kernel's
    rounding errors (of dS and of delta) multiply k_t - c_i, c_i its block's
    key centre, so its terms are taken with |K - c_i|."""
    n = q.shape[2]
    s = (q @ k.transpose(-1, -2)) * SCALE
    s = s.masked_fill(torch.ones(n, n, dtype=torch.bool).triu(1), float("-inf"))
    p = torch.softmax(s, -1)
    dp = do @ v.transpose(-1, -2)
    e = (p * (dp - delta[..., None])).abs() + p * (dp.abs() + (do.abs() * o.abs()).sum(-1)[..., None])
    u = 4 * 2.0 ** -9
    c = key_centres(k)
    bq = torch.empty_like(q)
    for q0 in range(0, n, BLOCK_Q):
        q1 = min(q0 + BLOCK_Q, n)
        bq[:, :, q0:q1] = e[:, :, q0:q1] @ (k - c[:, :, q0:q0 + 1]).abs()
    return (u * SCALE * bq, u * SCALE * e.transpose(-1, -2) @ q.abs(),
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
        wide = kind == "falling" and name == "dq"
        assert_close(got, r, f"{kind} {name}", max_abs=2.5e-2 if wide else 2e-2)


def _dense_case(pkg, dev, kind, n, H, dt=torch.bfloat16):
    """Device O, dq, dk, dv and the fp32 oracle's (O and grads), rows of type dt."""
    N = pkg._native
    cpu = _inputs(kind, n, H, 7, dt)
    gpu = [c.to(dev) for c in cpu]
    x = gpu[0]
    rows = N.Rows(*gpu, (x.stride(0), x.stride(1), x.stride(2)))
    o, lse = N.attn_fwd(rows, None, 1, H, n)
    q, k, v = [c.float().transpose(1, 2).clone().requires_grad_() for c in cpu]
    ref = O.sdpa_causal(q, k, v)
    g = torch.Generator().manual_seed(8)
    do = torch.randn(1, H, n, 128, generator=g).to(dt)
    ref.backward(do.float())
    delta = (do.float() * o.float().cpu()).sum(-1)  # from the rounded O, as the layer forms it
    dq, dk, dv = N.attn_bwd(rows, None, 1, H, n, do.to(dev), lse, delta.to(dev))
    return (o, dq, dk, dv), (ref, q.grad, k.grad, v.grad)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_shared_key_channels(pkg, dev, dt):
    """Four key channels constant (32) over all keys: standard tolerance for O and
    every gradient (without the key centring, dQ misses it in bf16: max-abs 2.1x
    the bound, rel-L2 1.5e-2 in a CPU emulation of the kernel's roundings); fp16
    rows take the same centring path."""
    n, H = 1500, 2
    print(f"softmax edges shared n={n} {dt}", flush=True)
    got, ref = _dense_case(pkg, dev, "shared", n, H, dt)
    assert all(a.dtype == dt for a in got)
    for name, a, r in zip(("out", "dq", "dk", "dv"), got, ref):
        assert_close(a, r, f"shared {name}")


def test_shared_key_channels_layer_cfg2(pkg, dev):
    """The whole layer at the cfg2 size (S = 32768, k = 2048, L = 3, p = 4) with
    four channels of every key row set to 32: output and dq, dk, dv within the
    standard tolerance against the fp32 oracle on the device's index set (two
    heads, so the CPU oracle stays within seconds)."""
    B, S, H, L, p, k = 1, 32768, 2, 3, 4, 2048
    print(f"shared key channels layer S={S} H={H} k={k}", flush=True)
    g = torch.Generator().manual_seed(3)
    xs = [torch.randn(B, S, H, 128, generator=g) for _ in range(3)]
    xs[1][..., :4] = 32.0
    xs = [x.bfloat16() for x in xs]
    dout = torch.randn(B, H, S, 128, generator=g).bfloat16()
    xg = [x.to(dev).requires_grad_() for x in xs]
    out, idx = pkg.lighthouse_layer(*xg, num_levels=L, pooling_factor=p, topk=k)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    xc = [x.float().requires_grad_() for x in xs]
    ref_out, _ = O.lighthouse_layer(*xc, L, p, k, indices=idx.cpu().numpy())
    ref_out.backward(dout.float())
    assert_close(out, ref_out, "shared layer out")
    for name, a, c in zip("qkv", xg, xc):
        assert_close(a.grad, c.grad, f"shared layer d{name}")
