"""Query-block plans of the query-stationary attention kernels.

With B*H a multiple of 8 and between 1 and 3.5 query blocks per CU of a (b, h),
the forward and dQ kernels run one workgroup per CU, each taking a host-packed
list of query blocks (lh_attn.hip, make_plan / plan_slot) instead of one block
per workgroup.  Per-block arithmetic is unchanged, so results must be bit-equal
to the same heads run one at a time (B*H = 1: no plan).  The oracle checks of
these kernels at full size (test_gpu_configs.py) run with plans where these
conditions hold (cfg2, cfg3 at k = 1536 and 3072, cfg4's selected attention).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rand(shape, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).bfloat16().to(dev)


def _per_head(pkg, xs, pxs, idx, split, B, H, n, do, lse_all, delta_all):
    """O, lse, dq, dk, dv of every (b, h) computed alone (B = H = 1: no plan)."""
    N = pkg._native
    outs = {k: [] for k in ("o", "lse", "dq", "dk", "dv")}
    for b in range(B):
        for h in range(H):
            sl = [x[b:b + 1, :, h:h + 1] for x in xs]
            if pxs is None:
                rows = N.Rows(*sl, (sl[0].stride(0), sl[0].stride(1), sl[0].stride(2)))
                ix = None
            else:
                psl = [x[b:b + 1, :, h:h + 1] for x in pxs]
                rows = N.Rows(*sl, (sl[0].stride(0), sl[0].stride(1), sl[0].stride(2)), *psl,
                              (psl[0].stride(0), psl[0].stride(1), psl[0].stride(2)), split=split)
                ix = idx[b:b + 1, h:h + 1].contiguous()
            o, lse = N.attn_fwd(rows, ix, 1, 1, n)
            d = do[b:b + 1, h:h + 1].contiguous()
            dq, dk, dv = N.attn_bwd(rows, ix, 1, 1, n, d, lse_all[b:b + 1, h:h + 1].contiguous(),
                                    delta_all[b:b + 1, h:h + 1].contiguous())
            for k, v in zip(("o", "lse", "dq", "dk", "dv"), (o, lse, dq, dk, dv)):
                outs[k].append(v)
    return {k: torch.cat(v, 1).reshape(B, H, *v[0].shape[2:]) for k, v in outs.items()}


@pytest.mark.parametrize("n,B,H", [(9001, 1, 8), (12345, 2, 4), (8448, 1, 16)])
def test_plan_gathered_bit_equal(pkg, dev, n, B, H):
    """Gathered rows (random distinct base and pooled rows), ragged n (partial last block)."""
    print(f"plan gathered n={n} B={B} H={H}", flush=True)
    N = pkg._native
    S, Sp = n, n // 3
    xs = [_rand((B, S, H, 128), 10 + i, dev) for i in range(3)]
    pxs = [_rand((B, Sp, H, 128), 20 + i, dev) for i in range(3)]
    g = torch.Generator().manual_seed(n)
    idx = torch.stack([torch.stack([torch.randperm(S + Sp, generator=g)[:n] for _ in range(H)])
                       for _ in range(B)]).int().to(dev)
    rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)), *pxs,
                  (pxs[0].stride(0), pxs[0].stride(1), pxs[0].stride(2)), split=S)
    o, lse = N.attn_fwd(rows, idx, B, H, n)
    do = _rand((B, H, n, 128), 30, dev)
    delta = (do.float() * o.float()).sum(-1)
    dq, dk, dv = N.attn_bwd(rows, idx, B, H, n, do, lse, delta)
    ref = _per_head(pkg, xs, pxs, idx, S, B, H, n, do, lse, delta)
    for name, got in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.equal(got, ref[name]), f"{name} differs from the per-head (no plan) result"


@pytest.mark.parametrize("n,B,H", [(10000, 2, 4)])
def test_plan_dense_bit_equal(pkg, dev, n, B, H):
    """Identity row map (the dense layers' path)."""
    print(f"plan dense n={n} B={B} H={H}", flush=True)
    N = pkg._native
    xs = [_rand((B, n, H, 128), 40 + i, dev) for i in range(3)]
    rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)))
    o, lse = N.attn_fwd(rows, None, B, H, n)
    do = _rand((B, H, n, 128), 50, dev)
    delta = (do.float() * o.float()).sum(-1)
    dq, dk, dv = N.attn_bwd(rows, None, B, H, n, do, lse, delta)
    ref = _per_head(pkg, xs, None, None, None, B, H, n, do, lse, delta)
    for name, got in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.equal(got, ref[name]), f"{name} differs from the per-head (no plan) result"


def test_plan_dilated_scores_bit_equal(pkg, dev):
    """Dilated scorer: 8 heads x dilation 4 = 32 virtual heads of 4096 tokens (8 bins of 2 blocks per head)."""
    S, H, dil, L, p = 16384, 8, 4, 3, 4
    print(f"plan dilated S={S} H={H} dil={dil}", flush=True)
    N = pkg._native
    xs = [_rand((1, S, H, 128), 60 + i, dev) for i in range(3)]
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    sqk, skq = N.dilated_scores(*xs, dil, S_tot)
    for h in range(H):
        sl = [x[:, :, h:h + 1].contiguous() for x in xs]
        rq, rk = N.dilated_scores(*sl, dil, S_tot)
        assert torch.equal(sqk[:, h:h + 1, :S], rq[..., :S]), f"head {h}: qk scores differ"
        assert torch.equal(skq[:, h:h + 1, :S], rk[..., :S]), f"head {h}: kq scores differ"
