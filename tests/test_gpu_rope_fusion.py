"""GPU parity of the rotary embedding fused into the Lighthouse layer.

rotate + pyramid  <- torchtitan apply_rotary_emb on q, k (lighthouse-attention.patch:707-712)
                     then DialatedLighthouseNormScorer.forward (src/lighthouse_selection.py:589-616)
pyramid backward  <- autograd of gather/cat/mean (src/lighthouse_selection.py:604-614,800-813)
                     then of the rotation

The fused forward must give the same bits as the two pinned kernels it replaces
(rotation, then pyramid), so it inherits their pins; the fused backward is checked
against autograd of the fp64 rotation composed with the oracle's pyramid (within
one bf16 ulp), and is at least as accurate as the unfused composition, which
rounds twice.
"""
import pytest
import torch

from conftest import assert_close
from oracle import lh_oracle as O

pytestmark = pytest.mark.gpu

D = 128


def _inputs(pkg, dev, B, S, H, pad, seed):
    g = torch.Generator().manual_seed(seed)
    W = 3 * H * D
    full = torch.randn(B, S, W + pad, generator=g).bfloat16()
    x = full.to(dev)[..., :W]  # row stride W + pad when padded
    fc = pkg.llama3.precompute_freqs_cis(D, S + 64, 10000.0)
    return full[..., :W], x, fc, torch.view_as_real(fc).contiguous().to(dev)


def _bf16_ulps(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    ulp = torch.pow(2.0, torch.floor(torch.log2(b.abs().clamp_min(1e-30))) - 7)
    return (a - b).abs() / ulp


@pytest.mark.parametrize("B,S,H,L,p,pad", [(1, 4096, 2, 3, 4, 0), (2, 1000, 3, 3, 4, 64), (1, 2048, 1, 5, 2, 0),
                                           (1, 512, 2, 1, 4, 0)])
def test_rope_pyramid_fwd_is_rotate_then_pyramid(pkg, dev, B, S, H, L, p, pad):
    N = pkg._native
    print(f"rope pyramid fwd B={B} S={S} H={H} L={L} p={p} pad={pad}", flush=True)
    cpu, x, fc, fr = _inputs(pkg, dev, B, S, H, pad, S + H)
    xr, pq, pk, pv, sqk, skq = N.rope_pyramid_fwd(x, fr, H, L, p)
    q, k, v = N.rope_qkv_fwd(x, fr, H, H)
    pq2, pk2, pv2, sqk2, skq2 = N.pyramid_fwd(q, k, v, L, p)
    torch.cuda.synchronize()
    hd = H * D
    assert torch.equal(xr[..., :hd].reshape(B, S, H, D), q)
    assert torch.equal(xr[..., hd:2 * hd].reshape(B, S, H, D), k)
    for a, b, name in ((pq, pq2, "pooled q"), (pk, pk2, "pooled k"), (pv, pv2, "pooled v"),
                       (sqk, sqk2, "scores qk"), (skq, skq2, "scores kq")):
        assert torch.equal(a, b), name
    # and the rotated rows themselves against the fp64 rotation of the same inputs
    rq, rk = pkg.llama3.apply_rotary_emb(cpu[..., :hd].reshape(B, S, H, D).double(),
                                         cpu[..., hd:2 * hd].reshape(B, S, H, D).double(),
                                         fc[:S].to(torch.complex128))
    for got, ref in ((q, rq), (k, rk)):
        d = _bf16_ulps(got, ref.bfloat16())
        assert (d <= 1).float().mean().item() >= 0.999 and (d == 0).float().mean().item() >= 0.99


def test_rope_pyramid_fwd_rejects_bad_freqs(pkg, dev):
    N = pkg._native
    _, x, _, fr = _inputs(pkg, dev, 1, 256, 1, 0, 1)
    with pytest.raises(AssertionError):
        N.rope_pyramid_fwd(x, fr[:100].contiguous(), 1, 3, 4)  # fewer positions than S


def _selection(pkg, dev, x, fr, H, L, p, k):
    N = pkg._native
    S = x.shape[1]
    _, _, _, _, sqk, skq = N.rope_pyramid_fwd(x, fr, H, L, p)
    idx, inv = N.select_topk(sqk, skq, S, L, p, k, tie="reference", strict=False)
    return idx, inv


@pytest.mark.parametrize("S,L,p,k,H", [(4096, 3, 4, 256, 2), (2048, 4, 2, 128, 1)])
def test_pyramid_rope_bwd(pkg, dev, S, L, p, k, H):
    N = pkg._native
    print(f"pyramid rope bwd S={S} L={L} p={p} k={k} H={H}", flush=True)
    _, x, fc, fr = _inputs(pkg, dev, 1, S, H, 0, 5)
    idx, inv = _selection(pkg, dev, x, fr, H, L, p, k)
    n = idx.shape[-1]
    g = torch.Generator().manual_seed(S + k)
    gs = [torch.randn(1, H, n, D, generator=g).bfloat16() for _ in range(3)]
    dx = N.pyramid_rope_bwd(*[t.to(dev) for t in gs], inv, fr, 1, S, H, L, p)
    assert dx.shape == (1, S, 3 * H * D)
    # reference: autograd of (fp64 rotation -> oracle pyramid -> gather) on a differentiable input
    idx_t = idx.long().cpu()
    hd = H * D
    x0 = torch.zeros(1, S, 3 * hd, dtype=torch.float64, requires_grad=True)
    q0, k0, v0 = x0[..., :hd].reshape(1, S, H, D), x0[..., hd:2 * hd].reshape(1, S, H, D), x0[..., 2 * hd:].reshape(1, S, H, D)
    rq, rk = pkg.llama3.apply_rotary_emb(q0, k0, fc[:S].to(torch.complex128))
    _, _, cq, ck, cv = O.norm_scorer(rq, rk, v0, p, L)
    gi = idx_t[..., None].expand(-1, -1, -1, D)
    loss = sum((torch.gather(c, 2, gi) * gsel.double()).sum() for c, gsel in zip((cq, ck, cv), gs))
    loss.backward()
    ref = x0.grad
    for sl, name in ((slice(0, hd), "dq"), (slice(hd, 2 * hd), "dk"), (slice(2 * hd, 3 * hd), "dv")):
        assert_close(dx[..., sl], ref[..., sl], f"fused pyramid bwd {name}", max_abs=1e-2, rel_l2=4e-3)
        d = _bf16_ulps(dx[..., sl], ref[..., sl].bfloat16())
        assert (d <= 1).float().mean().item() >= 0.999, f"{name}: not within one ulp of the fp64 gradient"
    # the unfused composition rounds before rotating back (a rotation of rounded values
    # loses ulps where the pair nearly cancels): the fused result is at least as close
    dq, dk, dv = N.pyramid_bwd(*[t.to(dev) for t in gs], inv, 1, S, H, L, p)
    gx = N.rope_qkv_bwd(dq, dk, dv, fr, H, H)
    e_fused = (dx[..., :2 * hd].double().cpu() - ref[..., :2 * hd]).norm()
    e_unfused = (gx[..., :2 * hd].double().cpu() - ref[..., :2 * hd]).norm()
    assert e_fused <= e_unfused, (e_fused.item(), e_unfused.item())
    assert torch.equal(dx[..., 2 * hd:], gx[..., 2 * hd:])  # v is not rotated: same single rounding


@pytest.mark.parametrize("S,L,p,k,H,seq_major", [(4096, 3, 4, 256, 2, False), (3000, 3, 4, 128, 1, True)])
def test_layer_rope_equals_rope_then_layer(pkg, dev, S, L, p, k, H, seq_major):
    """lighthouse_layer_rope(xqkv) == lighthouse_layer(rope(q), rope(k), v): identical
    forward bits and indices; gradients w.r.t. xqkv within tolerance of each other
    (the fused backward rounds once where the composition rounds twice), the v block
    bit-equal."""
    N, ops = pkg._native, pkg.block_ops
    print(f"layer rope S={S} L={L} p={p} k={k} H={H} seq_major={seq_major}", flush=True)
    _, x, _, fr = _inputs(pkg, dev, 1, S, H, 0, 9)
    x1 = x.clone().requires_grad_()
    out, idx = pkg.lighthouse_layer_rope(x1, fr, H, L, p, k, strict=False, seq_major=seq_major)
    x2 = x.clone().requires_grad_()
    q, kk, v = ops.rope_qkv(x2, fr, H, H, D)
    out2, idx2 = pkg.lighthouse_layer(q, kk, v, L, p, k, strict=False, seq_major=seq_major)
    assert torch.equal(idx, idx2)
    assert torch.equal(out, out2)
    g = torch.Generator(device=dev).manual_seed(3)
    do = torch.randn(out.shape, device=dev, generator=g).bfloat16()
    out.backward(do)
    out2.backward(do)
    assert_close(x1.grad, x2.grad.float(), "d xqkv", max_abs=1e-2, rel_l2=4e-3)
    hd = H * D
    assert torch.equal(x1.grad[..., 2 * hd:], x2.grad[..., 2 * hd:])
