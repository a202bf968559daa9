"""GPU parity of the transformer-block kernels (rotary embedding + q/k/v split,
RMSNorm, SwiGLU, split-K linear) against torch restatements of torchtitan's ops.

The torch references run in fp32 (or fp64 where the exact value is wanted) on
the same bf16 inputs; bf16 outputs must be the correctly rounded value up to
one bf16 ulp.
"""
import pytest
import torch
import torch.nn.functional as F

from conftest import assert_close

pytestmark = pytest.mark.gpu


def _ulp_diff(a, b, slack=None):
    """|a - b| in units of the bf16 ulp of b (elementwise, inputs bf16-valued).
    ``slack`` (same shape) is an absolute allowance subtracted first: fp32
    cancellation in a difference of products loses up to ~2^-23 of the operands'
    size, which is many ulps of a result near zero."""
    a, b = a.float().cpu(), b.float().cpu()
    e = torch.floor(torch.log2(b.abs().clamp_min(1e-30)))
    ulp = torch.pow(2.0, e - 7)
    d = (a - b).abs()
    if slack is not None:
        d = (d - slack.float().cpu()).clamp_min(0)
    return d / ulp


def _pair_norm(x):
    """Norm of each (x[2j], x[2j+1]) pair, repeated on both elements."""
    n = x.float().reshape(*x.shape[:-1], -1, 2).norm(dim=-1, keepdim=True)
    return n.expand(*n.shape[:-1], 2).reshape(x.shape)


@pytest.mark.parametrize("B,S,Hq,Hkv,pad", [(2, 300, 4, 4, 0), (1, 1024, 8, 2, 64)])
def test_rope_qkv(pkg, dev, B, S, Hq, Hkv, pad):
    L, ops = pkg.llama3, pkg.block_ops
    D = 128
    W = (Hq + 2 * Hkv) * D
    print(f"rope B={B} S={S} Hq={Hq} Hkv={Hkv} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(S)
    full = torch.randn(B, S, W + pad, generator=g).bfloat16()
    x = full.to(dev)[..., :W]  # row stride W + pad
    fc = L.precompute_freqs_cis(D, 2 * S, 10000.0)
    q, k, v = ops.rope_qkv(x.requires_grad_(), torch.view_as_real(fc).to(dev), Hq, Hkv, D)
    xc = full[..., :W].float()
    rq, rk = L.apply_rotary_emb(xc[..., :Hq * D].reshape(B, S, Hq, D).double(),
                                xc[..., Hq * D:(Hq + Hkv) * D].reshape(B, S, Hkv, D).double(), fc.to(torch.complex128))
    assert torch.equal(v.cpu(), full[..., (Hq + Hkv) * D:W].reshape(B, S, Hkv, D))
    xin = {"q": xc[..., :Hq * D].reshape(B, S, Hq, D), "k": xc[..., Hq * D:(Hq + Hkv) * D].reshape(B, S, Hkv, D)}
    for got, ref, name in ((q, rq, "q"), (k, rk, "k")):
        assert got.shape == ref.shape and got.is_contiguous()
        d = _ulp_diff(got, ref.bfloat16(), 2.0 ** -22 * _pair_norm(xin[name]))
        assert d.max().item() <= 1, f"rope {name}: {d.max().item()} ulp"
        assert (d == 0).float().mean().item() >= 0.99, f"rope {name}: not the correctly rounded value"
    # backward: rotation by the negative angle, grads given in transposed layouts
    dq = torch.randn(B, Hq, S, D, generator=g).bfloat16()
    dk = torch.randn(B, Hkv, S, D, generator=g).bfloat16()
    dv = torch.randn(B, S, Hkv, D, generator=g).bfloat16()
    torch.autograd.backward([q, k, v], [dq.to(dev).transpose(1, 2), dk.to(dev).transpose(1, 2), dv.to(dev)])
    xr = xc.double().requires_grad_()
    rq, rk = L.apply_rotary_emb(xr[..., :Hq * D].reshape(B, S, Hq, D), xr[..., Hq * D:(Hq + Hkv) * D].reshape(B, S, Hkv, D),
                                fc.to(torch.complex128))
    torch.autograd.backward([rq, rk, xr[..., (Hq + Hkv) * D:]],
                            [dq.transpose(1, 2).double(), dk.transpose(1, 2).double(), dv.reshape(B, S, -1).double()])
    gx = x.grad
    assert gx.shape == (B, S, W)
    gin = torch.cat([dq.transpose(1, 2).reshape(B, S, -1), dk.transpose(1, 2).reshape(B, S, -1),
                     dv.reshape(B, S, -1)], -1)
    d = _ulp_diff(gx, xr.grad.bfloat16(), 2.0 ** -22 * _pair_norm(gin))
    assert d.max().item() <= 1 and (d == 0).float().mean().item() >= 0.99


@pytest.mark.parametrize("rows,dim", [(1000, 1024), (37, 512), (64, 4096), (50, 264)])
def test_rmsnorm(pkg, dev, rows, dim):
    ops = pkg.block_ops
    print(f"rmsnorm rows={rows} dim={dim}", flush=True)
    g = torch.Generator().manual_seed(rows + dim)
    x = (torch.randn(rows, dim, generator=g) * 3).bfloat16()
    w = (1 + 0.1 * torch.randn(dim, generator=g)).bfloat16()
    xd, wd = x.to(dev).requires_grad_(), w.to(dev).requires_grad_()
    y = ops.rms_norm(xd, wd, 1e-5)
    xr, wr = x.double().requires_grad_(), w.double().requires_grad_()
    yr = F.rms_norm(xr, (dim,), wr, 1e-5)
    d = _ulp_diff(y, yr.bfloat16())
    assert d.max().item() <= 1 and (d == 0).float().mean().item() >= 0.98
    dy = torch.randn(rows, dim, generator=g).bfloat16()
    y.backward(dy.to(dev))
    yr.backward(dy.double())
    assert_close(xd.grad, xr.grad, "rmsnorm dx", max_abs=1e-2, rel_l2=4e-3)
    assert_close(wd.grad, wr.grad, "rmsnorm dw", max_abs=1e-2, rel_l2=4e-3)


@pytest.mark.parametrize("rows,dim", [(1000, 1024), (50, 264)])
def test_add_rmsnorm(pkg, dev, rows, dim):
    """h = x + r exactly as torch's bf16 add; y = RMSNorm(h); gradients with both
    the residual branch (dh) and the normalised branch (dy) against fp64."""
    ops = pkg.block_ops
    g = torch.Generator().manual_seed(rows + 7)
    x = torch.randn(rows, dim, generator=g).bfloat16()
    r = torch.randn(rows, dim, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(dim, generator=g)).bfloat16()
    xd, rd, wd = (t.to(dev).requires_grad_() for t in (x, r, w))
    h, y = ops.add_rms_norm(xd, rd, wd, 1e-5)
    assert torch.equal(h, x.to(dev) + r.to(dev))
    hr = (x.double() + r.double()).bfloat16().double().requires_grad_()  # the rounded sum, as h
    wr = w.double().requires_grad_()
    yr = F.rms_norm(hr, (dim,), wr, 1e-5)
    d = _ulp_diff(y, yr.bfloat16())
    assert d.max().item() <= 1 and (d == 0).float().mean().item() >= 0.98
    dh = torch.randn(rows, dim, generator=g).bfloat16()
    dy = torch.randn(rows, dim, generator=g).bfloat16()
    torch.autograd.backward([h, y], [dh.to(dev), dy.to(dev)])
    torch.autograd.backward([hr, yr], [dh.double(), dy.double()])
    assert_close(xd.grad, hr.grad, "add_rmsnorm dx", max_abs=1e-2, rel_l2=4e-3)
    assert torch.equal(xd.grad, rd.grad)
    assert_close(wd.grad, wr.grad, "add_rmsnorm dw", max_abs=1e-2, rel_l2=4e-3)


@pytest.mark.parametrize("rows,Fh", [(777, 1024), (64, 8)])
def test_swiglu_matches_torch_bf16_ops(pkg, dev, rows, Fh):
    """Same roundings as torch's separate bf16 silu and mul (and their backward)."""
    ops = pkg.block_ops
    g = torch.Generator().manual_seed(rows)
    h = (torch.randn(rows, 2 * Fh, generator=g) * 2).bfloat16().to(dev)
    h1 = h.clone().requires_grad_()
    a = ops.swiglu(h1)
    h2 = h.clone().requires_grad_()
    ar = F.silu(h2[:, :Fh]) * h2[:, Fh:]
    da = torch.randn(rows, Fh, generator=g).bfloat16().to(dev)
    a.backward(da)
    ar.backward(da)
    for got, ref, name in ((a, ar, "swiglu"), (h1.grad, h2.grad, "swiglu grad")):
        d = _ulp_diff(got, ref)
        assert d.max().item() <= 1, f"{name}: {d.max().item()} ulp"
        assert (d == 0).float().mean().item() >= 0.999, f"{name}: {(d == 0).float().mean().item()} exact"


@pytest.mark.parametrize("T,O,I", [(32768, 1024, 1024), (8192, 3072, 1024), (1000, 256, 512)])
def test_linear_split_k_weight_grad(pkg, dev, T, O, I):
    ops = pkg.block_ops
    print(f"linear T={T} O={O} I={I} splits={ops.wgrad_splits(T, O, I)}", flush=True)
    g = torch.Generator(device=dev).manual_seed(T)
    x = torch.randn(T, I, device=dev, generator=g).bfloat16().requires_grad_()
    w = (torch.randn(O, I, device=dev, generator=g) * I ** -0.5).bfloat16().requires_grad_()
    y = ops.linear(x, w)
    assert torch.equal(y, F.linear(x.detach(), w.detach()))
    dy = torch.randn(T, O, device=dev, generator=g).bfloat16()
    y.backward(dy)
    ref_dw = dy.float().t() @ x.detach().float()
    ref_dx = dy.float() @ w.detach().float()
    assert_close(w.grad, ref_dw, "dW", max_abs=1e-2, rel_l2=4e-3)
    assert_close(x.grad, ref_dx, "dX", max_abs=1e-2, rel_l2=4e-3)


def test_bf16_rounding_matches_torch(pkg, dev):
    """The library's fp32 -> bf16 conversion (one v_cvt_pk_bf16_f32 per pair) is
    torch's round-to-nearest-even, checked through lh_splitk_sum with one slice
    (out = bf16(0 + x)) on ties of both parities, subnormals, the largest finite
    values, overflow to infinity, infinities and random values of every scale."""
    g = torch.Generator().manual_seed(0)
    hi = torch.randint(0, 1 << 16, (1 << 16,), generator=g, dtype=torch.int64)
    lo = torch.tensor([0x0000, 0x0001, 0x7fff, 0x8000, 0x8001, 0xffff], dtype=torch.int64)
    bits = ((hi[:, None] << 16) | lo[None, :]).flatten()
    bits = bits[((bits >> 23) & 0xff) != 0xff]  # NaN / inf patterns checked separately below
    x = torch.cat([bits.to(torch.int32).view(torch.float32),
                   torch.tensor([float("inf"), float("-inf"), 3.3895314e38, -3.3895314e38, 3.4e38, 1e-45, -1e-45]),
                   torch.randn(1 << 16, generator=g) * torch.pow(2.0, torch.randint(-140, 120, (1 << 16,), generator=g))])
    x = x[: (x.numel() // 8) * 8].contiguous()
    got = pkg._native.splitk_sum(x[None].to(dev)).cpu()
    want = (torch.zeros_like(x) + x).bfloat16()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    nan = pkg._native.splitk_sum(torch.full((1, 8), float("nan"), device=dev)).cpu()
    assert torch.isnan(nan.float()).all()
