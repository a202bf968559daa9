"""GPU parity of the fp16 (IEEE half) row path against the CPU oracle.

The reference path is dtype-generic: its scorers are torch ops on the layer's
rows, its fan-out allocates in the attention output's dtype and SDPA takes
fp16 (src/lighthouse_selection.py:522,528,559,562,589-616,815).  Here fp16 rows
run the same kernels as bf16 ones with fp16 MFMAs (v_mfma_f32_32x32x16_f16) and
fp16 rounding of P, dS, pooled rows, outputs and scores; the norm scorer rounds
its norms to fp16, as torch's norm of fp16 rows does.  Checks mirror the bf16
ones (test_gpu_kernels.py, test_gpu_layer.py): scores equal the fp16-rounded
fp32 norms (up to 1e-3 of them one ulp off from summation order), pooled rows
the fp16-rounded fp32 means, selection bit-exact on the device's own scores,
outputs and gradients within the standard tolerance against the fp32 oracle.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import lh_oracle as O
from oracle import select_ref as R

pytestmark = pytest.mark.gpu
F16 = torch.float16


def _inputs(shape, n, seed, dev):
    g = torch.Generator().manual_seed(seed)
    cpu = [torch.randn(*shape, generator=g).to(F16) for _ in range(n)]
    return cpu, [c.to(dev) for c in cpu]


@pytest.mark.parametrize("S,L,p,H", [(4096, 3, 4, 2), (2000, 6, 2, 1)])
def test_pyramid_fwd_fp16(pkg, dev, S, L, p, H):
    print(f"fp16 pyramid S={S} L={L} p={p} H={H}", flush=True)
    cpu, gpu = _inputs((2, S, H, 128), 3, S + L, dev)
    pq, pk, pv, sqk, skq = pkg._native.pyramid_fwd(*gpu, L, p)
    assert pq.dtype == F16 and sqk.dtype == torch.float32
    r_sqk, r_skq, r_q, r_k, r_v = O.norm_scorer(*[c.float() for c in cpu], p, L)
    for got, ref, name in [(sqk, r_sqk, "scores_qk"), (skq, r_skq, "scores_kq")]:
        got = got.cpu()
        mism = (got != ref.to(F16).float()).float().mean().item()
        assert mism <= 1e-3, f"{name}: {mism:.2e} of scores differ from the fp16-rounded oracle"
        assert_close(got, ref, name, max_abs=1e-2, rel_l2=4e-3)
    for got, ref, name in [(pq, r_q, "pooled q"), (pk, r_k, "pooled k"), (pv, r_v, "pooled v")]:
        ref_p = ref[:, :, S:].transpose(1, 2)
        exact = (got.cpu().float() == ref_p.to(F16).float()).float().mean().item()
        assert exact >= 0.999, f"{name}: only {exact:.4f} of values equal the fp16-rounded fp32 mean"
        assert_close(got, ref_p, name)


@pytest.mark.parametrize("n,B,H", [(17, 2, 1), (333, 2, 2), (3000, 1, 3)])
def test_attention_fp16_gathered(pkg, dev, n, B, H):
    """Explicit row maps over base and pooled fp16 rows, ragged lengths; the last
    case has more blocks than CUs (persistent launch with work queues)."""
    S, Sp = max(640, n), max(160, n // 3)
    print(f"fp16 gathered attention n={n} B={B} H={H}", flush=True)
    cpu, gpu = _inputs((B, S, H, 128), 3, 40 + n, dev)
    pcpu, pgpu = _inputs((B, Sp, H, 128), 3, 50 + n, dev)
    g = torch.Generator().manual_seed(n)
    idx = torch.stack([torch.stack([torch.randperm(S + Sp, generator=g)[:n] for _ in range(H)])
                       for _ in range(B)]).int()
    x, px = gpu[0], pgpu[0]
    rows = pkg._native.Rows(*gpu, (x.stride(0), x.stride(1), x.stride(2)), *pgpu,
                            (px.stride(0), px.stride(1), px.stride(2)), split=S)
    o, lse = pkg._native.attn_fwd(rows, idx.to(dev), B, H, n)
    assert o.dtype == F16
    gi = idx.long()[..., None].expand(-1, -1, -1, 128)
    sel = [torch.gather(torch.cat([c, p], 1).float().transpose(1, 2), 2, gi) for c, p in zip(cpu, pcpu)]
    q, k, v = [s.clone().requires_grad_() for s in sel]
    ref = O.sdpa_causal(q, k, v)
    assert_close(o, ref, "fp16 gathered attention out")
    do = torch.randn(B, H, n, 128, generator=g).to(F16)
    ref.backward(do.float())
    delta = (do.float() * o.float().cpu()).sum(-1).to(dev)
    dq, dk, dv = pkg._native.attn_bwd(rows, idx.to(dev), B, H, n, do.to(dev), lse, delta)
    for name, got, r in (("dq", dq, q.grad), ("dk", dk, k.grad), ("dv", dv, v.grad)):
        assert got.dtype == F16
        assert_close(got, r, f"fp16 gathered {name}")


def test_attention_fp16_dense(pkg, dev):
    n, H = 1000, 3
    print(f"fp16 dense attention n={n} H={H}", flush=True)
    cpu, gpu = _inputs((1, n, H, 128), 3, n, dev)
    x = gpu[0]
    rows = pkg._native.Rows(*gpu, (x.stride(0), x.stride(1), x.stride(2)))
    o, lse = pkg._native.attn_fwd(rows, None, 1, H, n)
    q, k, v = [c.float().transpose(1, 2).clone().requires_grad_() for c in cpu]
    ref = O.sdpa_causal(q, k, v)
    assert_close(o, ref, "fp16 dense out")
    do = torch.randn(1, H, n, 128).to(F16)
    ref.backward(do.float())
    delta = (do.float() * o.float().cpu()).sum(-1).to(dev)
    dq, dk, dv = pkg._native.attn_bwd(rows, None, 1, H, n, do.to(dev), lse, delta)
    for name, got, r in (("dq", dq, q.grad), ("dk", dk, k.grad), ("dv", dv, v.grad)):
        assert_close(got, r, f"fp16 dense {name}")


def test_dense_module_fp16(pkg, dev):
    """The full-attention layers' module on fp16 [B, H, S, D] views."""
    B, H, S = 1, 2, 700
    g = torch.Generator().manual_seed(3)
    xs = [torch.randn(B, S, H, 128, generator=g).to(F16) for _ in range(3)]
    xg = [x.to(dev).transpose(1, 2).requires_grad_() for x in xs]
    out = pkg.dense_attention.dense_causal_attention(*xg)
    assert out.dtype == F16
    do = torch.randn(B, H, S, 128, generator=g).to(F16)
    out.backward(do.to(dev))
    xc = [x.float().transpose(1, 2).requires_grad_() for x in xs]
    ref = O.sdpa_causal(*xc)
    ref.backward(do.float())
    assert_close(out, ref, "fp16 dense module out")
    for name, a, c in zip("qkv", xg, xc):
        assert_close(a.grad, c.grad, f"fp16 dense module d{name}")


def _selection(S, L, p, k, H, seed, strict=True):
    """An index set from random scores (the kernels under test only use the indices)."""
    g = torch.Generator().manual_seed(seed)
    S_tot = sum(O.level_lengths(S, L, p))
    a = (torch.randn(1, H, S_tot, generator=g).abs() * 4).float().numpy()
    b = (torch.randn(1, H, S_tot, generator=g).abs() * 4).float().numpy()
    return O.select_indices(a, b, L, p, k, S, strict=strict), S_tot


def test_scatter_fp16(pkg, dev):
    S, L, p, k = 4096, 3, 4, 256
    idx, S_tot = _selection(S, L, p, k, 2, 11)
    n = idx.shape[-1]
    g = torch.Generator().manual_seed(12)
    attn = torch.randn(1, 2, n, 128, generator=g).to(F16)
    dout = torch.randn(1, 2, S, 128, generator=g).to(F16)
    o = torch.randn(1, 2, n, 128, generator=g).to(F16)
    idx_t = torch.from_numpy(idx)
    inv = torch.from_numpy(O.inverse_map(idx, S_tot)).to(dev)
    print(f"fp16 scatter S={S} n={n}", flush=True)
    out = pkg._native.scatter_fwd(attn.to(dev), inv, S, S, L, p)
    assert out.dtype == F16
    assert_close(out, O.scatter_fwd(attn.float(), idx_t, S, L, p, N_total=S), "fp16 scatter fwd",
                 max_abs=2e-3, rel_l2=1e-3)
    dattn, delta = pkg._native.scatter_bwd(dout.to(dev), idx_t.to(dev), o.to(dev), S, L, p)
    assert dattn.dtype == F16
    assert_close(dattn, O.scatter_bwd(dout.float(), idx_t, S, L, p), "fp16 scatter bwd", max_abs=2e-3, rel_l2=1e-3)
    assert_close(delta, (dattn.float().cpu() * o.float()).sum(-1), "fp16 delta", max_abs=1e-4, rel_l2=1e-5)


def test_pyramid_bwd_fp16(pkg, dev):
    S, L, p, k, H = 4096, 3, 4, 256, 2
    print(f"fp16 pyramid bwd S={S}", flush=True)
    idx, S_tot = _selection(S, L, p, k, H, 31)
    n = idx.shape[-1]
    g = torch.Generator().manual_seed(32)
    gs = [torch.randn(1, H, n, 128, generator=g).to(F16) for _ in range(3)]
    inv = torch.from_numpy(O.inverse_map(idx, S_tot)).to(dev)
    out = pkg._native.pyramid_bwd(*[x.to(dev) for x in gs], inv, 1, S, H, L, p)
    idx_t = torch.from_numpy(idx).long()
    for name, gsel, got in zip("qkv", gs, out):
        assert got.dtype == F16
        x = torch.zeros(1, S, H, 128, requires_grad=True)
        _, _, xc, _, _ = O.norm_scorer(x, x, x, p, L)
        sel = torch.gather(xc, 2, idx_t[..., None].expand(-1, -1, -1, 128))
        (sel * gsel.float()).sum().backward()
        assert_close(got, x.grad, f"fp16 pyramid bwd d{name}", max_abs=2e-3, rel_l2=1e-3)


def test_dilated_scores_fp16(pkg, dev):
    S, H, dil, L, p = 1024, 2, 4, 3, 4
    cpu, gpu = _inputs((1, S, H, 128), 3, S * dil, dev)
    _, _, S_tot = pkg._native.pyramid_lengths(S, L, p)
    sqk, skq = pkg._native.dilated_scores(*gpu, dil, S_tot)
    r_qk, r_kq, *_ = O.dilated_scorer(*[c.float() for c in cpu], dil, p, L)
    assert_close(sqk[..., :S], r_qk[..., :S], "fp16 dilated scores qk", max_abs=1e-2, rel_l2=5e-3)
    assert_close(skq[..., :S], r_kq[..., :S], "fp16 dilated scores kq", max_abs=1e-2, rel_l2=5e-3)


def _check_layer_fp16(pkg, dev, B, S, H, L, p, k, heads=None, dilation=0, strict=True, seed=0):
    print(f"fp16 layer B={B} S={S} H={H} L={L} p={p} k={k} dil={dilation} heads={heads}", flush=True)
    g = torch.Generator().manual_seed(seed)
    cpu = [torch.randn(B, S, H, 128, generator=g).to(F16) for _ in range(3)]
    dout = torch.randn(B, H, S, 128, generator=g).to(F16)
    xs = [c.to(dev).requires_grad_() for c in cpu]
    out, idx = pkg.lighthouse_layer(*xs, num_levels=L, pooling_factor=p, topk=k, strict=strict, dilation=dilation)
    assert out.dtype == F16
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    with torch.no_grad():
        _, _, S_tot = pkg._native.pyramid_lengths(S, L, p)
        det = [x.detach() for x in xs]
        if dilation:
            sc = pkg._native.dilated_scores(*det, dilation, S_tot)
            _, _, _, sqk, skq = pkg._native.pyramid_fwd(*det, L, p, scores=sc)
        else:
            _, _, _, sqk, skq = pkg._native.pyramid_fwd(*det, L, p)
    S_sel = O.tile_geometry(S, L, p, k).S_sel if strict else pkg._native.geometry(S, L, p, k, strict=False)[3]
    ref_idx = R.select_indices_c(sqk.cpu().numpy(), skq.cpu().numpy(), L, p, k, S, S_sel, strict=strict)
    got_idx = idx.cpu().numpy()
    assert np.array_equal(got_idx, ref_idx), f"{(got_idx != ref_idx).sum()} selected indices differ"
    hs = list(range(H)) if heads is None else list(heads)
    xc = [c[:, :, hs].float().requires_grad_() for c in cpu]
    ref_out, _ = O.lighthouse_layer(*xc, L, p, k, scorer="dilated" if dilation else "norm",
                                    dilation=dilation or 4, indices=ref_idx[:, hs], strict=strict)
    ref_out.backward(dout[:, hs].float())
    assert_close(out.detach()[:, hs], ref_out, "fp16 layer out")
    for n, x, c in zip("qkv", xs, xc):
        assert x.grad.dtype == F16
        assert_close(x.grad[:, :, hs], c.grad, f"fp16 layer d{n}")


def test_layer_fp16_small(pkg, dev):
    _check_layer_fp16(pkg, dev, 1, 4096, 2, 3, 4, 256)


def test_layer_fp16_dilated(pkg, dev):
    _check_layer_fp16(pkg, dev, 1, 4096, 2, 3, 4, 256, dilation=4, seed=5)


def test_layer_fp16_cfg2(pkg, dev):
    """cfg2's shape (S = 32768, H = 8, k = 2048, L = 3, p = 4) in fp16: indices
    bit-exact on every head, output and gradients on a subset of heads."""
    _check_layer_fp16(pkg, dev, 1, 32768, 8, 3, 4, 2048, heads=(0, 5), seed=2)
