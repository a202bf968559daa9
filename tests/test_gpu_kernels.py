"""GPU parity of the individual kernels against the CPU oracle.

pyramid fwd   <- DialatedLighthouseNormScorer.forward   (src/lighthouse_selection.py:589-616)
scatter f/b   <- _scatter_fanout_{fwd,bwd}_kernel        (src/lighthouse_selection.py:408-514)
attention f/b <- gather + causal SDPA                    (src/lighthouse_selection.py:800-815)
dilated       <- DilatedLighthouseScorer.forward          (src/lighthouse_selection.py:635-653)
pyramid bwd   <- autograd of gather/cat/mean              (src/lighthouse_selection.py:604-614,800-813)
"""
import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import lh_oracle as O

pytestmark = pytest.mark.gpu


def _bf16_inputs(shape, n, seed, dev):
    g = torch.Generator().manual_seed(seed)
    cpu = [torch.randn(*shape, generator=g).bfloat16() for _ in range(n)]
    return cpu, [c.to(dev) for c in cpu]


@pytest.mark.parametrize("S,L,p,H", [(4096, 3, 4, 2), (4100, 3, 4, 2), (2048, 5, 2, 3), (1024, 2, 8, 1),
                                     (4096, 3, 32, 1), (2000, 6, 2, 1)])
def test_pyramid_fwd(pkg, dev, S, L, p, H):
    print(f"pyramid S={S} L={L} p={p} H={H}", flush=True)
    cpu, gpu = _bf16_inputs((2, S, H, 128), 3, S + L, dev)
    pq, pk, pv, sqk, skq = pkg._native.pyramid_fwd(*gpu, L, p)
    torch.cuda.synchronize()
    # oracle in fp32 on the same bf16 inputs; the reference rounds each output to bf16 once
    r_sqk, r_skq, r_q, r_k, r_v = O.norm_scorer(*[c.float() for c in cpu], p, L)
    lens, offs, S_tot = pkg._native.pyramid_lengths(S, L, p)
    assert sqk.shape == (2, H, S_tot)
    for got, ref, name in [(sqk, r_sqk, "scores_qk"), (skq, r_skq, "scores_kq")]:
        ref_b = ref.bfloat16().float()
        got = got.cpu()
        mism = (got != ref_b).float().mean().item()
        assert mism <= 1e-3, f"{name}: {mism:.2e} of scores differ from the bf16-rounded oracle"
        assert_close(got, ref, name, max_abs=1e-2, rel_l2=4e-3)
    for got, ref, name in [(pq, r_q, "pooled q"), (pk, r_k, "pooled k"), (pv, r_v, "pooled v")]:
        ref_p = ref[:, :, S:].transpose(1, 2)  # [B, Sp, H, D]
        exact = (got.cpu().float() == ref_p.bfloat16().float()).float().mean().item()
        assert exact >= 0.999, f"{name}: only {exact:.4f} of values equal the bf16-rounded fp32 mean"
        assert_close(got, ref_p, name)


def test_pyramid_fwd_given_scores_pools_only(pkg, dev):
    S, L, p, H = 2048, 3, 4, 2
    cpu, gpu = _bf16_inputs((1, S, H, 128), 3, 7, dev)
    _, _, S_tot = pkg._native.pyramid_lengths(S, L, p)
    base = torch.rand(1, H, S, device=dev)
    sqk = torch.full((1, H, S_tot), float("nan"), device=dev)
    skq = torch.full((1, H, S_tot), float("nan"), device=dev)
    sqk[..., :S] = base
    skq[..., :S] = base * 2
    pkg._native.pyramid_fwd(*gpu, L, p, scores=(sqk, skq))
    lens, offs, _ = pkg._native.pyramid_lengths(S, L, p)
    for l in range(1, L):
        c = p ** l
        ref = base.reshape(1, H, S // c, c).amax(-1)
        assert torch.equal(sqk[..., offs[l]:offs[l] + lens[l]], ref)
        assert torch.equal(skq[..., offs[l]:offs[l] + lens[l]], 2 * ref)


def _selection(S, L, p, k, H, seed, strict=True):
    g = torch.Generator().manual_seed(seed)
    S_tot = sum(O.level_lengths(S, L, p))
    a = (torch.randn(1, H, S_tot, generator=g).abs() * 4).bfloat16().float().numpy()
    b = (torch.randn(1, H, S_tot, generator=g).abs() * 4).bfloat16().float().numpy()
    return O.select_indices(a, b, L, p, k, S, strict=strict), S_tot


@pytest.mark.parametrize("S,L,p,k,S_out", [(4096, 3, 4, 256, 4096), (2048, 2, 2, 128, 2048),
                                           (4096, 3, 4, 1536, 4096), (2048, 3, 4, 128, 2100)])
def test_scatter_fwd_bwd(pkg, dev, S, L, p, k, S_out):
    idx, S_tot = _selection(S, L, p, k, 2, 11, strict=(k != 1536))
    n = idx.shape[-1]
    g = torch.Generator().manual_seed(12)
    attn = torch.randn(1, 2, n, 128, generator=g).bfloat16()
    dout = torch.randn(1, 2, S_out, 128, generator=g).bfloat16()
    o = torch.randn(1, 2, n, 128, generator=g).bfloat16()
    idx_t = torch.from_numpy(idx)
    inv = torch.from_numpy(O.inverse_map(idx, S_tot)).to(dev)
    print(f"scatter S={S} L={L} p={p} k={k} S_out={S_out} n={n}", flush=True)
    out = pkg._native.scatter_fwd(attn.to(dev), inv, S, S_out, L, p)
    ref = O.scatter_fwd(attn.float(), idx_t, S, L, p, N_total=S_out)
    assert_close(out, ref, "scatter fwd", max_abs=8e-3, rel_l2=4e-3)
    dattn, delta = pkg._native.scatter_bwd(dout.to(dev), idx_t.to(dev), o.to(dev), S, L, p)
    ref_d = O.scatter_bwd(dout.float(), idx_t, S, L, p)
    assert_close(dattn, ref_d, "scatter bwd", max_abs=8e-3, rel_l2=4e-3)
    ref_delta = (dattn.float().cpu() * o.float()).sum(-1)
    assert_close(delta, ref_delta, "delta", max_abs=1e-4, rel_l2=1e-5)
    # sequence-major storage ([B, S, H, D]) of the output and of the incoming gradient
    out_sm = pkg._native.scatter_fwd(attn.to(dev), inv, S, S_out, L, p, seq_major=True)
    assert out_sm.shape == out.shape and out_sm.transpose(1, 2).is_contiguous()
    assert torch.equal(out_sm, out)
    dout_sm = dout.to(dev).transpose(1, 2).contiguous().transpose(1, 2)
    dattn_sm, delta_sm = pkg._native.scatter_bwd(dout_sm, idx_t.to(dev), o.to(dev), S, L, p)
    assert torch.equal(dattn_sm, dattn) and torch.equal(delta_sm, delta)


def _attn_case(pkg, dev, S, L, p, k, H, seed):
    """Native pyramid + selection, then return everything the attention tests need."""
    cpu, gpu = _bf16_inputs((1, S, H, 128), 3, seed, dev)
    pq, pk, pv, sqk, skq = pkg._native.pyramid_fwd(*gpu, L, p)
    idx, inv = pkg._native.select_topk(sqk, skq, S, L, p, k, strict=False)
    cat = [torch.cat([x, pp], 1).transpose(1, 2).float().cpu() for x, pp in zip(gpu, (pq, pk, pv))]
    gi = idx.long().cpu()[..., None].expand(-1, -1, -1, 128)
    sel = [torch.gather(c, 2, gi) for c in cat]  # fp32 copies of the exact bf16 rows
    return gpu, (pq, pk, pv), idx, inv, sel


@pytest.mark.parametrize("S,L,p,k,H", [(4096, 3, 4, 256, 2), (4096, 3, 4, 1536, 1), (2048, 2, 2, 128, 2)])
def test_attention_fwd_bwd_gathered(pkg, dev, S, L, p, k, H):
    print(f"attention S={S} L={L} p={p} k={k} H={H}", flush=True)
    gpu, pooled, idx, inv, sel = _attn_case(pkg, dev, S, L, p, k, H, 21)
    n = idx.shape[-1]
    rows = pkg.lighthouse_selection._base_rows(*gpu, *pooled)
    o, lse = pkg._native.attn_fwd(rows, idx, 1, H, n)
    q, kk, v = [s.clone().requires_grad_() for s in sel]
    ref = O.sdpa_causal(q, kk, v)
    assert_close(o, ref, "attention out")
    # log-sum-exp (stored in the exp2 domain)
    sc = (q @ kk.transpose(-1, -2)) / 128 ** 0.5
    sc = sc.masked_fill(~torch.ones(n, n, dtype=torch.bool).tril(), float("-inf"))
    ref_lse = torch.logsumexp(sc, -1) / np.log(2.0)
    assert_close(lse, ref_lse.detach(), "lse", max_abs=1e-3, rel_l2=1e-4)
    g = torch.Generator().manual_seed(5)
    do = torch.randn(1, H, n, 128, generator=g).bfloat16()
    ref.backward(do.float())
    delta = (do.float() * o.float().cpu()).sum(-1).to(dev)
    dq, dk, dv = pkg._native.attn_bwd(rows, idx, 1, H, n, do.to(dev), lse, delta)
    assert_close(dq, q.grad, "dq")
    assert_close(dk, kk.grad, "dk")
    assert_close(dv, v.grad, "dv")


@pytest.mark.parametrize("n,B,H", [(8, 1, 2), (17, 2, 1), (100, 1, 3), (333, 2, 2)])
def test_attention_gathered_ragged(pkg, dev, n, B, H):
    """Explicit row maps (random distinct rows of the base and pooled tensors,
    in random order) at lengths that leave partial tiles and partial index
    groups: the gathered-row copies of every kernel, forward and backward."""
    S, Sp = 640, 160
    print(f"gathered attention n={n} B={B} H={H}", flush=True)
    cpu, gpu = _bf16_inputs((B, S, H, 128), 3, 40 + n, dev)
    pcpu, pgpu = _bf16_inputs((B, Sp, H, 128), 3, 50 + n, dev)
    g = torch.Generator().manual_seed(n)
    idx = torch.stack([torch.stack([torch.randperm(S + Sp, generator=g)[:n] for _ in range(H)]) for _ in range(B)])
    idx = idx.int()
    x, px = gpu[0], pgpu[0]
    rows = pkg._native.Rows(*gpu, (x.stride(0), x.stride(1), x.stride(2)), *pgpu,
                            (px.stride(0), px.stride(1), px.stride(2)), split=S)
    o, lse = pkg._native.attn_fwd(rows, idx.to(dev), B, H, n)
    gi = idx.long()[..., None].expand(-1, -1, -1, 128)
    sel = [torch.gather(torch.cat([c, p], 1).float().transpose(1, 2), 2, gi) for c, p in zip(cpu, pcpu)]
    q, k, v = [s.clone().requires_grad_() for s in sel]
    ref = O.sdpa_causal(q, k, v)
    assert_close(o, ref, "gathered attention out")
    do = torch.randn(B, H, n, 128, generator=g).bfloat16()
    ref.backward(do.float())
    delta = (do.float() * o.float().cpu()).sum(-1).to(dev)
    dq, dk, dv = pkg._native.attn_bwd(rows, idx.to(dev), B, H, n, do.to(dev), lse, delta)
    assert_close(dq, q.grad, "gathered dq")
    assert_close(dk, k.grad, "gathered dk")
    assert_close(dv, v.grad, "gathered dv")


@pytest.mark.parametrize("n", [1000, 64, 200])
def test_attention_dense_ragged(pkg, dev, n):
    """Identity row map, lengths not a multiple of the 128-row block."""
    H = 3
    cpu, gpu = _bf16_inputs((1, n, H, 128), 3, n, dev)
    x = gpu[0]
    rows = pkg._native.Rows(*gpu, (x.stride(0), x.stride(1), x.stride(2)))  # (batch, seq, head)
    print(f"dense attention n={n} H={H}", flush=True)
    o, lse = pkg._native.attn_fwd(rows, None, 1, H, n)
    q, k, v = [c.float().transpose(1, 2).clone().requires_grad_() for c in cpu]
    ref = O.sdpa_causal(q, k, v)
    assert_close(o, ref, "dense attention out")
    do = torch.randn(1, H, n, 128).bfloat16()
    ref.backward(do.float())
    delta = (do.float() * o.float().cpu()).sum(-1).to(dev)
    dq, dk, dv = pkg._native.attn_bwd(rows, None, 1, H, n, do.to(dev), lse, delta)
    assert_close(dq, q.grad, "dense dq")
    assert_close(dk, k.grad, "dense dk")
    assert_close(dv, v.grad, "dense dv")


@pytest.mark.parametrize("S,H,dil", [(1024, 2, 4), (2048, 1, 2)])
def test_dilated_scores(pkg, dev, S, H, dil):
    cpu, gpu = _bf16_inputs((1, S, H, 128), 3, S * dil, dev)
    L, p = 3, 4
    _, _, S_tot = pkg._native.pyramid_lengths(S, L, p)
    sqk, skq = pkg._native.dilated_scores(*gpu, dil, S_tot)
    r_qk, r_kq, *_ = O.dilated_scorer(*[c.float() for c in cpu], dil, p, L)
    assert_close(sqk[..., :S], r_qk[..., :S], "dilated scores qk", max_abs=1e-2, rel_l2=5e-3)
    assert_close(skq[..., :S], r_kq[..., :S], "dilated scores kq", max_abs=1e-2, rel_l2=5e-3)


@pytest.mark.parametrize("S,L,p,k,strict", [(4096, 3, 4, 256, True), (4096, 3, 4, 1536, False),
                                             (4100, 3, 4, 256, False)])
def test_pyramid_bwd(pkg, dev, S, L, p, k, strict):
    """(4100 tokens x 2 heads: a grid of 513 blocks, not a multiple of the 8
    XCDs, takes the plain block order and ends in a partial block.)"""
    H = 2
    print(f"pyramid bwd S={S} L={L} p={p} k={k}", flush=True)
    idx, S_tot = _selection(S, L, p, k, H, 31, strict=strict)
    n = idx.shape[-1]
    g = torch.Generator().manual_seed(32)
    gs = [torch.randn(1, H, n, 128, generator=g).bfloat16() for _ in range(3)]
    inv = torch.from_numpy(O.inverse_map(idx, S_tot)).to(dev)
    out = pkg._native.pyramid_bwd(*[x.to(dev) for x in gs], inv, 1, S, H, L, p)
    # reference: autograd of the oracle's gather + pyramid on a differentiable input
    idx_t = torch.from_numpy(idx).long()
    for name, gsel, got in zip("qkv", gs, out):
        x = torch.zeros(1, S, H, 128, requires_grad=True)
        _, _, xc, _, _ = O.norm_scorer(x, x, x, p, L)
        sel = torch.gather(xc, 2, idx_t[..., None].expand(-1, -1, -1, 128))
        (sel * gsel.float()).sum().backward()
        assert_close(got, x.grad, f"pyramid bwd d{name}", max_abs=1e-2, rel_l2=4e-3)
