"""GPU checks of the committed golden fixtures, the index check mode and the
block ops' handling of non-contiguous inputs.

golden selection <- lighthouse_selection_chunked_topk_kernel + sort
                    (src/lighthouse_selection_cuda.py:114-331,359-428): the index dumps
                    in tests/golden/ (cfg1's geometry on fp32 scores, and a tie-heavy
                    strict case), reproduced by the device kernel bit for bit
index checks     <- the reference's scatter kernels skip idx = -1
                    (src/lighthouse_selection.py:432-459); duplicates are refused here
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from conftest import assert_close

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("tie", ["reference", "lower_index"])
@pytest.mark.parametrize("name", ["cfg1_selection.npz", "ties_4096_k256.npz"])
def test_golden_selection_on_device(pkg, dev, name, tie):
    meta = json.load(open(os.path.join(GOLDEN, "manifest.json")))[name]
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    S, L, p, k, strict = meta["S"], meta["L"], meta["p"], meta["topk"], meta["strict"]
    print(f"golden {name} tie={tie} S={S} L={L} p={p} k={k} strict={strict} H={meta['H']}", flush=True)
    sqk = torch.from_numpy(g["scores_qk"]).to(dev)
    skq = torch.from_numpy(g["scores_kq"]).to(dev)
    idx, inv = pkg._native.select_topk(sqk, skq, S, L, p, k, tie=tie, strict=strict)
    got = idx.cpu().numpy()
    want = g[f"indices_{tie}"]
    assert got.shape == want.shape
    assert np.array_equal(got, want), f"{(got != want).sum()} of {want.size} indices differ"
    assert hashlib.sha256(got.tobytes()).hexdigest() == meta[f"sha256_{tie}"]
    # the inverse map written by the same launch names every selected position once
    inv = inv.cpu().numpy()
    for h in range(got.shape[1]):
        assert np.array_equal(inv[0, h][got[0, h]], np.arange(got.shape[-1]))
        assert (inv[0, h] >= 0).sum() == got.shape[-1]


def test_check_indices(pkg, dev):
    N = pkg._native
    n, hi = 64, 100
    base = torch.stack([torch.randperm(hi)[:n] for _ in range(6)]).view(1, 6, n).int().to(dev)
    N.check_indices(base, 0, hi)                          # valid: passes
    bad = base.clone()
    bad[0, 3, 7] = hi + 5
    with pytest.raises(IndexError, match="outside"):
        N.check_indices(bad, 0, hi)
    neg = base.clone()
    neg[0, 1, 0] = -2
    with pytest.raises(IndexError, match="outside"):
        N.check_indices(neg, 0, hi)
    dup = base.clone()
    dup[0, 2, 5] = dup[0, 2, 9]
    dup[0, 4, 1] = dup[0, 4, 2] = dup[0, 4, 3]
    with pytest.raises(IndexError, match="3 duplicate"):
        N.check_indices(dup, 0, hi)
    N.check_indices(dup, 0, hi, unique=False)            # range only: passes
    empty = base.clone()
    empty[0, 0, :10] = -1                                 # empty slots (lo = -1) are not duplicates
    N.check_indices(empty, -1, hi)


def test_check_mode_refuses_out_of_range_attention_rows(pkg, dev):
    """With the check mode on, an index past the pooled rows raises before the
    attention kernel is launched (the kernel itself reads rows unguarded)."""
    N = pkg._native
    B, S, H, D, L, p, k = 1, 2048, 2, 128, 3, 4, 128
    xs = [torch.randn(B, S, H, D, device=dev).bfloat16() for _ in range(3)]
    pq, pk, pv, sqk, skq = N.pyramid_fwd(*xs, L, p)
    idx, _ = N.select_topk(sqk, skq, S, L, p, k)
    limit = S + pq.shape[1]
    bad = idx.clone()
    bad[0, 1, -1] = limit                                 # one row past the end
    with pytest.raises(IndexError):                       # the check itself must fire first
        N.check_indices(bad, 0, limit, unique=False)
    rows = N.Rows(*xs, xs[0].stride()[:3], pq, pk, pv, pq.stride()[:3], split=S, limit=limit)
    prev = N.set_check_indices(True)
    try:
        o, _ = N.attn_fwd(rows, idx, B, H, idx.shape[-1], D)  # valid indices still run
        torch.cuda.synchronize()
        assert torch.isfinite(o.float()).all()
        with pytest.raises(IndexError):
            N.attn_fwd(rows, bad, B, H, idx.shape[-1], D)
    finally:
        N.set_check_indices(prev)


def test_scatter_to_base_sequence_refuses_duplicates(pkg, dev):
    S, L, p, H, D = 1024, 2, 4, 2, 128
    S_tot = S + S // p
    n = 300
    idx = torch.stack([torch.randperm(S_tot)[:n].sort().values for _ in range(H)]).view(1, H, n).int().to(dev)
    attn = torch.randn(1, H, n, D, device=dev).bfloat16()
    out = pkg.scatter_to_base_sequence(attn, idx, None, S, S, L, p)
    assert out.shape == (1, H, S, D)
    with_empty = idx.clone()
    with_empty[0, 0, 5] = -1                              # an empty slot: skipped, as in the reference
    out2 = pkg.scatter_to_base_sequence(attn, with_empty, None, S, S, L, p)
    torch.cuda.synchronize()
    assert torch.isfinite(out2.float()).all()
    dup = idx.clone()
    dup[0, 1, 10] = dup[0, 1, 11]
    with pytest.raises(IndexError, match="duplicate"):
        pkg.scatter_to_base_sequence(attn, dup, None, S, S, L, p)


def test_rmsnorm_and_swiglu_on_non_contiguous_inputs(pkg, dev):
    """A transposed input: the backward reads the same contiguous rows the forward
    normalised (gradients against torch autograd in fp32)."""
    ops = pkg.block_ops
    g = torch.Generator(device=dev).manual_seed(0)
    base = torch.randn(512, 3, 1024, device=dev, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(1024, device=dev, generator=g)).bfloat16()
    x = base.transpose(0, 1).requires_grad_()            # [3, 512, 1024], not contiguous
    wp = w.clone().requires_grad_()
    y = ops.rms_norm(x, wp, 1e-5)
    dy = torch.randn(y.shape, device=dev, generator=g).bfloat16()
    y.backward(dy)
    xr = base.transpose(0, 1).float().requires_grad_()
    wr = w.float().requires_grad_()
    yr = torch.nn.functional.rms_norm(xr, (1024,), wr, 1e-5)
    yr.backward(dy.float())
    assert_close(y, yr, "rmsnorm y")
    assert_close(x.grad, xr.grad, "rmsnorm dx")
    assert_close(wp.grad, wr.grad, "rmsnorm dw")
    h0 = torch.randn(256, 4, 2 * 768, device=dev, generator=g).bfloat16()
    h = h0.transpose(0, 1).requires_grad_()
    a = ops.swiglu(h)
    da = torch.randn(a.shape, device=dev, generator=g).bfloat16()
    a.backward(da)
    hr = h0.transpose(0, 1).float().requires_grad_()
    ar = torch.nn.functional.silu(hr[..., :768]) * hr[..., 768:]
    ar.backward(da.float())
    assert_close(a, ar, "swiglu a")
    assert_close(h.grad, hr.grad, "swiglu dh")
