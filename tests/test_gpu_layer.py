"""GPU parity of the whole Lighthouse layer (forward + backward) against the oracle.

Reference: LighthouseLocal.forward (src/lighthouse_selection.py:789-825) and the
autograd of its backward.  Selection is checked bit-exact on the device's own
scores; outputs and gradients are checked against the fp32 oracle on that
same index set (a 1-ulp difference in a bf16 norm could flip a tie and change
the set, so both sides share it).
"""
import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import lh_oracle as O
from oracle import select_ref as R

pytestmark = pytest.mark.gpu


def _inputs(B, S, H, seed, dev):
    g = torch.Generator().manual_seed(seed)
    cpu = [torch.randn(B, S, H, 128, generator=g).bfloat16() for _ in range(3)]
    dout = torch.randn(B, H, S, 128, generator=g).bfloat16()
    return cpu, [c.to(dev).requires_grad_() for c in cpu], dout


def _check_layer(pkg, dev, B, S, H, L, p, k, dilation=0, strict=True, tie="reference", seed=0):
    print(f"layer B={B} S={S} H={H} L={L} p={p} k={k} dil={dilation} strict={strict} tie={tie}", flush=True)
    cpu, xs, dout = _inputs(B, S, H, seed, dev)
    out, idx = pkg.lighthouse_layer(*xs, num_levels=L, pooling_factor=p, topk=k, tie_break=tie,
                                    strict=strict, dilation=dilation)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    # selection is bit-exact on the scores this device computed
    with torch.no_grad():
        _, _, S_tot = pkg._native.pyramid_lengths(S, L, p)
        if dilation:
            sc = pkg._native.dilated_scores(*[x.detach() for x in xs], dilation, S_tot)
            _, _, _, sqk, skq = pkg._native.pyramid_fwd(*[x.detach() for x in xs], L, p, scores=sc)
        else:
            _, _, _, sqk, skq = pkg._native.pyramid_fwd(*[x.detach() for x in xs], L, p)
    g = O.tile_geometry(S, L, p, k)
    ref_idx = R.select_indices_c(sqk.cpu().numpy(), skq.cpu().numpy(), L, p, k, S, g.S_sel, tie=tie,
                                 strict=strict)
    assert np.array_equal(idx.cpu().numpy(), ref_idx), "selected indices differ"
    # fp32 oracle on the same index set
    xc = [c.float().requires_grad_() for c in cpu]
    ref_out, _ = O.lighthouse_layer(*xc, L, p, k, scorer="dilated" if dilation else "norm",
                                    dilation=dilation or 4, indices=ref_idx, strict=strict)
    ref_out.backward(dout.float())
    assert_close(out, ref_out, "layer out")
    for n, x, c in zip("qkv", xs, xc):
        assert_close(x.grad, c.grad, f"d{n}")


def test_layer_small_strict(pkg, dev):
    _check_layer(pkg, dev, 1, 4096, 2, 3, 4, 256)


def test_layer_two_levels_batch2(pkg, dev):
    _check_layer(pkg, dev, 2, 2048, 2, 2, 2, 128, seed=1)


def test_layer_lower_index(pkg, dev):
    _check_layer(pkg, dev, 1, 4096, 1, 3, 4, 256, tie="lower_index", seed=2)


def test_layer_generalized_cfg1_shape(pkg, dev):
    """cfg1 geometry (S=4096, k=1536), outside the reference's domain: per-tile compaction."""
    _check_layer(pkg, dev, 1, 4096, 2, 3, 4, 1536, strict=False, seed=3)


def test_layer_dilated(pkg, dev):
    _check_layer(pkg, dev, 1, 4096, 2, 3, 4, 256, dilation=4, seed=4)


def test_local_module_api(pkg, dev):
    """LighthouseLocal built the way the reference model wiring builds it
    (lighthouse-attention.patch:675-681), plus the reference-shaped scorer path."""
    S, H, L, p, k = 2048, 2, 3, 4, 128
    cpu, xs, dout = _inputs(1, S, H, 7, dev)
    scorer = pkg.DialatedLighthouseNormScorer(pooling_factor=p, levels=L)
    layer = pkg.LighthouseLocal(scorer=scorer, num_levels=L, pooling_factor=p, topk=k, attention=None)
    out = layer(*xs)
    assert out.shape == (1, H, S, 128) and out.dtype == torch.bfloat16
    out.backward(dout.to(dev))
    grads = [x.grad.clone() for x in xs]
    # generic composition through the scorer's 5-tuple must give the same result
    xs2 = [c.to(dev).requires_grad_() for c in cpu]
    sqk, skq, qc, kc, vc = scorer(*xs2)
    assert sqk.shape == (1, H, S + S // 4 + S // 16) and sqk.dtype == torch.bfloat16
    assert qc.shape == (1, H, S + S // 4 + S // 16, 128)
    idx = pkg.LighthouseSelectionQkKqChunkedTopkNvrtc.forward(sqk.float(), skq.float(), L, p, k, S)
    assert torch.equal(idx, layer.last_indices)
    attn = pkg.lighthouse_selection._GatheredAttnFn.apply(qc, kc, vc, idx)
    out2 = pkg.scatter_to_base_sequence(attn, idx, torch.zeros_like(idx), S, S, L, p)
    assert_close(out2, out.float(), "generic path out", max_abs=1e-2, rel_l2=2e-3)
    out2.backward(dout.to(dev))
    for n, g1, x in zip("qkv", grads, xs2):
        assert_close(x.grad, g1.float(), f"generic path d{n}", max_abs=1e-2, rel_l2=4e-3)


def test_layer_backward_two_streams(pkg, dev):
    """set_backward_streams(2) runs the dQ kernel on a side stream beside the
    dK/dV kernel: the same kernels on the same inputs, so the gradients must be
    bit-equal to the one-stream order."""
    S, H, L, p, k = 4096, 8, 3, 4, 256
    cpu, _, dout = _inputs(1, S, H, 11, dev)
    grads = []
    for streams in (1, 2):
        prev = pkg.lighthouse_selection.set_backward_streams(streams)
        try:
            xs = [c.to(dev).requires_grad_() for c in cpu]
            out, _ = pkg.lighthouse_layer(*xs, num_levels=L, pooling_factor=p, topk=k)
            out.backward(dout.to(dev))
            torch.cuda.synchronize()
            grads.append([x.grad.clone() for x in xs])
        finally:
            pkg.lighthouse_selection.set_backward_streams(prev)
    for n, g1, g2 in zip("qkv", *grads):
        assert torch.equal(g1, g2), f"d{n} differs between one and two backward streams"
