"""Benchmark config 5 at its own size: the 270M Llama3 Lighthouse model
(``ablation_270m_lighthouse_topk1536_pool4_lvl3``, lighthouse-attention.patch:283-296),
B=1, S=32768, byte vocabulary.

- the fused rotary Lighthouse layer its norm-scorer layers run
  (lighthouse-attention.patch:707-712 -> src/lighthouse_selection.py:772-825) at
  S=32768, H=8, k=1536, L=3, p=4 (generalized geometry): indices bit-exact against
  the slot-literal C restatement on the device's scores, and equal to rotating first
  and running the plain layer (whose outputs and gradients are checked against the
  fp32 oracle at this size in test_gpu_configs.py, case cfg5_layer);
- one full training step (forward, backward, clip, AdamW): finite loss near
  ln(256) at initialisation, finite gradient norm, and one Lighthouse layer's
  indices bit-exact against the C restatement on that layer's own inputs.
"""
import dataclasses
import math

import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import select_ref as R

pytestmark = pytest.mark.gpu

S, H, D, L, P, K = 32768, 8, 128, 3, 4, 1536


def _ref_indices(pkg, xqkv, fr):
    N = pkg._native
    with torch.no_grad():
        _, _, _, _, sqk, skq = N.rope_pyramid_fwd(xqkv, fr, H, L, P)
    n = N.geometry(S, L, P, K, False)[3]
    return R.select_indices_c(sqk.cpu().numpy(), skq.cpu().numpy(), L, P, K, S, n, strict=False)


def test_cfg5_rope_layer_full_size(pkg, dev):
    ops = pkg.block_ops
    print(f"cfg5 rope layer S={S} H={H} k={K} L={L} p={P}", flush=True)
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(1, S, 3 * H * D, device=dev, generator=g).bfloat16()
    fc = pkg.llama3.precompute_freqs_cis(D, S, 10000.0)
    fr = torch.view_as_real(fc).contiguous().to(dev)
    x1 = x.clone().requires_grad_()
    out, idx = pkg.lighthouse_layer_rope(x1, fr, H, L, P, K, strict=False, seq_major=True)
    x2 = x.clone().requires_grad_()
    q, k, v = ops.rope_qkv(x2, fr, H, H, D)
    out2, idx2 = pkg.lighthouse_layer(q, k, v, L, P, K, strict=False, seq_major=True)
    ref = _ref_indices(pkg, x, fr)
    got = idx.cpu().numpy()
    assert np.array_equal(got, ref), f"{(got != ref).sum()} of {ref.size} indices differ"
    assert torch.equal(idx, idx2)
    assert torch.equal(out, out2)
    do = torch.randn(out.shape, device=dev, generator=g).bfloat16()
    out.backward(do)
    out2.backward(do)
    assert_close(x1.grad, x2.grad.float(), "cfg5 d xqkv", max_abs=1e-2, rel_l2=4e-3)
    assert torch.equal(x1.grad[..., 2 * H * D:], x2.grad[..., 2 * H * D:])


def test_cfg5_training_step(pkg, dev):
    L3 = pkg.llama3
    margs = dataclasses.replace(L3.llama3_args["ablation_270m_lighthouse_topk1536_pool4_lvl3"], vocab_size=256,
                                lighthouse_strict=False)
    margs.update_from_config(seq_len=S)
    print(f"cfg5 training step: {margs.n_layers} layers, dim {margs.dim}, S={S}", flush=True)
    trainer = L3.Trainer(margs, dev, seed=0)
    layer = trainer.model.layers["5"].attention
    assert layer._use_lighthouse and layer._fuses_rope()
    light = sum(1 for b in trainer.model.layers.values() if b.attention._use_lighthouse)
    assert light == 26
    captured = {}
    orig = layer.selection_attn.forward_rope

    def spy(xqkv, freqs, n_heads):
        captured["x"], captured["f"] = xqkv.detach().clone(), freqs
        return orig(xqkv, freqs, n_heads)

    layer.selection_attn.forward_rope = spy
    g = torch.Generator(device=dev).manual_seed(1234)
    tok = torch.randint(0, 256, (1, S + 1), device=dev, generator=g)
    x, y = tok[:, :-1].contiguous(), tok[:, 1:].contiguous()
    loss = trainer.step(x, y).item()
    gn = trainer.last_grad_norm.item()
    idx = layer.selection_attn.last_indices.cpu().numpy()
    print(f"loss {loss:.4f} grad-norm {gn:.4f}", flush=True)
    assert math.isfinite(loss) and math.isfinite(gn) and gn > 0
    assert abs(loss - math.log(256)) < 1.0, loss
    for prm in trainer.master.parameters():
        assert torch.isfinite(prm).all()
    ref = _ref_indices(pkg, captured["x"], captured["f"])
    assert np.array_equal(idx, ref), f"{(idx != ref).sum()} of {ref.size} indices differ"
