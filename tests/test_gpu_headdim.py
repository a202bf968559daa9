"""Head dims below 128 (the patch's ablation_270m flavor has 72, ablation_2b 64;
lighthouse-attention.patch:78-89,514-526; the reference path takes any D through
BLOCK_D = next_power_of_2(D), src/lighthouse_selection.py:532,566).

The kernels move 128-wide rows; a D-wide head runs zero-padded with the softmax
scale 1/sqrt(D).  Checked against the fp32 oracle at the original width:
selection bit-exact on the device's scores, outputs and gradients within the
bf16 tolerance."""
import dataclasses

import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import lh_oracle as O
from oracle import select_ref as R

pytestmark = pytest.mark.gpu


def _xs(B, S, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, S, H, D, generator=g).bfloat16() for _ in range(3)]


@pytest.mark.parametrize("D,scorer", [(64, "norm"), (72, "norm"), (64, "dilated"), (72, "gla")])
def test_layer_small_head_dim(pkg, dev, D, scorer):
    N = pkg._native
    B, S, H, L, p, k, dil = 1, 4096, 2, 3, 4, 256, 4
    print(f"layer D={D} scorer={scorer}", flush=True)
    xs = _xs(B, S, H, D, D)
    gk = (torch.nn.functional.logsigmoid(torch.randn(B, S, H, generator=torch.Generator().manual_seed(3))) / 16
          ).bfloat16() if scorer == "gla" else None
    xg = [x.to(dev).requires_grad_() for x in xs]
    out, idx = pkg.lighthouse_layer(*xg, L, p, k, dilation=dil if scorer != "norm" else 0,
                                    gk=gk.to(dev) if gk is not None else None)
    assert out.shape == (B, H, S, D)
    do = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(4)).bfloat16()
    out.backward(do.to(dev))
    # scores of the zero-padded rows are the D-wide rows' scores: selection bit-exact on them
    pad = [torch.nn.functional.pad(x.to(dev), (0, 128 - D)) for x in xs]
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    if scorer == "norm":
        _, _, _, sqk, skq = N.pyramid_fwd(*pad, L, p)
    elif scorer == "dilated":
        _, _, _, sqk, skq = N.pyramid_fwd(*pad, L, p, scores=N.dilated_scores(*pad, dil, S_tot, D ** -0.5))
    else:
        _, _, _, sqk, skq = N.pyramid_fwd(*pad, L, p, scores=N.gla_scores(*pad, gk.to(dev), dil, S_tot, D ** -0.5))
    ref_idx = R.select_indices_c(sqk.cpu().numpy(), skq.cpu().numpy(), L, p, k, S, idx.shape[-1])
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    if scorer == "norm":  # the norm scores do not depend on the padding: the oracle's own selection agrees
        r_qk, r_kq, *_ = O.norm_scorer(*[x.float() for x in xs], p, L)
        assert_close(sqk, r_qk, "norm scores", max_abs=1e-2, rel_l2=5e-3)
    xc = [x.float().requires_grad_() for x in xs]
    ref, _ = O.lighthouse_layer(*xc, L, p, k, scorer="norm", indices=ref_idx)
    ref.backward(do.float())
    assert_close(out, ref, f"D={D} out")
    for n_, x, c in zip("qkv", xg, xc):
        assert_close(x.grad, c.grad, f"D={D} d{n_}")


def test_dense_attention_small_head_dim(pkg, dev):
    B, S, H, D = 1, 1500, 3, 72
    base = _xs(B, S, H, D, 9)
    xs = [b.to(dev).transpose(1, 2).requires_grad_() for b in base]
    out = pkg.dense_attention.dense_causal_attention(*xs)
    assert out.shape == (B, H, S, D)
    refs = [b.float().transpose(1, 2).clone().requires_grad_() for b in base]
    ref = O.sdpa_causal(*refs)
    assert_close(out, ref, "dense D=72 out")
    do = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(1)).bfloat16()
    out.backward(do.to(dev))
    ref.backward(do.float())
    for x, r, n_ in zip(xs, refs, ("dq", "dk", "dv")):
        assert_close(x.grad, r.grad, f"dense D=72 {n_}")


def test_generic_composition_small_head_dim(pkg, dev):
    """LighthouseLocal with an attention from elsewhere (use_native_attention=False):
    the scorer's 5-tuple, the gather and scatter_to_base_sequence at D = 64."""
    B, S, H, D, L, p, k = 1, 2048, 2, 64, 3, 4, 128

    class Fp32Attn(torch.nn.Module):
        def forward(self, q, k_, v):
            return O.sdpa_causal(q.float(), k_.float(), v.float()).to(q.dtype)

    scorer = pkg.DialatedLighthouseNormScorer(pooling_factor=p, levels=L)
    layer = pkg.LighthouseLocal(attention=Fp32Attn(), scorer=scorer, num_levels=L, pooling_factor=p, topk=k,
                                use_native_attention=False)
    xs = _xs(B, S, H, D, 21)
    xg = [x.to(dev).requires_grad_() for x in xs]
    out = layer(*xg)
    do = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(5)).bfloat16()
    out.backward(do.to(dev))
    idx = layer.last_indices.cpu().numpy()
    xc = [x.float().requires_grad_() for x in xs]
    ref, ridx = O.lighthouse_layer(*xc, L, p, k, indices=idx)
    ref.backward(do.float())
    assert_close(out, ref, "generic D=64 out")
    for n_, x, c in zip("qkv", xg, xc):
        assert_close(x.grad, c.grad, f"generic D=64 d{n_}")


@pytest.mark.parametrize("flavor,dim", [("ablation_270m", None), ("ablation_2b", None),
                                        ("ablation_270m_lighthouse_topk1536_pool4_lvl3", 576)])
def test_ablation_flavor_head_dims_train(pkg, dev, flavor, dim):
    """The flavors whose heads are not 128 wide (ablation_270m: 72, dense attention;
    ablation_2b: 64, dense) and the 270M Lighthouse flavor at ablation_270m's width
    (heads of 72 through the Lighthouse layers) run a training step, shortened to 3
    layers at S = 4096."""
    L3 = pkg.llama3
    base = L3.llama3_args[flavor]
    if dim:
        base = dataclasses.replace(base, dim=dim)
    args = dataclasses.replace(base, n_layers=3, vocab_size=256, lighthouse_strict=False,
                               lighthouse_full_attn_layers=[0])
    args.update_from_config(seq_len=4096)
    hd = args.dim // args.n_heads
    print(f"{flavor}: dim {args.dim}, {args.n_heads} heads of {hd}, lighthouse={args.use_selection_lighthouse}",
          flush=True)
    assert hd < 128
    T = L3.Trainer(args, dev, seed=0, warmup_steps=0)
    tok = torch.randint(0, 256, (1, 4097), device=dev, generator=torch.Generator(dev).manual_seed(0))
    loss = T.step(tok[:, :-1].contiguous(), tok[:, 1:].contiguous())
    assert torch.isfinite(loss) and torch.isfinite(T.last_grad_norm)
