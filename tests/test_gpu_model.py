"""GPU checks of the dense causal layers and the Llama3 model built on the native kernels.

dense attention <- torchtitan ScaledDotProductAttentionWrapper, causal (lighthouse-attention.patch:707-724)
model wiring    <- Attention / TransformerBlock / Transformer (lighthouse-attention.patch:583-769)
training step   <- configs/scorer/norm.toml:25-49 (AdamW, max_norm)
"""
import copy

import pytest
import torch
import torch.nn as nn

from conftest import assert_close
from oracle import lh_oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,S,H", [(2, 777, 3), (1, 2048, 2), (1, 64, 1)])
def test_dense_causal_module(pkg, dev, B, S, H):
    """[B, H, S, D] transposed views of [B, S, H, D] buffers, read in place."""
    print(f"dense module B={B} S={S} H={H}", flush=True)
    g = torch.Generator().manual_seed(S + H)
    base = [torch.randn(B, S, H, 128, generator=g).bfloat16() for _ in range(3)]
    xs = [b.to(dev).transpose(1, 2).requires_grad_() for b in base]
    out = pkg.dense_attention.dense_causal_attention(*xs)
    assert out.shape == (B, H, S, 128) and out.dtype == torch.bfloat16
    refs = [b.float().transpose(1, 2).clone().requires_grad_() for b in base]
    ref = O.sdpa_causal(*refs)
    assert_close(out, ref, "dense out")
    do = torch.randn(B, H, S, 128, generator=g).bfloat16()
    out.backward(do.to(dev))
    ref.backward(do.float())
    for x, r, name in zip(xs, refs, ("dq", "dk", "dv")):
        assert_close(x.grad, r.grad, name)


class _Fp32Attention(nn.Module):
    """Causal attention in fp32 on the GPU (torch ops), result rounded to the input dtype."""

    def forward(self, q, k, v):
        return O.sdpa_causal(q.float(), k.float(), v.float()).to(q.dtype)


def _tiny(pkg, **kw):
    base = dict(dim=256, n_layers=3, n_heads=2, n_kv_heads=2, vocab_size=256, hidden_dim=768, max_seq_len=4096,
                use_selection_lighthouse=False)
    base.update(kw)
    return pkg.llama3.TransformerModelArgs(**base)


def test_model_dense_layers_against_fp32_attention(pkg, dev):
    """Same bf16 model twice: native dense attention vs fp32 torch attention.  The
    difference comes only from the attention kernels; logits rel-L2 <= 1e-2 and
    every parameter gradient rel-L2 <= 3e-2."""
    L = pkg.llama3
    torch.manual_seed(0)
    with torch.device(dev):
        m = L.Transformer(_tiny(pkg))
    m.init_weights(dev)
    L.cast_params_(m, torch.bfloat16)
    ref = copy.deepcopy(m)
    for b in ref.layers.values():
        b.attention.inner_attention = _Fp32Attention()
    tok = torch.randint(0, 256, (2, 1000), device=dev, generator=torch.Generator(dev).manual_seed(1))
    out = m(tok)
    out_r = ref(tok)
    assert_close(out, out_r.float(), "logits", max_abs=5e-2, rel_l2=1e-2)
    lbl = tok.roll(-1, 1)
    torch.nn.functional.cross_entropy(out.flatten(0, 1).float(), lbl.flatten()).backward()
    torch.nn.functional.cross_entropy(out_r.flatten(0, 1).float(), lbl.flatten()).backward()
    for (name, p), pr in zip(m.named_parameters(), ref.parameters()):
        assert_close(p.grad, pr.grad.float(), name, max_abs=1e-1, rel_l2=3e-2)


def _torch_forward(m, tok):
    """torchtitan's Llama3 forward restated with torch ops in fp32 on the model's
    (bf16-valued) weights; causal attention from the oracle."""
    a = m.model_args
    P = {k: v.float() for k, v in m.state_dict().items() if k != "freqs_cis"}
    import importlib
    L = importlib.import_module(type(m).__module__)
    h = P["tok_embeddings.weight"][tok]
    S = tok.shape[1]
    hd = a.dim // a.n_heads
    for i in range(a.n_layers):
        p = f"layers.{i}."
        xn = torch.nn.functional.rms_norm(h, (a.dim,), P[p + "attention_norm.weight"], a.norm_eps)
        q = (xn @ P[p + "attention.wq.weight"].t()).view(*tok.shape, -1, hd)
        k = (xn @ P[p + "attention.wk.weight"].t()).view(*tok.shape, -1, hd)
        v = (xn @ P[p + "attention.wv.weight"].t()).view(*tok.shape, -1, hd)
        q, k = L.apply_rotary_emb(q, k, m.freqs_cis)
        o = O.sdpa_causal(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
        h = h + o.transpose(1, 2).reshape(*tok.shape, -1) @ P[p + "attention.wo.weight"].t()
        xn = torch.nn.functional.rms_norm(h, (a.dim,), P[p + "ffn_norm.weight"], a.norm_eps)
        f = torch.nn.functional.silu(xn @ P[p + "feed_forward.w1.weight"].t()) * (xn @ P[p + "feed_forward.w3.weight"].t())
        h = h + f @ P[p + "feed_forward.w2.weight"].t()
    h = torch.nn.functional.rms_norm(h, (a.dim,), P["norm.weight"], a.norm_eps)
    return h @ P["output.weight"].t()


def test_model_against_torch_restatement(pkg, dev):
    """Whole dense model (native RMSNorm, fused projections, RoPE, SwiGLU, attention)
    against the fp32 torch restatement on the same bf16 weights: logits rel-L2 <= 2e-2,
    loss within 1e-2."""
    L = pkg.llama3
    torch.manual_seed(3)
    with torch.device(dev):
        m = L.Transformer(_tiny(pkg, n_layers=2))
    m.init_weights(dev)
    L.cast_params_(m, torch.bfloat16)
    tok = torch.randint(0, 256, (1, 1536), device=dev, generator=torch.Generator(dev).manual_seed(4))
    with torch.no_grad():
        out = m(tok).float()
        ref = _torch_forward(m, tok)
    assert_close(out, ref, "logits", max_abs=5e-2, rel_l2=2e-2)
    lbl = tok.roll(-1, 1).flatten()
    l1 = torch.nn.functional.cross_entropy(out.flatten(0, 1), lbl).item()
    l2 = torch.nn.functional.cross_entropy(ref.flatten(0, 1), lbl).item()
    assert abs(l1 - l2) < 1e-2, (l1, l2)


def test_lighthouse_layer_wiring_is_exact(pkg, dev):
    """A Lighthouse layer of the model computes wo(lighthouse_layer(rope(wq x), rope(wk x), wv x))."""
    L, ops = pkg.llama3, pkg.block_ops
    args = _tiny(pkg, use_selection_lighthouse=True, lighthouse_num_levels=2, lighthouse_pooling_factor=4,
                 lighthouse_topk=256, lighthouse_full_attn_layers=[0, 2])
    torch.manual_seed(1)
    with torch.device(dev):
        m = L.Transformer(args)
    m.init_weights(dev)
    L.cast_params_(m, torch.bfloat16)
    att = m.layers["1"].attention
    S = 2048
    x = torch.randn(1, S, 256, device=dev, generator=torch.Generator(dev).manual_seed(2)).bfloat16()
    fr = torch.view_as_real(m.freqs_cis)

    def qkv(a):
        # separate projections equal the fused one's column blocks; rope as torchtitan's op
        q, k, v = a.wq(x).view(1, S, 2, 128), a.wk(x).view(1, S, 2, 128), a.wv(x).view(1, S, 2, 128)
        fq, fk, fv = ops.rope_qkv(ops.linear(x, torch.cat([a.wq.weight, a.wk.weight, a.wv.weight])), fr, 2, 2, 128)
        rq, rk = L.apply_rotary_emb(q, k, m.freqs_cis)
        assert_close(fv, v, "v split", max_abs=1e-2, rel_l2=5e-3)
        assert_close(fq, rq, "rotated q", max_abs=1e-2, rel_l2=5e-3)
        assert_close(fk, rk, "rotated k", max_abs=1e-2, rel_l2=5e-3)
        return fq, fk, fv

    with torch.no_grad():
        got = att(x, m.freqs_cis)
        q, k, v = qkv(att)
        o, _ = pkg.lighthouse_layer(q, k, v, 2, 4, 256)
        want = ops.linear(o.transpose(1, 2).reshape(1, S, 256), att.wo.weight)
    assert torch.equal(got, want)
    # the full-attention layers of the same model take the dense kernel
    with torch.no_grad():
        a0 = m.layers["0"].attention
        got0 = a0(x, m.freqs_cis)
        q, k, v = qkv(a0)
        o = pkg.dense_attention.dense_causal_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
        want0 = ops.linear(o.transpose(1, 2).reshape(1, S, 256), a0.wo.weight)
    assert torch.equal(got0, want0)


def test_trainer_learns_a_sequence(pkg, dev):
    """Ten mixed-precision steps on one batch of a mostly deterministic sequence
    (next token = perm[token] with probability 0.9): the loss falls below half."""
    L = pkg.llama3
    args = _tiny(pkg, n_layers=4, use_selection_lighthouse=True, lighthouse_num_levels=2,
                 lighthouse_pooling_factor=4, lighthouse_topk=256, lighthouse_full_attn_layers=[0, 3])
    T = L.Trainer(args, dev, lr=2e-3, warmup_steps=0, seed=0)
    g = torch.Generator().manual_seed(0)
    perm = torch.randperm(256, generator=g)
    S = 2048
    tok = torch.empty(S + 1, dtype=torch.long)
    tok[0] = 3
    noise = torch.rand(S, generator=g) < 0.1
    rnd = torch.randint(0, 256, (S,), generator=g)
    for t in range(1, S + 1):
        tok[t] = rnd[t - 1] if noise[t - 1] else perm[tok[t - 1]]
    x, y = tok[None, :-1].to(dev), tok[None, 1:].to(dev)
    losses = []
    for i in range(10):
        losses.append(T.step(x, y).item())
        print(f"step {i} loss {losses[-1]:.4f} grad-norm {T.last_grad_norm.item():.3f}", flush=True)
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < 0.5 * losses[0], losses
    # the bf16 compute copy is the masters rounded once
    T.step(x, y)
    for mp, bp in zip(T.master.parameters(), T.model.parameters()):
        assert bp.dtype == torch.bfloat16 and mp.dtype == torch.float32
    assert T.model.freqs_cis.is_complex()
