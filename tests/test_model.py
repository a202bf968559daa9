"""CPU checks of the Llama3 model wiring (no kernels run).

The model restates torchtitan's Llama3 with the Lighthouse patch
(lighthouse-attention.patch:551-769).  torchtitan is not vendored with the
reference, so its unchanged parts are pinned here by what published numbers
and mathematics fix: the FFN width rule against the published Llama-3 widths,
RoPE against the closed-form rotation and its invariants, the frequency
scaling against its regime boundaries, parameter counts against the closed
form.
"""
import dataclasses
import math

import pytest
import torch


@pytest.fixture(scope="module")
def L(pkg):
    return pkg.llama3


def test_ffn_width_rule_matches_published_llama3_widths(L):
    # upstream flavors: (dim, ffn_dim_multiplier, multiple_of) -> published intermediate size
    assert L.ffn_hidden_dim(4 * 4096, 1024, 1.3) == 14336   # Llama-3 8B
    assert L.ffn_hidden_dim(4 * 8192, 4096, 1.3) == 28672   # Llama-3 70B
    assert L.ffn_hidden_dim(4 * 16384, 4096, 1.2) == 53248  # Llama-3.1 405B
    # the patch's explicit hidden_dim goes through the same rule
    assert L.ffn_hidden_dim(1536, 256, None) == 1024
    assert L.ffn_hidden_dim(14336, 256, None) == 9728


def test_flavors(L):
    a = L.llama3_args["ablation_270m_lighthouse_topk1536_pool4_lvl3"]
    assert (a.dim, a.n_layers, a.n_heads, a.n_kv_heads, a.hidden_dim, a.rope_theta) == (1024, 30, 8, 8, 1536, 10000)
    assert (a.lighthouse_num_levels, a.lighthouse_pooling_factor, a.lighthouse_topk) == (3, 4, 1536)
    assert a.use_selection_lighthouse and not a.use_lighthouse_cp
    assert a.lighthouse_full_attn_layers == [0, 1, 28, 29] and a.lighthouse_scorer == "norm"
    cfg2 = L.llama3_args["ablation_270m_lighthouse_topk2048_pool4_lvl3"]
    assert (cfg2.lighthouse_num_levels, cfg2.lighthouse_pooling_factor, cfg2.lighthouse_topk) == (3, 4, 2048)
    assert not L.llama3_args["ablation_270m_topk1536_pool4_lvl3_sdpa"].use_selection_lighthouse
    assert L.llama3_args["ablation_270m_lighthouse_topk4096_pool4_lvl4_cp_1m"].lighthouse_full_attn_layers == []
    assert sum(a.use_lighthouse_cp for a in L.llama3_args.values()) == 6
    # flavors do not share mutable lists
    assert a.lighthouse_full_attn_layers is not cfg2.lighthouse_full_attn_layers


def _small(L, **kw):
    base = dict(dim=256, n_layers=4, n_heads=2, n_kv_heads=2, vocab_size=256, hidden_dim=768, rope_theta=10000,
                max_seq_len=4096, use_selection_lighthouse=True, lighthouse_num_levels=2,
                lighthouse_pooling_factor=4, lighthouse_topk=256, lighthouse_full_attn_layers=[0, 3])
    base.update(kw)
    return L.TransformerModelArgs(**base)


def test_full_attention_layers_switch_off_lighthouse(L):
    m = L.Transformer(_small(L))
    use = {k: (b.attention.use_selection_lighthouse and b.attention._use_lighthouse) for k, b in m.layers.items()}
    assert use == {"0": False, "1": True, "2": True, "3": False}
    assert m._full_attn_layers == {"0", "3"}
    sel = m.layers["1"].attention.selection_attn
    assert (sel.num_levels, sel.pooling_factor, sel.topk) == (2, 4, 256)
    assert type(sel.scorer).__name__ == "DialatedLighthouseNormScorer"
    m2 = L.Transformer(_small(L, lighthouse_scorer="dilated", dilation=4))
    assert m2.layers["1"].attention.selection_attn.scorer.dilation == 4
    with pytest.raises(ValueError):
        L.Transformer(_small(L, lighthouse_scorer="bogus"))
    with pytest.raises(ValueError):
        L.Transformer(_small(L, lighthouse_scorer="dilated", use_lighthouse_cp=True))


def test_param_count_closed_form(L):
    a = dataclasses.replace(L.llama3_args["ablation_270m_lighthouse_topk1536_pool4_lvl3"], vocab_size=256,
                            max_seq_len=64)
    m = L.Transformer(a)
    d, h, V, n = a.dim, L.ffn_hidden_dim(a.hidden_dim, a.multiple_of, None), a.vocab_size, a.n_layers
    per_layer = 4 * d * d + 3 * d * h + 2 * d
    assert L.num_params(m) == n * per_layer + 2 * V * d + d
    assert L.num_params(m) == 220_787_712


def test_rope_matches_closed_form_rotation(L):
    D, S = 128, 64
    sa = L.RoPEScalingArgs(scaling_factor=1.0)  # factor 1: plain RoPE at every wavelength
    fc = L.precompute_freqs_cis(D, S, 10000.0, sa)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, S, 2, D, generator=g, dtype=torch.float64).float()
    q, k = L.apply_rotary_emb(x, x.flip(2), fc)
    t = torch.arange(S, dtype=torch.float64)[:, None]
    f = 10000.0 ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    c, s = torch.cos(t * f)[None, :, None, :], torch.sin(t * f)[None, :, None, :]
    a0, a1 = x[..., 0::2].double(), x[..., 1::2].double()
    ref = torch.stack([a0 * c - a1 * s, a0 * s + a1 * c], dim=-1).flatten(3)
    assert (q.double() - ref).abs().max().item() < 2e-5


def test_rope_invariants(L):
    D, S = 128, 300
    fc = L.precompute_freqs_cis(D, S, 10000.0)
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 1, 1, D, generator=g).expand(1, S, 1, D).contiguous()
    k = torch.randn(1, 1, 1, D, generator=g).expand(1, S, 1, D).contiguous()
    rq, rk = L.apply_rotary_emb(q, k, fc)
    # position 0 is the identity, pair norms are kept
    assert torch.equal(rq[0, 0], q[0, 0])
    pn = lambda x: x.reshape(*x.shape[:-1], -1, 2).norm(dim=-1)
    assert (pn(rq) - pn(q)).abs().max().item() < 1e-5
    # <R(m) q, R(n) k> depends on m - n only
    dots = (rq[0, :, 0, None, :] * rk[0, None, :, 0, :]).sum(-1)  # [m, n]
    for delta in (0, 7, 123):
        diag = torch.diagonal(dots, offset=-delta)
        assert (diag - diag[0]).abs().max().item() < 2e-4 * diag[0].abs().clamp_min(1).item()


def test_rope_frequency_scaling_regimes(L):
    D = 128
    sa = L.RoPEScalingArgs()
    f0 = 1.0 / (10000.0 ** (torch.arange(0, D, 2)[: D // 2].float() / D))
    f = torch.angle(L.precompute_freqs_cis(D, 2, 10000.0, sa)[1]).double()  # angle at t=1 is the frequency
    w = 2 * math.pi / f0.double()
    hi = w < sa.original_max_position_embeddings / sa.high_freq_factor
    lo = w > sa.original_max_position_embeddings / sa.low_freq_factor
    assert hi.any() and lo.any() and (~hi & ~lo).any()
    assert torch.allclose(f[hi], f0[hi].double(), rtol=1e-6)
    assert torch.allclose(f[lo], f0[lo].double() / sa.scaling_factor, rtol=1e-6)
    mid = ~hi & ~lo
    # in between: strictly between the two limits, monotone in wavelength
    assert ((f[mid] < f0[mid].double()) & (f[mid] > f0[mid].double() / sa.scaling_factor)).all()
    assert (f[:-1] > f[1:]).all()


def test_repeat_kv(L):
    x = torch.arange(2 * 3 * 2 * 4).reshape(2, 3, 2, 4)
    r = L.repeat_kv(x, 3)
    assert r.shape == (2, 3, 6, 4)
    for h in range(6):
        assert torch.equal(r[:, :, h], x[:, :, h // 3])


def test_attention_needs_gpu(L):
    # the product path has no CPU fallback
    m = L.Transformer(_small(L, n_layers=1, use_selection_lighthouse=False, lighthouse_full_attn_layers=None))
    L.cast_params_(m, torch.bfloat16)
    assert m.freqs_cis.is_complex()
    with pytest.raises(Exception, match="GPU|no CPU path|liblighthouse"):
        m(torch.zeros(1, 64, dtype=torch.long))


def test_state_dict_matches_dense_flavor_and_gla_adds_the_gate(L):
    """Checkpoint compatibility (the norm and dilated scorers add no
    parameters, so a Lighthouse flavor's state dict equals its dense `_sdpa`
    twin's, lighthouse-attention.patch:303-310; the GLA scorer adds `wg`,
    :662-664)."""
    def keys(**kw):
        m = L.Transformer(_small(L, **kw))
        return {k: tuple(v.shape) for k, v in m.state_dict().items()}
    dense = keys(use_selection_lighthouse=False)
    assert keys() == dense
    assert keys(lighthouse_scorer="dilated", dilation=4) == dense
    gla = keys(lighthouse_scorer="gla", dilation=4)
    extra = {k: v for k, v in gla.items() if k not in dense}
    assert {k: v for k, v in gla.items() if k in dense} == dense
    assert extra == {f"layers.{i}.attention.wg.{n}": ((2, 256) if n == "weight" else (2,))
                     for i in range(4) for n in ("weight", "bias")}


def test_builder_errors_like_reference(L):
    """_build_lighthouse_scorer's ValueErrors (lighthouse-attention.patch:610-615, 635-638)."""
    with pytest.raises(ValueError, match="Unknown lighthouse_scorer"):
        L.Transformer(_small(L, lighthouse_scorer="bogus"))
    for name in ("dilated", "gla"):
        with pytest.raises(ValueError, match="not supported under context parallelism"):
            L.Transformer(_small(L, lighthouse_scorer=name, use_lighthouse_cp=True))
    m = L.Transformer(_small(L, lighthouse_scorer="gla", dilation=2))
    sc = m.layers["1"].attention.selection_attn.scorer
    assert type(sc).__name__ == "DilatedLighthouseGLAScorer" and sc.dilation == 2 and sc.head_dim == 128
