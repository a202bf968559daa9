"""GPU parity of the GLA scorer (DilatedLighthouseGLAScorer, src/lighthouse_selection.py:692-755).

The reference scores with fla's chunk_simple_gla (not importable here); the
oracle restates its published recurrence as a float64 quadratic form, pinned in
tests/test_oracle.py against the token-by-token recurrence, the g = 0 and
g -> -inf closed forms and a per-virtual-head slicing of the dilated view.
Parity against fla's own kernels stays unpinned.

Tolerances: base scores are bf16-rounded norms of bf16-rounded outputs, compared
with the oracle's (same roundings, float64 arithmetic) at max-abs 2e-2 * max and
rel-L2 1e-2; at least 95% of them must be within one bf16 ulp.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import lh_oracle as O
from oracle import select_ref as R

pytestmark = pytest.mark.gpu
D = 128


def _inputs(B, S, H, gate, seed, dev):
    g = torch.Generator().manual_seed(seed)
    xs = [torch.randn(B, S, H, D, generator=g).bfloat16() for _ in range(3)]
    if gate == "typical":   # the patch's gate: logsigmoid(wg(x)) / 16
        gk = torch.nn.functional.logsigmoid(torch.randn(B, S, H, generator=g)) / 16
    elif gate == "strong":  # fast decay
        gk = torch.nn.functional.logsigmoid(torch.randn(B, S, H, generator=g) * 3 - 2)
    else:                   # no decay: plain causal linear attention
        gk = torch.zeros(B, S, H)
    return xs, gk.bfloat16(), [x.to(dev) for x in xs], gk.bfloat16().to(dev)


def _ulps(a, b):
    a, b = a.float(), b.float()
    ulp = torch.pow(2.0, torch.floor(torch.log2(b.abs().clamp_min(1e-30))) - 7)
    return (a - b).abs() / ulp


@pytest.mark.parametrize("B,S,H,dil,gate", [(1, 1024, 2, 4, "typical"), (2, 1000, 1, 4, "strong"),
                                            (1, 4096, 2, 2, "typical"), (1, 2048, 3, 4, "none"),
                                            (1, 256, 1, 1, "strong"), (1, 16384, 1, 4, "typical")])
def test_gla_scores(pkg, dev, B, S, H, dil, gate):
    print(f"gla scores B={B} S={S} H={H} dil={dil} gate={gate}", flush=True)
    N = pkg._native
    L, p = 3, 2
    xs, gk, xd, gd = _inputs(B, S, H, gate, S + H, dev)
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    sqk, skq = N.gla_scores(*xd, gd, dil, S_tot)
    r_qk, r_kq, *_ = O.gla_scorer(*[x.float() for x in xs], gk.float(), dil, p, L, round_bf16=True)
    for got, ref, name in ((sqk, r_qk, "qk"), (skq, r_kq, "kq")):
        got = got[..., :S].cpu()
        ref = ref[..., :S]
        assert_close(got, ref, f"gla scores {name}")
        assert (_ulps(got, ref) <= 1).float().mean().item() >= 0.95, f"{name}: fewer than 95% within 1 ulp"


def _inputs_f16(B, S, H, gate, seed, dev):
    xs, gk, _, _ = _inputs(B, S, H, gate, seed, dev)
    g = torch.Generator().manual_seed(seed)
    xs = [torch.randn(B, S, H, D, generator=g).half() for _ in range(3)]
    return xs, gk, [x.to(dev) for x in xs], gk.to(dev)


def _ulps16(a, b, mant):
    a, b = a.float(), b.float()
    ulp = torch.pow(2.0, torch.floor(torch.log2(b.abs().clamp_min(1e-30))) - mant)
    return (a - b).abs() / ulp


@pytest.mark.parametrize("B,S,H,dil,gate,segs", [(1, 1024, 2, 4, "typical", 0), (2, 1000, 1, 4, "strong", 0),
                                                 (1, 8192, 1, 2, "none", 3), (1, 16384, 1, 4, "typical", 0)])
def test_gla_scores_fp16(pkg, dev, B, S, H, dil, gate, segs):
    """fp16 rows: fp16 MFMAs and an fp16 state copy; outputs and norms rounded to
    fp16, against the float64 oracle with the same roundings (standard tolerance,
    at least 90% within one fp16 ulp)."""
    print(f"gla scores fp16 B={B} S={S} H={H} dil={dil} gate={gate} segments={segs}", flush=True)
    N = pkg._native
    L, p = 3, 2
    xs, gk, xd, gd = _inputs_f16(B, S, H, gate, S + H + 1, dev)
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    sqk, skq = N.gla_scores(*xd, gd, dil, S_tot, segments=segs)
    r_qk, r_kq, *_ = O.gla_scorer(*[x.float() for x in xs], gk.float(), dil, p, L, round_to=torch.float16)
    for got, ref, name in ((sqk, r_qk, "qk"), (skq, r_kq, "kq")):
        got = got[..., :S].cpu()
        ref = ref[..., :S]
        assert torch.equal(got, got.half().float()), f"{name}: scores are not fp16 values"
        assert_close(got, ref, f"gla fp16 scores {name}")
        assert (_ulps16(got, ref, 10) <= 1).float().mean().item() >= 0.90, f"{name}: fewer than 90% within 1 ulp"


def test_gla_layer_fp16(pkg, dev):
    """The layer with the GLA scorer on fp16 rows: indices bit-exact on the
    device's own scores, outputs and gradients (fp16) against the fp32 oracle on
    that index set."""
    N = pkg._native
    B, S, H, L, p, k, dil = 1, 4096, 2, 3, 4, 256, 4
    print(f"gla layer fp16 S={S} H={H} k={k} dil={dil}", flush=True)
    xs, gk, xd, gd = _inputs_f16(B, S, H, "typical", 12, dev)
    xg = [x.clone().requires_grad_() for x in xd]
    out, idx = pkg.lighthouse_layer(*xg, num_levels=L, pooling_factor=p, topk=k, dilation=dil, gk=gd)
    assert out.dtype == torch.float16
    do = torch.randn(out.shape, generator=torch.Generator().manual_seed(3)).half()
    out.backward(do.to(dev))
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    sc = N.gla_scores(*xd, gd, dil, S_tot)
    _, _, _, sqk, skq = N.pyramid_fwd(*xd, L, p, scores=sc)
    ref_idx = R.select_indices_c(sqk.cpu().numpy(), skq.cpu().numpy(), L, p, k, S, idx.shape[-1])
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    xc = [x.float().requires_grad_() for x in xs]
    ref, _ = O.lighthouse_layer(*xc, L, p, k, scorer="gla", dilation=dil, gk=gk.float(), indices=ref_idx)
    ref.backward(do.float())
    assert_close(out, ref, "gla fp16 layer out")
    for n_, x, c in zip("qkv", xg, xc):
        assert x.grad.dtype == torch.float16
        assert_close(x.grad, c.grad, f"gla fp16 layer d{n_}")


def test_gla_layer_against_oracle(pkg, dev):
    """LighthouseLocal with the GLA scorer: selection bit-exact on the device's own
    scores (C restatement), outputs and gradients against the fp32 oracle on that
    index set; the gate receives no gradient."""
    N = pkg._native
    B, S, H, L, p, k, dil = 1, 4096, 2, 3, 4, 256, 4
    print(f"gla layer S={S} H={H} k={k} dil={dil}", flush=True)
    xs, gk, xd, gd = _inputs(B, S, H, "typical", 11, dev)
    scorer = pkg.DilatedLighthouseGLAScorer(head_dim=D, dilation=dil, pooling_factor=p, levels=L)
    layer = pkg.LighthouseLocal(attention=None, scorer=scorer, num_levels=L, pooling_factor=p, topk=k)
    xg = [x.clone().requires_grad_() for x in xd]
    gg = gd.clone().requires_grad_()
    out = layer(*xg, gk=gg)
    do = torch.randn(out.shape, generator=torch.Generator().manual_seed(2)).bfloat16()
    out.backward(do.to(dev))
    assert gg.grad is None
    idx = layer.last_indices.cpu().numpy()
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    sc = N.gla_scores(*xd, gd, dil, S_tot)
    _, _, _, sqk, skq = N.pyramid_fwd(*xd, L, p, scores=sc)
    ref_idx = R.select_indices_c(sqk.cpu().numpy(), skq.cpu().numpy(), L, p, k, S, idx.shape[-1])
    assert np.array_equal(idx, ref_idx)
    xc = [x.float().requires_grad_() for x in xs]
    ref, _ = O.lighthouse_layer(*xc, L, p, k, scorer="gla", dilation=dil, gk=gk.float(), indices=ref_idx)
    ref.backward(do.float())
    assert_close(out, ref, "gla layer out")
    for n_, x, c in zip("qkv", xg, xc):
        assert_close(x.grad, c.grad, f"gla layer d{n_}")
    # the scorer module's 5-tuple carries the same scores
    s5 = scorer(*xd, gd)
    assert torch.equal(s5[0].float(), sqk.bfloat16().float())


def test_gla_model_layer(pkg, dev):
    """The model's Attention with lighthouse_scorer='gla' builds the gate projection
    wg and runs forward and backward through the native layer (the patch's wiring,
    lighthouse-attention.patch:245-360,709-710); wg receives no gradient, as in the
    reference, whose scores only feed the selection."""
    L3 = pkg.llama3
    args = L3.TransformerModelArgs(dim=256, n_layers=2, n_heads=2, n_kv_heads=2, vocab_size=256, hidden_dim=768,
                                   max_seq_len=4096, use_selection_lighthouse=True, lighthouse_scorer="gla",
                                   lighthouse_num_levels=3, lighthouse_pooling_factor=4, lighthouse_topk=128,
                                   lighthouse_full_attn_layers=[0])
    torch.manual_seed(0)
    with torch.device(dev):
        m = L3.Transformer(args)
    m.init_weights(dev)
    L3.cast_params_(m, torch.bfloat16)
    att = m.layers["1"].attention
    assert att._needs_gate and hasattr(att, "wg")
    tok = torch.randint(0, 256, (1, 2048), device=dev, generator=torch.Generator(dev).manual_seed(1))
    out = m(tok)
    loss = torch.nn.functional.cross_entropy(out.flatten(0, 1).float(), tok.roll(-1, 1).flatten())
    loss.backward()
    assert torch.isfinite(loss)
    assert att.wg.weight.grad is None
    assert att.wq.weight.grad is not None and torch.isfinite(att.wq.weight.grad.float()).all()


@pytest.mark.parametrize("B,S,H,dil,gate,segs", [(1, 8192, 1, 2, "typical", (2, 3, 5, 0, 64)),
                                                 (1, 1000, 2, 4, "strong", (2, 3, 4)),
                                                 (2, 4096, 1, 1, "none", (3, 0, 64))])
def test_gla_segments(pkg, dev, B, S, H, dil, gate, segs):
    """The segmented walk (a first pass forms each segment's final state from a zero
    state; segment s starts from the decayed sum of the earlier ones) against the
    oracle and against the one-segment walk on the same inputs, including a last
    chunk shorter than 64 tokens and one chunk per segment."""
    N = pkg._native
    L, p = 3, 2
    xs, gk, xd, gd = _inputs(B, S, H, gate, 7 * S + H, dev)
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    r_qk, r_kq, *_ = O.gla_scorer(*[x.float() for x in xs], gk.float(), dil, p, L, round_bf16=True)
    one = N.gla_scores(*xd, gd, dil, S_tot, segments=1)
    assert N.lib().lh_gla_workspace_bytes(B, S, H, D, dil, 1) == 0
    for segments in segs:
        print(f"gla segments={segments} B={B} S={S} H={H} dil={dil} gate={gate}", flush=True)
        assert N.lib().lh_gla_workspace_bytes(B, S, H, D, dil, segments) > 0 or segments == 0
        got = N.gla_scores(*xd, gd, dil, S_tot, segments=segments)
        for g_, o_, ref, name in zip(got, one, (r_qk, r_kq), ("qk", "kq")):
            g_ = g_[..., :S].cpu()
            o_ = o_[..., :S].cpu()
            assert_close(g_, ref[..., :S], f"gla segments={segments} {name}")
            assert (_ulps(g_, ref[..., :S]) <= 1).float().mean().item() >= 0.95
            # against the sequential walk: the state differs only by fp32 rounding
            u = _ulps(g_, o_)
            assert u.max().item() <= 2, f"segments={segments} {name}: {u.max().item()} ulps from one segment"
            assert (u == 0).float().mean().item() >= 0.97, f"segments={segments} {name}: too many differ"


def test_gla_workspace_errors(pkg, dev):
    """A missing or short workspace is rejected before any launch."""
    N = pkg._native
    lib = N.lib()
    B, S, H, dil = 1, 8192, 1, 2
    xs, gk, xd, gd = _inputs(B, S, H, "typical", 3, dev)
    need = lib.lh_gla_workspace_bytes(B, S, H, D, dil, 4)
    assert need > 0
    out = [torch.empty(B, H, S, device=dev) for _ in range(2)]
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    ptr = N._ptr
    args = [ptr(xd[0]), ptr(xd[1]), ptr(xd[2]), ptr(gd.float().contiguous()), ptr(out[0]), ptr(out[1]),
            B, S, H, D, dil, S, 1.0 / D ** 0.5, 4]
    assert lib.lh_gla_scores(*args, None, 0, 0, N._stream(dev)) == 1  # LH_ERR_INVALID_ARG
    assert lib.lh_gla_scores(*args, ptr(ws), need - 4, 0, N._stream(dev)) == 1  # LH_ERR_INVALID_ARG
    assert lib.lh_gla_scores(*args, ptr(ws), need, 0, N._stream(dev)) == 0
    torch.cuda.synchronize()


def test_gla_scores_independent_of_batch(pkg, dev):
    """A sequence's scores are bit-identical whether it is scored alone or as one
    of several sequences and heads: the automatic segment count depends on the
    per-sequence length only (here 4 segments of 32 chunks)."""
    N = pkg._native
    B, S, H, dil, L, p = 3, 32768, 2, 4, 3, 4
    print(f"gla batch independence B={B} S={S} H={H} dil={dil}", flush=True)
    xs, gk, xd, gd = _inputs(B, S, H, "typical", 11, dev)
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    assert N.lib().lh_gla_workspace_bytes(B, S, H, D, dil, 0) == B * dil * H * 2 * 3 * (D * D + 1) * 4
    full = N.gla_scores(*xd, gd, dil, S_tot)
    for b in (0, 2):
        for h in range(H):
            one = N.gla_scores(*[x[b:b + 1, :, h:h + 1].contiguous() for x in xd],
                               gd[b:b + 1, :, h:h + 1].contiguous(), dil, S_tot)
            for f_, o_, name in zip(full, one, ("qk", "kq")):
                assert torch.equal(f_[b:b + 1, h:h + 1, :S], o_[..., :S]), f"batch {b} head {h} {name} differs"
