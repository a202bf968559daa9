"""GPU parity at the benchmark configurations' full sizes (B=1, H=8, D=128).

Each case runs the whole layer forward + backward on the device through
LighthouseLocal, built the way the reference model builds it
(lighthouse-attention.patch:601-638, 675-681), on the same seeded inputs that
bench.py times.  Checks:
  * selection bit-exact on every head against the slot-literal C restatement,
    on the scores the device computed;
  * outputs and input gradients against the fp32 oracle on a subset of heads,
    on the device's index set.  Heads never mix along the path (scores,
    selection, attention and fan-out are per head), so one head's results
    depend only on that head's inputs;
  * for the dilated scorer, the base-level scores of the checked heads against
    the oracle's dilated scorer at the full sequence length.
"""
import numpy as np
import pytest
import torch

import bench
from conftest import assert_close
from oracle import lh_oracle as O
from oracle import select_ref as R

pytestmark = pytest.mark.gpu

CASES = [  # (workload, heads checked against the fp32 oracle)
    ("cfg2", (0, 5)),
    ("cfg3_k1536", (3,)),
    ("cfg3_k3072", (6,)),
    ("cfg3_k6144", (1,)),
    ("cfg4", (2,)),
    ("cfg5_layer", (4,)),
    ("gla", (7,)),
]


@pytest.mark.parametrize("name,heads", CASES)
def test_config_full_size(pkg, dev, name, heads):
    w = bench.WORKLOADS[name]
    S, L, p, k, strict = w["S"], w["L"], w["p"], w["topk"], w["strict"]
    dil = w.get("dilation", 0)
    print(f"config {name}: S={S} L={L} p={p} k={k} scorer={w['scorer']} strict={strict} heads={heads}",
          flush=True)
    xs, dout, *gate = bench.make_inputs(w, torch, dev)
    gk = gate[0] if gate else None
    xg = [x.clone().requires_grad_() for x in xs]
    layer = bench.make_layer(w, pkg)
    out = layer(*xg, gk=gk) if gk is not None else layer(*xg)
    out.backward(dout)
    idx = layer.last_indices
    torch.cuda.synchronize()

    _, _, S_tot = pkg._native.pyramid_lengths(S, L, p)
    with torch.no_grad():
        if gk is not None:
            sc = pkg._native.gla_scores(*xs, gk, dil, S_tot)
            _, _, _, sqk, skq = pkg._native.pyramid_fwd(*xs, L, p, scores=sc)
        elif dil:
            sc = pkg._native.dilated_scores(*xs, dil, S_tot)
            _, _, _, sqk, skq = pkg._native.pyramid_fwd(*xs, L, p, scores=sc)
        else:
            _, _, _, sqk, skq = pkg._native.pyramid_fwd(*xs, L, p)
    S_sel = pkg._native.geometry(S, L, p, k, strict)[3]
    ref_idx = R.select_indices_c(sqk.cpu().numpy(), skq.cpu().numpy(), L, p, k, S, S_sel, strict=strict)
    got_idx = idx.cpu().numpy()
    assert np.array_equal(got_idx, ref_idx), f"{(got_idx != ref_idx).sum()} of {ref_idx.size} indices differ"

    hs = list(heads)
    xc = [x.detach().cpu()[:, :, hs].float().requires_grad_() for x in xs]
    if gk is not None:
        r_qk, r_kq, *_ = O.gla_scorer(*[x.detach() for x in xc], gk.cpu()[:, :, hs].float(), dil, p, L,
                                      round_bf16=True)
        assert_close(sqk[:, hs, :S], r_qk[..., :S], f"{name} gla scores qk", max_abs=1e-2, rel_l2=5e-3)
        assert_close(skq[:, hs, :S], r_kq[..., :S], f"{name} gla scores kq", max_abs=1e-2, rel_l2=5e-3)
    elif dil:
        r_qk, r_kq, *_ = O.dilated_scorer(*[x.detach() for x in xc], dil, p, L)
        assert_close(sqk[:, hs, :S], r_qk[..., :S], f"{name} dilated scores qk", max_abs=1e-2, rel_l2=5e-3)
        assert_close(skq[:, hs, :S], r_kq[..., :S], f"{name} dilated scores kq", max_abs=1e-2, rel_l2=5e-3)
    # with the index set given, the oracle's scores are unused; both scorers share the Q/K/V pyramid
    ref_out, _ = O.lighthouse_layer(*xc, L, p, k, scorer="norm", indices=ref_idx[:, hs], strict=strict)
    ref_out.backward(dout.cpu()[:, hs].float())
    assert_close(out.detach()[:, hs], ref_out, f"{name} out")
    for n, x, c in zip("qkv", xg, xc):
        assert_close(x.grad[:, :, hs], c.grad, f"{name} d{n}")


@pytest.mark.parametrize("name,heads", [("cfg2", (1,)), ("cfg4", (6,)), ("gla", (3,))])
def test_config_full_size_fp16(pkg, dev, name, heads):
    """The same full-size layers on fp16 rows (the bench inputs cast to fp16):
    selection bit-exact on every head on the device's fp16 scores, scores of
    the dilated and GLA scorers against the oracle with fp16 roundings, outputs
    and gradients (fp16) against the fp32 oracle on the checked heads."""
    w = bench.WORKLOADS[name]
    S, L, p, k, strict = w["S"], w["L"], w["p"], w["topk"], w["strict"]
    dil = w.get("dilation", 0)
    print(f"config fp16 {name}: S={S} L={L} p={p} k={k} scorer={w['scorer']} heads={heads}", flush=True)
    xs, dout, *gate = bench.make_inputs(w, torch, dev)
    xs, dout = [x.half() for x in xs], dout.half()
    gk = gate[0] if gate else None
    xg = [x.clone().requires_grad_() for x in xs]
    layer = bench.make_layer(w, pkg)
    out = layer(*xg, gk=gk) if gk is not None else layer(*xg)
    assert out.dtype == torch.float16
    out.backward(dout)
    idx = layer.last_indices
    torch.cuda.synchronize()

    N = pkg._native
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    with torch.no_grad():
        if gk is not None:
            sc = N.gla_scores(*xs, gk, dil, S_tot)
            _, _, _, sqk, skq = N.pyramid_fwd(*xs, L, p, scores=sc)
        elif dil:
            sc = N.dilated_scores(*xs, dil, S_tot)
            _, _, _, sqk, skq = N.pyramid_fwd(*xs, L, p, scores=sc)
        else:
            _, _, _, sqk, skq = N.pyramid_fwd(*xs, L, p)
    S_sel = N.geometry(S, L, p, k, strict)[3]
    ref_idx = R.select_indices_c(sqk.cpu().numpy(), skq.cpu().numpy(), L, p, k, S, S_sel, strict=strict)
    got_idx = idx.cpu().numpy()
    assert np.array_equal(got_idx, ref_idx), f"{(got_idx != ref_idx).sum()} of {ref_idx.size} indices differ"

    hs = list(heads)
    xc = [x.detach().cpu()[:, :, hs].float().requires_grad_() for x in xs]
    if gk is not None:
        r_qk, r_kq, *_ = O.gla_scorer(*[x.detach() for x in xc], gk.cpu()[:, :, hs].float(), dil, p, L,
                                      round_to=torch.float16)
        assert_close(sqk[:, hs, :S], r_qk[..., :S], f"{name} fp16 gla scores qk", max_abs=1e-2, rel_l2=5e-3)
        assert_close(skq[:, hs, :S], r_kq[..., :S], f"{name} fp16 gla scores kq", max_abs=1e-2, rel_l2=5e-3)
    elif dil:
        r_qk, r_kq, *_ = O.dilated_scorer(*[x.detach() for x in xc], dil, p, L)
        assert_close(sqk[:, hs, :S], r_qk[..., :S], f"{name} fp16 dilated scores qk", max_abs=1e-2, rel_l2=5e-3)
        assert_close(skq[:, hs, :S], r_kq[..., :S], f"{name} fp16 dilated scores kq", max_abs=1e-2, rel_l2=5e-3)
    ref_out, _ = O.lighthouse_layer(*xc, L, p, k, scorer="norm", indices=ref_idx[:, hs], strict=strict)
    ref_out.backward(dout.cpu()[:, hs].float())
    assert_close(out.detach()[:, hs], ref_out, f"{name} fp16 out")
    for n, x, c in zip("qkv", xg, xc):
        assert x.grad.dtype == torch.float16
        assert_close(x.grad[:, :, hs], c.grad, f"{name} fp16 d{n}")
