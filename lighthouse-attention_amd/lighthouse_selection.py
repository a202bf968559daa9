"""Lighthouse selection attention on MI355X (gfx950): the ``lighthouse_selection``
module API, backed by hand-written HIP kernels behind a C ABI.

Drop-in for the reference module ``torchtitan/models/llama3/model/lighthouse_selection.py``
(reference repository ``src/lighthouse_selection.py``): the names imported by the
reference's model wiring (``lighthouse-attention.patch:591-598``) all exist here
with the same constructor arguments and the same forward signatures.

==================================  =====================================================
name here                           reference
==================================  =====================================================
``DialatedLighthouseNormScorer``    ``src/lighthouse_selection.py:578-616``
``DilatedLighthouseScorer``         ``src/lighthouse_selection.py:618-689``
``DilatedLighthouseGLAScorer``      ``src/lighthouse_selection.py:692-755``
``LighthouseLocal``                 ``src/lighthouse_selection.py:772-825``
``scatter_to_base_sequence``        ``src/lighthouse_selection.py:758-770``
``DialatedLighthouseNormScorerCP``  ``src/lighthouse_selection.py:943-982`` (not built)
``LighthouseCP``                    ``src/lighthouse_selection.py:985-1054`` (not built)
``LighthouseSelectionQkKqChunkedTopkNvrtc``  ``src/lighthouse_selection_cuda.py:359-428``
``compute_output_indices_selection``         ``src/lighthouse_selection_cuda.py:346-357``
==================================  =====================================================

Differences from the reference, all deliberate:
  * ``LighthouseLocal`` runs the whole layer natively (pyramid, selection,
    gathered causal attention with softmax scale 1/sqrt(D), fan-out) when its
    scorer is one of this module's; the ``attention`` argument is kept for the
    constructor signature and is only called when ``use_native_attention=False``.
  * Selection is reference-exact by default (``tie_break="reference"``);
    ``tie_break="lower_index"`` breaks score ties by lower index instead.
  * ``strict=True`` (default) raises where the reference asserts or overruns
    its output slots; ``strict=False`` compacts each tile's entries instead.
  * ``DilatedLighthouseScorer``'s ``attention`` is optional and ``head_dim`` is
    accepted, so the reference's own builder call (``lighthouse-attention.patch:623-628``)
    constructs it.
  * ``LighthouseLocal.forward`` takes the GLA scorer's gate as ``gk`` (the
    reference's caller passes it, lighthouse-attention.patch:709-710, but the
    reference's ``LighthouseLocal.forward`` has no such parameter).
"""
from __future__ import annotations

import math
import os
from functools import lru_cache

import torch
import torch.nn as nn

from . import _native as N

__all__ = [
    "DilatedLighthouseScorer", "DialatedLighthouseNormScorer", "DilatedLighthouseGLAScorer",
    "LighthouseLocal", "DialatedLighthouseNormScorerCP", "LighthouseCP", "scatter_to_base_sequence",
    "LighthouseSelectionQkKqChunkedTopkNvrtc", "LighthouseSelectionQkKqChunkedTopkHip",
    "compute_output_indices_selection", "lighthouse_layer", "lighthouse_layer_rope",
]


@lru_cache(maxsize=100)
def compute_output_indices_selection(N_: int, num_levels: int, pooling_factor: int, topk: int) -> int:
    """Selected length by the reference's formula (``src/lighthouse_selection_cuda.py:346-357``):
    the coarsest level whole plus ``pooling_factor * topk`` per finer level."""
    total = 0
    for level in range(num_levels, 0, -1):
        c_l = pooling_factor ** (level - 1)
        total += N_ // c_l if level == num_levels else pooling_factor * topk
    return total


class LighthouseSelectionQkKqChunkedTopkHip:
    """Per-tile hierarchical top-k selection (``src/lighthouse_selection_cuda.py:359-428``)."""

    @staticmethod
    @torch.no_grad()
    def forward(scores_qk, scores_kq, num_levels, pooling_factor, topk, actual_seq_len,
                tie_break: str = "reference", strict: bool = True):
        assert scores_qk.shape == scores_kq.shape
        assert scores_qk.is_cuda and scores_kq.is_cuda
        assert scores_qk.dtype == torch.float32
        assert topk % 128 == 0, "topk must be a multiple of 128"
        assert (pooling_factor & (pooling_factor - 1)) == 0, "pf must be power of 2"
        assert topk // 2 >= pooling_factor
        idx, _ = N.select_topk(scores_qk.float(), scores_kq.float(), actual_seq_len, num_levels,
                               pooling_factor, topk, tie=tie_break, strict=strict, with_inverse=False)
        return idx


# The reference's class name, so callers written against it keep working.
LighthouseSelectionQkKqChunkedTopkNvrtc = LighthouseSelectionQkKqChunkedTopkHip


# ---------------------------------------------------------------------------
# autograd functions
# ---------------------------------------------------------------------------
def _base_rows(xq, xk, xv, pq=None, pk=None, pv=None):
    S = xq.shape[1]
    sb, ss, sh, _ = xq.stride()
    if pq is None:
        return N.Rows(xq, xk, xv, (sb, ss, sh))
    pb, ps, ph, _ = pq.stride()
    return N.Rows(xq, xk, xv, (sb, ss, sh), pq, pk, pv, (pb, ps, ph), split=S, limit=S + pq.shape[1])


_op_hook = None


def set_op_hook(fn):
    """Install ``fn(name)``, called on the host right after each native op of the
    layer is enqueued (names: ``pyramid``, ``dilated_scores``, ``select``,
    ``attn_fwd``, ``scatter_fwd``, ``scatter_bwd``, ``attn_bwd_dkdv``,
    ``attn_bwd_dq``, ``pyramid_bwd``) and with ``fwd_start`` / ``bwd_start``
    before the first one; e.g. to record a stream event per op.  The dense causal
    layers report ``dense_attn_fwd`` / ``dense_attn_bwd`` after ``dense_fwd_start`` /
    ``dense_bwd_start``.  ``None`` removes it."""
    global _op_hook
    _op_hook = fn


def _mark(name):
    if _op_hook is not None:
        _op_hook(name)


def _layer_fwd(xq, xk, xv, L, p, topk, tie, strict, dilation, seq_major, gk=None, scale=None):
    """Forward of the whole layer on contiguous bf16 [B, S, H, D] inputs:
    pyramid -> selection -> gathered causal attention -> fan-out.  The scorer is
    the norm scorer (dilation 0), the dilated one (dilation > 0) or, with the gate
    ``gk`` [B, S, H], the GLA one.  Returns ``(out, idx, saved)`` with
    ``saved = (pq, pk, pv, inv, o, lse)``.  ``scale``: the attention (and scorer)
    scale, 1/sqrt(D) when None."""
    B, S, H, D = xq.shape
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    _, _, _, S_sel = N.geometry(S, L, p, topk, strict)
    _mark("fwd_start")
    if gk is not None:
        scores = N.gla_scores(xq, xk, xv, gk, dilation, S_tot, scale)
        _mark("gla_scores")
        pq, pk, pv, sqk, skq = N.pyramid_fwd(xq, xk, xv, L, p, scores=scores)
    elif dilation:
        scores = N.dilated_scores(xq, xk, xv, dilation, S_tot, scale)
        _mark("dilated_scores")
        pq, pk, pv, sqk, skq = N.pyramid_fwd(xq, xk, xv, L, p, scores=scores)
    else:
        pq, pk, pv, sqk, skq = N.pyramid_fwd(xq, xk, xv, L, p)
    _mark("pyramid")
    idx, inv = N.select_topk(sqk, skq, S, L, p, topk, tie=tie, strict=strict)
    _mark("select")
    rows = _base_rows(xq, xk, xv, pq, pk, pv)
    o, lse = N.attn_fwd(rows, idx, B, H, S_sel, D, scale)
    _mark("attn_fwd")
    out = N.scatter_fwd(o, inv, S, S, L, p, seq_major=seq_major)
    _mark("scatter_fwd")
    return out, idx, (pq, pk, pv, inv, o, lse)


# The dK/dV and dQ kernels are independent: with two streams the dQ kernel runs on a
# side stream (default priority) beside the dK/dV kernel.  One stream is the default:
# the dQ kernel's query-block plan assumes the whole GPU, and beside the dK/dV kernel
# the pair measured slower than one after the other.
_bwd_streams = int(os.environ.get("LH_BWD_STREAMS", "1"))
_side = {}


def set_backward_streams(n: int) -> int:
    """1: dK/dV then dQ on the caller's stream; 2: dQ on a side stream beside dK/dV.
    Returns the previous setting."""
    global _bwd_streams
    prev, _bwd_streams = _bwd_streams, int(n)
    return prev


def _attn_bwd_pair(rows, idx, B, H, S_sel, dattn, lse, delta, D, scale=None):
    if _bwd_streams < 2 or torch.compiler.is_compiling():
        dks, dvs = N.attn_bwd_dkdv(rows, idx, B, H, S_sel, dattn, lse, delta, D, scale)
        _mark("attn_bwd_dkdv")
        dqs = N.attn_bwd_dq(rows, idx, B, H, S_sel, dattn, lse, delta, D, scale)
        _mark("attn_bwd_dq")
        return dqs, dks, dvs
    dev = dattn.device
    main = torch.cuda.current_stream(dev)
    side = _side.get(dev)
    if side is None:
        side = _side[dev] = torch.cuda.Stream(dev)
    side.wait_stream(main)  # dattn, delta (and everything before) are ready
    with torch.cuda.stream(side):
        _mark("side_start")
        dqs = N.attn_bwd_dq(rows, idx, B, H, S_sel, dattn, lse, delta, D, scale)
        _mark("attn_bwd_dq")
    dks, dvs = N.attn_bwd_dkdv(rows, idx, B, H, S_sel, dattn, lse, delta, D, scale)
    _mark("attn_bwd_dkdv")
    main.wait_stream(side)
    dqs.record_stream(main)  # allocated on the side stream, consumed and freed on the caller's
    _mark("join_start")
    return dqs, dks, dvs


def _layer_bwd(dout, xq, xk, xv, pq, pk, pv, idx, inv, o, lse, L, p, scale=None):
    """Backward of ``_layer_fwd``: fan-out adjoint (+ softmax delta) -> attention
    backward in selected space -> pyramid backward onto the base rows."""
    B, S, H, D = xq.shape
    S_sel = idx.shape[-1]
    _mark("bwd_start")
    dattn, delta = N.scatter_bwd(dout, idx, o, S, L, p)
    _mark("scatter_bwd")
    rows = _base_rows(xq, xk, xv, pq, pk, pv)
    dqs, dks, dvs = _attn_bwd_pair(rows, idx, B, H, S_sel, dattn, lse, delta, D, scale)
    dxq, dxk, dxv = N.pyramid_bwd(dqs, dks, dvs, inv, B, S, H, L, p, D)
    _mark("pyramid_bwd")
    return dxq, dxk, dxv


class _LighthouseLayerFn(torch.autograd.Function):
    """Whole layer (``_layer_fwd`` / ``_layer_bwd``) as one autograd node."""

    @staticmethod
    def forward(ctx, xq, xk, xv, L, p, topk, tie, strict, dilation, seq_major, gk, scale):
        xq, xk, xv = xq.contiguous(), xk.contiguous(), xv.contiguous()
        out, idx, (pq, pk, pv, inv, o, lse) = _layer_fwd(xq, xk, xv, L, p, topk, tie, strict, dilation,
                                                         seq_major, gk, scale)
        ctx.save_for_backward(xq, xk, xv, pq, pk, pv, idx, inv, o, lse)
        ctx.geo = (L, p, scale)
        ctx.mark_non_differentiable(idx)
        ctx.set_materialize_grads(False)  # no zero-filled gradient for the index output
        return out, idx

    @staticmethod
    def backward(ctx, dout, _didx):
        if dout is None:
            return (None,) * 12
        dx = _layer_bwd(dout, *ctx.saved_tensors, *ctx.geo)
        return dx + (None,) * 9  # the gate gets no gradient: the scores only feed the selection


def _need_layer_dtype(*ts):
    """The layer's kernels read and write bf16 or fp16 rows (all three inputs of
    one type; selection, softmax statistics and sums stay fp32).  The reference
    path is dtype-generic (``src/lighthouse_selection.py:522,528,559,562``);
    float32 inputs are refused rather than silently downcast: cast them (or run
    under autocast) to bfloat16 or float16 first."""
    for t in ts:
        if t.dtype not in N.ROW_DTYPES:
            raise TypeError("the native layer computes in bfloat16 or float16 (cast float32 inputs first, "
                            "e.g. under autocast); got " + str(t.dtype))
    if len({t.dtype for t in ts}) > 1:
        raise TypeError("xq, xk and xv must share a dtype; got " + ", ".join(str(t.dtype) for t in ts))


def lighthouse_layer(xq, xk, xv, num_levels: int = 3, pooling_factor: int = 4, topk: int = 1024,
                     tie_break: str = "reference", strict: bool = True, dilation: int = 0,
                     seq_major: bool = False, gk=None):
    """Functional form of the native layer: ``(out [B, H, S, D], indices [B, H, S_sel])``.

    ``dilation > 0`` selects the dilated scorer, 0 the norm scorer; a gate ``gk``
    [B, S, H] (log gates) selects the GLA scorer over ``dilation`` virtual heads per
    head (the gate receives no gradient, as in the reference).  ``seq_major``
    stores ``out`` as ``[B, S, H, D]`` (the returned tensor is its ``[B, H, S, D]``
    view), which is the layout the model's output projection reads.  Under
    ``torch.compile`` the layer is one registered custom op (traced without a
    graph break); eagerly it is an ``autograd.Function``; both run the same kernels.

    The kernels work on 128-wide heads.  A head dim D < 128 (a multiple of 8, e.g.
    the 64 and 72 of the patch's ablation flavors) runs zero-padded to 128 with the
    scale 1/sqrt(D): zero columns change no dot product, norm or mean, so the
    results are the D-wide layer's, at 128/D times the work."""
    D = xq.shape[-1]
    if D > N.D_SUPPORTED or D % 8:
        raise ValueError(f"head_dim must be a multiple of 8 and at most {N.D_SUPPORTED}, got {D}")
    if not (xq.shape == xk.shape == xv.shape):
        raise AssertionError("xq, xk and xv must have the same shape (n_kv_heads == n_heads)")
    _need_layer_dtype(xq, xk, xv)
    if tie_break not in N.TIE_MODES:
        raise ValueError(f"tie_break must be one of {sorted(N.TIE_MODES)}, got {tie_break!r}")
    if gk is not None:
        if dilation <= 0:
            raise ValueError("the GLA scorer needs dilation >= 1")
        gk = gk.detach()
    scale = None
    if D < N.D_SUPPORTED:
        scale = D ** -0.5
        xq, xk, xv = (torch.nn.functional.pad(x, (0, N.D_SUPPORTED - D)) for x in (xq, xk, xv))
    if torch.compiler.is_compiling():
        out, idx = _compiled_ops.layer_fwd(xq, xk, xv, num_levels, pooling_factor, topk, tie_break, bool(strict),
                                           int(dilation), bool(seq_major), gk, scale)[:2]
    else:
        out, idx = _LighthouseLayerFn.apply(xq, xk, xv, num_levels, pooling_factor, topk, tie_break, strict,
                                            int(dilation), bool(seq_major), gk, scale)
    return (out[..., :D] if D < N.D_SUPPORTED else out), idx


def _rope_layer_fwd(xqkv, freqs, H, L, p, topk, tie, strict, seq_major):
    """Forward of the layer fed from the fused [q | k | v] projection output; returns
    ``(out, idx, saved)`` with ``saved = (xr, pq, pk, pv, inv, o, lse)``."""
    B, S, W = xqkv.shape
    D = W // (3 * H)
    _, _, _, S_sel = N.geometry(S, L, p, topk, strict)
    _mark("fwd_start")
    xr, pq, pk, pv, sqk, skq = N.rope_pyramid_fwd(xqkv, freqs, H, L, p, D)
    _mark("pyramid")
    idx, inv = N.select_topk(sqk, skq, S, L, p, topk, tie=tie, strict=strict)
    _mark("select")
    rows = _rope_rows(xqkv, xr, H, D, pq, pk, pv)
    o, lse = N.attn_fwd(rows, idx, B, H, S_sel, D)
    _mark("attn_fwd")
    out = N.scatter_fwd(o, inv, S, S, L, p, seq_major=seq_major)
    _mark("scatter_fwd")
    return out, idx, (xr, pq, pk, pv, inv, o, lse)


def _rope_layer_bwd(dout, xqkv, freqs, xr, pq, pk, pv, idx, inv, o, lse, H, L, p):
    B, S, W = xqkv.shape
    D = W // (3 * H)
    S_sel = idx.shape[-1]
    _mark("bwd_start")
    dattn, delta = N.scatter_bwd(dout, idx, o, S, L, p)
    _mark("scatter_bwd")
    rows = _rope_rows(xqkv, xr, H, D, pq, pk, pv)
    dqs, dks, dvs = _attn_bwd_pair(rows, idx, B, H, S_sel, dattn, lse, delta, D)
    dx = N.pyramid_rope_bwd(dqs, dks, dvs, inv, freqs, B, S, H, L, p, D)
    _mark("pyramid_bwd")
    return dx


class _LighthouseRopeLayerFn(torch.autograd.Function):
    """The layer fed straight from the fused [q | k | v] projection output: the
    rotary embedding of q and k runs inside the pyramid pass (and its adjoint
    inside the pyramid backward), otherwise exactly ``_LighthouseLayerFn`` with
    the norm scorer.  The rotated rows are stored once, for the attention
    kernels' gathers; v rows are read from the projection output in place."""

    @staticmethod
    def forward(ctx, xqkv, freqs, H, L, p, topk, tie, strict, seq_major):
        out, idx, saved = _rope_layer_fwd(xqkv, freqs, H, L, p, topk, tie, strict, seq_major)
        xr, pq, pk, pv, inv, o, lse = saved
        ctx.save_for_backward(xqkv, freqs, xr, pq, pk, pv, idx, inv, o, lse)
        ctx.geo = (H, L, p)
        ctx.mark_non_differentiable(idx)
        ctx.set_materialize_grads(False)
        return out, idx

    @staticmethod
    def backward(ctx, dout, _didx):
        if dout is None:
            return (None,) * 9
        dx = _rope_layer_bwd(dout, *ctx.saved_tensors, *ctx.geo)
        return (dx,) + (None,) * 8


def _rope_rows(xqkv, xr, H, D, pq, pk, pv):
    B, S, _ = xqkv.shape
    hd = H * D
    q, k = xr[..., :hd], xr[..., hd:2 * hd]
    v = xqkv[..., 2 * hd:]
    sb, ss, _ = xqkv.stride()
    pb, ps, ph, _ = pq.stride()
    return N.Rows(q, k, v, (sb, ss, D), pq, pk, pv, (pb, ps, ph), split=S, limit=S + pq.shape[1])


def lighthouse_layer_rope(xqkv, freqs, n_heads: int, num_levels: int = 3, pooling_factor: int = 4,
                          topk: int = 1024, tie_break: str = "reference", strict: bool = True,
                          seq_major: bool = False):
    """The norm-scorer layer applied to the fused projection output.

    ``xqkv`` bf16 [B, S, 3*H*D] = [q | k | v] heads before the rotary embedding;
    ``freqs`` fp32 [>= S, D/2, 2] = (cos, sin) per position and pair (the real view
    of torchtitan's ``freqs_cis``).  Equal to ``lighthouse_layer(rope(q), rope(k), v)``:
    the forward gives the same bits as rotating first (rotation rounded to bf16 once
    per element), the gradient w.r.t. ``xqkv`` is the rotated-back pyramid gradient
    rounded once.  Returns ``(out [B, H, S, D], indices)``."""
    B, S, W = xqkv.shape
    if W % (3 * n_heads) or W // (3 * n_heads) != N.D_SUPPORTED:
        raise ValueError(f"xqkv must hold 3 x {n_heads} heads of dim {N.D_SUPPORTED}, got width {W}")
    if xqkv.dtype != torch.bfloat16:
        raise TypeError("the native layer computes in bfloat16; got " + str(xqkv.dtype))
    if tie_break not in N.TIE_MODES:
        raise ValueError(f"tie_break must be one of {sorted(N.TIE_MODES)}, got {tie_break!r}")
    if xqkv.stride(2) != 1 or xqkv.stride(1) % 8 or xqkv.stride(0) != S * xqkv.stride(1):
        xqkv = xqkv.contiguous()
    freqs = freqs.contiguous()
    if torch.compiler.is_compiling():
        out, idx = _compiled_ops.rope_layer_fwd(xqkv, freqs, n_heads, num_levels, pooling_factor, topk, tie_break,
                                                bool(strict), bool(seq_major))[:2]
        return out, idx
    return _LighthouseRopeLayerFn.apply(xqkv, freqs, n_heads, num_levels, pooling_factor, topk, tie_break, strict,
                                        bool(seq_major))


class _CompiledOps:
    """The two layer forms as ``torch.library`` custom ops with fake (meta)
    implementations and registered autograd, so ``torch.compile`` traces a
    caller's block through the layer without a graph break.  The reference marks
    its selection ``@torch.compiler.disable`` and compiles each block with
    ``fullgraph=False`` (``lighthouse-attention.patch:9-12,540-548``).  Saved
    tensors are extra outputs of the forward op (custom ops cannot hold state);
    the backward is a second op."""

    def __init__(self):
        lib = "lighthouse_amd"
        if hasattr(torch.ops, lib) and hasattr(getattr(torch.ops, lib), "layer_fwd"):
            ops = getattr(torch.ops, lib)  # already registered by an earlier import of this module
            self.layer_fwd, self.rope_layer_fwd = ops.layer_fwd, ops.rope_layer_fwd
            return

        @torch.library.custom_op(f"{lib}::layer_fwd", mutates_args=(), schema=(
            "(Tensor xq, Tensor xk, Tensor xv, int L, int p, int topk, str tie, bool strict, int dilation, "
            "bool seq_major, Tensor? gk, float? scale) -> "
            "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)"))
        def layer_fwd(xq, xk, xv, L, p, topk, tie, strict, dilation, seq_major, gk, scale):
            xq, xk, xv = xq.contiguous(), xk.contiguous(), xv.contiguous()
            out, idx, saved = _layer_fwd(xq, xk, xv, L, p, topk, tie, strict, dilation, seq_major, gk, scale)
            return (out, idx) + saved

        @layer_fwd.register_fake
        def _(xq, xk, xv, L, p, topk, tie, strict, dilation, seq_major, gk, scale):
            B, S, H, D = xq.shape
            _, _, S_tot = N.pyramid_lengths(S, L, p)
            S_sel = N.geometry(S, L, p, topk, strict)[3]
            out = xq.new_empty(B, S, H, D).transpose(1, 2) if seq_major else xq.new_empty(B, H, S, D)
            pooled = [xq.new_empty(B, S_tot - S, H, D) for _ in range(3)]
            return (out, xq.new_empty(B, H, S_sel, dtype=torch.int32), *pooled,
                    xq.new_empty(B, H, S_tot, dtype=torch.int32), xq.new_empty(B, H, S_sel, D),
                    xq.new_empty(B, H, S_sel, dtype=torch.float32))

        @torch.library.custom_op(f"{lib}::layer_bwd", mutates_args=(), schema=(
            "(Tensor dout, Tensor xq, Tensor xk, Tensor xv, Tensor pq, Tensor pk, Tensor pv, Tensor idx, "
            "Tensor inv, Tensor o, Tensor lse, int L, int p, float? scale) -> (Tensor, Tensor, Tensor)"))
        def layer_bwd(dout, xq, xk, xv, pq, pk, pv, idx, inv, o, lse, L, p, scale):
            xq, xk, xv = xq.contiguous(), xk.contiguous(), xv.contiguous()
            return _layer_bwd(dout, xq, xk, xv, pq, pk, pv, idx, inv, o, lse, L, p, scale)

        @layer_bwd.register_fake
        def _(dout, xq, xk, xv, pq, pk, pv, idx, inv, o, lse, L, p, scale):
            return tuple(torch.empty(xq.shape, dtype=xq.dtype, device=xq.device) for _ in range(3))

        def layer_setup(ctx, inputs, output):
            xq, xk, xv, L, p = inputs[:5]
            ctx.save_for_backward(xq, xk, xv, *output[2:5], output[1], *output[5:])
            ctx.geo = (L, p, inputs[11])

        def layer_grad(ctx, dout, *_unused):
            if dout is None:
                return (None,) * 12
            xq, xk, xv, pq, pk, pv, idx, inv, o, lse = ctx.saved_tensors
            dx = layer_bwd(dout, xq, xk, xv, pq, pk, pv, idx, inv, o, lse, *ctx.geo)
            return tuple(dx) + (None,) * 9

        layer_fwd.register_autograd(layer_grad, setup_context=layer_setup)

        @torch.library.custom_op(f"{lib}::rope_layer_fwd", mutates_args=(), schema=(
            "(Tensor xqkv, Tensor freqs, int H, int L, int p, int topk, str tie, bool strict, bool seq_major) -> "
            "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)"))
        def rope_layer_fwd(xqkv, freqs, H, L, p, topk, tie, strict, seq_major):
            out, idx, saved = _rope_layer_fwd(xqkv, freqs, H, L, p, topk, tie, strict, seq_major)
            return (out, idx) + saved

        @rope_layer_fwd.register_fake
        def _(xqkv, freqs, H, L, p, topk, tie, strict, seq_major):
            B, S, W = xqkv.shape
            D = W // (3 * H)
            _, _, S_tot = N.pyramid_lengths(S, L, p)
            S_sel = N.geometry(S, L, p, topk, strict)[3]
            e = xqkv.new_empty
            out = e(B, S, H, D).transpose(1, 2) if seq_major else e(B, H, S, D)
            xr = xqkv.new_empty_strided(xqkv.shape, xqkv.stride())
            pooled = [e(B, S_tot - S, H, D) for _ in range(3)]
            return (out, e(B, H, S_sel, dtype=torch.int32), xr, *pooled, e(B, H, S_tot, dtype=torch.int32),
                    e(B, H, S_sel, D), e(B, H, S_sel, dtype=torch.float32))

        @torch.library.custom_op(f"{lib}::rope_layer_bwd", mutates_args=(), schema=(
            "(Tensor dout, Tensor xqkv, Tensor freqs, Tensor xr, Tensor pq, Tensor pk, Tensor pv, Tensor idx, "
            "Tensor inv, Tensor o, Tensor lse, int H, int L, int p) -> Tensor"))
        def rope_layer_bwd(dout, xqkv, freqs, xr, pq, pk, pv, idx, inv, o, lse, H, L, p):
            return _rope_layer_bwd(dout, xqkv, freqs, xr, pq, pk, pv, idx, inv, o, lse, H, L, p)

        @rope_layer_bwd.register_fake
        def _(dout, xqkv, freqs, xr, pq, pk, pv, idx, inv, o, lse, H, L, p):
            return torch.empty(xqkv.shape, dtype=xqkv.dtype, device=xqkv.device)

        def rope_setup(ctx, inputs, output):
            xqkv, freqs, H, L, p = inputs[:5]
            ctx.save_for_backward(xqkv, freqs, *output[2:6], output[1], *output[6:])
            ctx.geo = (H, L, p)

        def rope_grad(ctx, dout, *_unused):
            if dout is None:
                return (None,) * 9
            dx = rope_layer_bwd(dout, *ctx.saved_tensors, *ctx.geo)
            return (dx,) + (None,) * 8

        rope_layer_fwd.register_autograd(rope_grad, setup_context=rope_setup)
        self.layer_fwd, self.rope_layer_fwd = layer_fwd, rope_layer_fwd


_compiled_ops = _CompiledOps()


class _PyramidCatFn(torch.autograd.Function):
    """The reference scorer's 5-tuple from the native pyramid; backward through the
    dense pyramid adjoint (``g[pyramid row]`` gathered onto base rows).  Head dims
    below 128 run zero-padded (the padded columns of the returned rows are cut off)."""

    @staticmethod
    def forward(ctx, xq, xk, xv, L, p, dilation, base_qk=None, base_kq=None):
        B, S, H, D0 = xq.shape
        xq, xk, xv = xq.contiguous(), xk.contiguous(), xv.contiguous()
        if D0 < N.D_SUPPORTED:
            xq, xk, xv = (torch.nn.functional.pad(x, (0, N.D_SUPPORTED - D0)) for x in (xq, xk, xv))
        D = xq.shape[-1]
        _, _, S_tot = N.pyramid_lengths(S, L, p)
        cats = [torch.empty(B, S_tot, H, D, dtype=xq.dtype, device=xq.device) for _ in range(3)]
        for c, x in zip(cats, (xq, xk, xv)):
            c[:, :S].copy_(x)
        if base_qk is not None:  # base-level scores computed by the caller ([B, H, S])
            scores = tuple(torch.empty(B, H, S_tot, dtype=torch.float32, device=xq.device) for _ in range(2))
            scores[0][..., :S].copy_(base_qk)
            scores[1][..., :S].copy_(base_kq)
        else:
            scores = N.dilated_scores(xq, xk, xv, dilation, S_tot, D0 ** -0.5) if dilation else None
        _, _, _, sqk, skq = N.pyramid_fwd(xq, xk, xv, L, p, scores=scores,
                                          pooled_out=tuple(c[:, S:] for c in cats))
        ctx.geo = (B, S, H, D, L, p, D0)
        ctx.mark_non_differentiable(sqk, skq)
        return (sqk.to(xq.dtype), skq.to(xq.dtype), *(c[..., :D0].transpose(1, 2) for c in cats))

    @staticmethod
    def backward(ctx, _g1, _g2, gq, gk, gv):
        B, S, H, D, L, p, D0 = ctx.geo
        gs = [g if g is not None else None for g in (gq, gk, gv)]
        ref = next((g for g in gs if g is not None), None)
        if ref is None:
            return None, None, None, None, None, None, None, None
        gs = [g.contiguous() if g is not None else torch.zeros_like(ref) for g in gs]
        if D0 < D:
            gs = [torch.nn.functional.pad(g, (0, D - D0)) for g in gs]
        dx = N.pyramid_bwd(*gs, None, B, S, H, L, p, D)
        return dx[0][..., :D0], dx[1][..., :D0], dx[2][..., :D0], None, None, None, None, None


class _GatheredAttnFn(torch.autograd.Function):
    """Causal attention over rows ``x_cat[b, h, idx[b, h, s]]`` of scorer outputs
    ``[B, H, S_tot, D]`` (any strides, D contiguous), for scorers from elsewhere."""

    @staticmethod
    def _rows(q_cat, k_cat, v_cat):
        # every row lives in the one [B, H, S_tot, D] tensor: rows >= split never occur
        assert k_cat.stride() == q_cat.stride() == v_cat.stride(), "scorer outputs must share strides"
        sb, sh, ss, _ = q_cat.stride()
        st = (sb, ss, sh)
        return N.Rows(q_cat, k_cat, v_cat, st, q_cat, k_cat, v_cat, st, split=q_cat.shape[2],
                      limit=q_cat.shape[2])

    @staticmethod
    def forward(ctx, q_cat, k_cat, v_cat, idx):
        B, H, S_tot, D0 = q_cat.shape
        scale = None
        if D0 < N.D_SUPPORTED:  # zero-padded head dim, scale 1/sqrt(D0)
            q_cat, k_cat, v_cat = (torch.nn.functional.pad(x, (0, N.D_SUPPORTED - D0)) for x in (q_cat, k_cat, v_cat))
            scale = D0 ** -0.5
        D = q_cat.shape[-1]
        rows = _GatheredAttnFn._rows(q_cat, k_cat, v_cat)
        n = idx.shape[-1]
        o, lse = N.attn_fwd(rows, idx, B, H, n, D, scale)
        ctx.save_for_backward(q_cat, k_cat, v_cat, idx, o, lse)
        ctx.geo = (D0, scale)
        return o[..., :D0] if D0 < D else o

    @staticmethod
    def backward(ctx, do):
        q_cat, k_cat, v_cat, idx, o, lse = ctx.saved_tensors
        D0, scale = ctx.geo
        B, H, S_tot, D = q_cat.shape
        rows = _GatheredAttnFn._rows(q_cat, k_cat, v_cat)
        n = idx.shape[-1]
        do = do.contiguous()
        if D0 < D:
            do = torch.nn.functional.pad(do, (0, D - D0))
        delta = (do.float() * o.float()).sum(-1)
        dqs, dks, dvs = N.attn_bwd(rows, idx, B, H, n, do, lse, delta, D, scale)
        inv = N.build_inverse(idx, S_tot)
        # one-level pyramid over S_tot rows: row r receives dsel[inv[r]] (or 0)
        dq, dk, dv = N.pyramid_bwd(dqs, dks, dvs, inv, B, S_tot, H, 1, 2, D)
        return tuple(g.transpose(1, 2)[..., :D0] for g in (dq, dk, dv)) + (None,)


class _ScatterToBaseFn(torch.autograd.Function):
    """``_ScatterToBaseAutograd`` (``src/lighthouse_selection.py:517-576``), gather-formulated."""

    @staticmethod
    def forward(ctx, attn_out, indices, N_shard, N_total, num_levels, pooling_factor, validate):
        _, _, S_tot = N.pyramid_lengths(N_shard, num_levels, pooling_factor)
        idx = indices.to(torch.int32).contiguous()
        if validate:
            # the gather formulation needs each row named at most once per (b, h); -1 marks an
            # empty slot (skipped, as the reference's kernels skip it)
            N.check_indices(idx, -1, S_tot, unique=True, what="scatter_to_base_sequence indices")
        inv = N.build_inverse(idx, S_tot)
        D0 = attn_out.shape[-1]
        if D0 < N.D_SUPPORTED:  # the kernels move 128-wide rows: zero-pad, then cut the columns off
            attn_out = torch.nn.functional.pad(attn_out, (0, N.D_SUPPORTED - D0))
        out = N.scatter_fwd(attn_out, inv, N_shard, N_total, num_levels, pooling_factor)
        ctx.save_for_backward(idx)
        ctx.geo = (N_shard, num_levels, pooling_factor, D0)
        return out[..., :D0] if D0 < N.D_SUPPORTED else out

    @staticmethod
    def backward(ctx, grad_output):
        (idx,) = ctx.saved_tensors
        S, L, p, D0 = ctx.geo
        if D0 < N.D_SUPPORTED:
            grad_output = torch.nn.functional.pad(grad_output, (0, N.D_SUPPORTED - D0))
        dattn, _ = N.scatter_bwd(grad_output, idx, None, S, L, p)
        return (dattn[..., :D0] if D0 < N.D_SUPPORTED else dattn), None, None, None, None, None, None


def scatter_to_base_sequence(attn_out, indices_hp, rank_ids_hp, N_shard: int, N_total: int,
                             num_levels: int, pooling_factor: int, validate: bool = True):
    """Fan-out of selected rows onto the base sequence (``src/lighthouse_selection.py:758-770``).

    Only the single-shard form is built: ``rank_ids_hp`` must be all zeros,
    which is what every reference caller passes (:817, :1045-1046).
    ``attn_out`` must be bfloat16 or float16 (``TypeError`` otherwise).  The fan-out is
    gather-formulated, so every (b, h) must name each pyramid row at most once;
    ``validate`` (default) checks that and the index range on the device and
    raises ``IndexError`` (one stream synchronisation); entries of -1 are empty
    slots, skipped as in the reference."""
    if rank_ids_hp is not None and bool((rank_ids_hp != 0).any()):
        raise NotImplementedError("non-zero rank_ids (sharded fan-out) belong to the context-parallel path, "
                                  "which this single-GPU build does not include")
    N._need_rows("scatter_to_base_sequence attn_out", attn_out)
    return _ScatterToBaseFn.apply(attn_out, indices_hp, N_shard, N_total, num_levels, pooling_factor,
                                  bool(validate))


# ---------------------------------------------------------------------------
# modules
# ---------------------------------------------------------------------------
class DialatedLighthouseNormScorer(nn.Module):
    """Norm scorer (``src/lighthouse_selection.py:578-616``).  Calling it returns the
    reference's 5-tuple; ``LighthouseLocal`` uses the fused native path instead."""

    def __init__(self, pooling_factor: int = 4, levels: int = 3):
        super().__init__()
        self.pooling_factor = pooling_factor
        self.levels = levels

    dilation = 0

    def forward(self, xq, xk, xv):
        return _PyramidCatFn.apply(xq, xk, xv, self.levels, self.pooling_factor, 0)


class DilatedLighthouseScorer(nn.Module):
    """Dilated scorer (``src/lighthouse_selection.py:618-689``).

    ``attention=None`` (default) uses the native causal kernel with a fused
    norm epilogue; a callable is used as in the reference.  ``head_dim`` is
    accepted for the reference builder's call (``lighthouse-attention.patch:623-628``)."""

    def __init__(self, attention=None, dilation: int = 4, pooling_factor: int = 4, levels: int = 3,
                 head_dim: int | None = None):
        super().__init__()
        self.dilation = dilation
        self.pooling_factor = pooling_factor
        self.levels = levels
        self.attention = attention
        self.head_dim = head_dim

    def forward(self, xq, xk, xv):
        if self.attention is None:
            return _PyramidCatFn.apply(xq, xk, xv, self.levels, self.pooling_factor, self.dilation)
        return self._forward_with_attention(xq, xk, xv)

    def _forward_with_attention(self, xq, xk, xv):
        b, s, h, d = xq.shape
        dil = self.dilation

        def virt(x):
            return x.reshape(b, s // dil, dil * h, d).transpose(1, 2)

        with torch.no_grad():  # scores only feed the (non-differentiable) selection
            out_qk = self.attention(virt(xq), virt(xk), virt(xv)).transpose(1, 2).reshape(b, s, h, d)
            out_kq = self.attention(virt(xk), virt(xq), virt(xv)).transpose(1, 2).reshape(b, s, h, d)
            sqk = out_qk.norm(dim=-1).transpose(1, 2).float()
            skq = out_kq.norm(dim=-1).transpose(1, 2).float()
        return _PyramidCatFn.apply(xq, xk, xv, self.levels, self.pooling_factor, 0, sqk, skq)


class DilatedLighthouseGLAScorer(nn.Module):
    """GLA scorer (``src/lighthouse_selection.py:692-755``): the scores are the L2
    norms of two simple gated linear attentions (q->k and k->q, both with v) over
    the dilated virtual heads, gated by ``gk`` [B, S, H] (log gates, e.g.
    ``logsigmoid(wg(x)) / 16``, lighthouse-attention.patch:709), computed by the
    native chunked GLA kernel (the reference calls ``fla``'s ``chunk_simple_gla``).
    Calling it returns the reference's 5-tuple; ``LighthouseLocal`` uses the fused
    native path instead."""

    def __init__(self, head_dim: int, dilation: int = 4, pooling_factor: int = 4, levels: int = 3):
        super().__init__()
        self.head_dim = head_dim
        self.dilation = dilation
        self.pooling_factor = pooling_factor
        self.levels = levels
        self.scaling = 1.0 / math.sqrt(head_dim)

    def forward(self, xq, xk, xv, gk):
        b, s, h, d = xq.shape
        _, _, S_tot = N.pyramid_lengths(s, self.levels, self.pooling_factor)
        with torch.no_grad():
            q, k, v = (x.contiguous() for x in (xq, xk, xv))
            if d < N.D_SUPPORTED:  # zero-padded head dim, as the native layer runs it
                q, k, v = (torch.nn.functional.pad(x, (0, N.D_SUPPORTED - d)) for x in (q, k, v))
            sqk, skq = N.gla_scores(q, k, v, gk.detach(), self.dilation, S_tot, self.scaling)
        return _PyramidCatFn.apply(xq, xk, xv, self.levels, self.pooling_factor, 0, sqk[..., :s], skq[..., :s])


class LighthouseLocal(nn.Module):
    """Selection attention layer (``src/lighthouse_selection.py:772-825``).

    ``forward(xq, xk, xv)`` takes ``[B, S, H, D]`` bf16 and returns ``[B, H, S, D]``."""

    def __init__(self, attention, scorer, num_levels: int = 3, pooling_factor: int = 4, topk: int = 1024,
                 tie_break: str = "reference", strict: bool = True, use_native_attention: bool = True):
        super().__init__()
        self.scorer = scorer
        self.num_levels = num_levels
        self.pooling_factor = pooling_factor
        self.topk = topk
        self.attention = attention
        self.tie_break = tie_break
        self.strict = strict
        self.use_native_attention = use_native_attention
        self.last_indices = None
        # True: the fused path stores its output as [B, S, H, D] and returns the
        # [B, H, S, D] view (same values and shape, strided)
        self.out_seq_major = False

    def _native_dilation(self):
        sc = self.scorer
        if type(sc) is DialatedLighthouseNormScorer:
            return 0
        if type(sc) is DilatedLighthouseScorer and sc.attention is None:
            return sc.dilation
        if type(sc) is DilatedLighthouseGLAScorer:
            return sc.dilation
        return None

    def fuses_rope(self) -> bool:
        """True when ``forward_rope`` applies: the native path with the norm scorer."""
        return self.use_native_attention and self._native_dilation() == 0 and \
            self.scorer.levels == self.num_levels and self.scorer.pooling_factor == self.pooling_factor

    def forward_rope(self, xqkv, freqs, n_heads: int):
        """``forward(rope(q), rope(k), v)`` from the fused ``[q | k | v]`` projection
        output ``xqkv`` [B, S, 3*H*D] and the rotary table ``freqs`` fp32
        [>= S, D/2, 2]; the rotation runs inside the layer's pyramid pass."""
        if not self.fuses_rope():
            raise RuntimeError("forward_rope needs the native layer with the norm scorer")
        out, idx = lighthouse_layer_rope(xqkv, freqs, n_heads, self.num_levels, self.pooling_factor, self.topk,
                                         self.tie_break, self.strict, self.out_seq_major)
        self.last_indices = idx
        return out

    def forward(self, xq, xk, xv, gk=None):
        """``gk`` [B, S, H]: the gate of the GLA scorer (required with it, unused
        otherwise); the reference's caller passes it as ``selection_attn(xq, xk,
        xv, gk=gk)`` (lighthouse-attention.patch:709-710)."""
        _, s, _, d = xq.shape
        gla = isinstance(self.scorer, DilatedLighthouseGLAScorer)
        if gla and gk is None:
            raise ValueError("the GLA scorer needs the gate gk ([B, S, H] log gates)")
        dil = self._native_dilation()
        if self.use_native_attention and dil is not None and \
                self.scorer.levels == self.num_levels and self.scorer.pooling_factor == self.pooling_factor:
            out, idx = lighthouse_layer(xq, xk, xv, self.num_levels, self.pooling_factor, self.topk,
                                        self.tie_break, self.strict, dil, self.out_seq_major,
                                        gk if gla else None)
            self.last_indices = idx
            return out
        # generic composition, as in the reference, for scorers and attentions from elsewhere
        sqk, skq, xq_cat, xk_cat, xv_cat = self.scorer(xq, xk, xv, gk) if gla else self.scorer(xq, xk, xv)
        with torch.no_grad():
            idx = LighthouseSelectionQkKqChunkedTopkHip.forward(
                sqk.to(torch.float32), skq.to(torch.float32), self.num_levels, self.pooling_factor, self.topk, s,
                tie_break=self.tie_break, strict=self.strict)
        self.last_indices = idx
        if self.use_native_attention:
            attn_out = _GatheredAttnFn.apply(xq_cat, xk_cat, xv_cat, idx)
        else:
            gi = idx.long().unsqueeze(-1).expand(-1, -1, -1, d)
            attn_out = self.attention(torch.gather(xq_cat, 2, gi), torch.gather(xk_cat, 2, gi),
                                      torch.gather(xv_cat, 2, gi))
        # indices from this module's selection are unique and in range by construction
        return scatter_to_base_sequence(attn_out, idx, None, s, s, self.num_levels, self.pooling_factor,
                                        validate=False)


class DialatedLighthouseNormScorerCP(nn.Module):
    """Name kept for the reference's imports (``src/lighthouse_selection.py:943-982``);
    context parallelism is not part of this single-GPU build."""

    def __init__(self, pooling_factor: int = 4, levels: int = 3):
        super().__init__()
        self.pooling_factor = pooling_factor
        self.levels = levels

    def forward(self, xq, xk, xv):
        raise NotImplementedError("context-parallel Lighthouse is not part of this single-GPU build")


class LighthouseCP(nn.Module):
    """Name kept for the reference's imports (``src/lighthouse_selection.py:985-1054``)."""

    def __init__(self, attention, scorer, num_levels: int = 3, pooling_factor: int = 4, topk: int = 1024):
        super().__init__()
        self.scorer = scorer
        self.num_levels = num_levels
        self.pooling_factor = pooling_factor
        self.topk = topk
        self.attention = attention
        self._rank, self._world_size, self._cp_group = 0, 1, None

    def set_cp_info(self, rank: int, world_size: int, cp_group):
        self._rank, self._world_size, self._cp_group = rank, world_size, cp_group

    def forward(self, xq, xk, xv):
        raise NotImplementedError("context-parallel Lighthouse is not part of this single-GPU build")
