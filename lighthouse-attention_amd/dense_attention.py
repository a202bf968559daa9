"""Dense causal attention on the native kernels (the full-attention layers).

The reference model keeps plain causal SDPA on its ``lighthouse_full_attn_layers``
(``lighthouse-attention.patch:759-765``, e.g. layers 0, 1, 28, 29 of the 270M
flavors, ``lighthouse-attention.patch:283-296``): ``Attention.forward`` then calls
``self.inner_attention(xq, xk, xv)`` (torchtitan's ``ScaledDotProductAttentionWrapper``,
causal, scale 1/sqrt(D)) on ``[B, H, S, D]`` transposed views
(``lighthouse-attention.patch:707-724``).  Here the same call runs the gfx950
attention kernels of the Lighthouse layer with the identity row map: the inputs
are read in place through their strides (no copy of the transposed views), the
forward writes O and the exp2-domain LSE, and the backward is the deterministic
dK/dV + dQ pair.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _native as N
from .block_ops import graph_break
from .lighthouse_selection import _mark

__all__ = ["dense_causal_attention", "ScaledDotProductAttention"]


def _rows(q, k, v):
    # [B, H, S, D] views with D contiguous; the kernels take (batch, seq, head) strides
    sb, sh, ss, sd = q.stride()
    if sd != 1 or k.stride() != q.stride() or v.stride() != q.stride():
        raise ValueError("q, k, v must share strides with the head dimension contiguous")
    return N.Rows(q, k, v, (sb, ss, sh))


class _DenseCausalFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, scale):
        B, H, S, D = q.shape
        _mark("dense_fwd_start")
        o, lse = N.attn_fwd(_rows(q, k, v), None, B, H, S, D, scale)
        _mark("dense_attn_fwd")
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale = scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        B, H, S, D = q.shape
        do = do.contiguous()
        # softmax-backward row term delta = rowsum(dO * O), accumulated in fp32
        delta = torch.linalg.vecdot(do.float(), o.float())
        _mark("dense_bwd_start")
        dq, dk, dv = N.attn_bwd(_rows(q, k, v), None, B, H, S, do, lse, delta, D, ctx.scale)
        _mark("dense_attn_bwd")
        return dq, dk, dv, None


@graph_break
def dense_causal_attention(q, k, v):
    """Causal softmax attention, scale 1/sqrt(D): ``q, k, v`` bf16 or fp16 ``[B, H, S, D]``
    (any batch/head/seq strides, D contiguous) -> ``[B, H, S, D]``.  D < 128 (a
    multiple of 8) runs zero-padded to the kernels' 128 with scale 1/sqrt(D)."""
    D = q.shape[-1]
    if D > N.D_SUPPORTED or D % 8:
        raise ValueError(f"head_dim must be a multiple of 8 and at most {N.D_SUPPORTED}, got {D}")
    if not (q.shape == k.shape == v.shape):
        raise ValueError("q, k and v must have the same shape")
    for t in (q, k, v):
        if t.dtype not in N.ROW_DTYPES or t.dtype != q.dtype:
            raise TypeError("the native attention computes in bfloat16 or float16 (one dtype for q, k, v); got "
                            + ", ".join(str(x.dtype) for x in (q, k, v)))
    if D < N.D_SUPPORTED:
        q, k, v = (torch.nn.functional.pad(x, (0, N.D_SUPPORTED - D)) for x in (q, k, v))
        return _DenseCausalFn.apply(q, k, v, D ** -0.5)[..., :D]
    return _DenseCausalFn.apply(q, k, v, None)


class ScaledDotProductAttention(nn.Module):
    """Drop-in for torchtitan's ``ScaledDotProductAttentionWrapper`` with the causal
    mask type: ``forward(xq, xk, xv)`` on ``[B, H, S, D]``."""

    def forward(self, xq, xk, xv, scale=None):
        if scale is not None and abs(scale - xq.shape[-1] ** -0.5) > 1e-12:
            raise NotImplementedError("only the default scale 1/sqrt(head_dim) is supported")
        return dense_causal_attention(xq, xk, xv)
