"""Autograd ops of the Llama3 block around the attention, on the native kernels.

Each op replaces a torch chain of torchtitan's llama3 model (upstream, not
vendored with the reference; its wiring is ``lighthouse-attention.patch:583-769``):

- ``linear``: ``F.linear`` with a weight gradient split along the token axis
  (fp32 partial products summed, then rounded once), so the long-K weight
  gradients of a 32K-token step fill the GPU.
- ``rope_qkv``: ``apply_rotary_emb`` on ``wq(x)``, ``wk(x)`` plus the split of
  ``wv(x)``, from one fused ``[q | k | v]`` projection output.
- ``rms_norm``: ``nn.RMSNorm``; ``add_rms_norm``: a residual add and the RMSNorm
  that reads its result, in one pass each way.
- ``swiglu``: ``F.silu(w1(x)) * w3(x)`` from one fused ``[h1 | h3]`` projection.

There is no CPU path: every op raises without the GPU library.  Under
``torch.compile`` each op is a graph break (``torch.compiler.disable``), as the
reference keeps its own native calls out of the graph; the Lighthouse layer
itself is a traceable custom op.
"""
from __future__ import annotations

import functools

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as N

__all__ = ["linear", "rope_qkv", "rms_norm", "add_rms_norm", "swiglu", "RMSNorm", "wgrad_splits"]


def graph_break(fn):
    """Run ``fn`` as a graph break under ``torch.compile`` (``torch.compiler.disable``)
    and as a plain call otherwise (no per-call wrapper cost in eager mode)."""
    disabled = torch.compiler.disable(fn)

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        if torch.compiler.is_compiling():
            return disabled(*args, **kwargs)
        return fn(*args, **kwargs)

    return wrapper


def wgrad_splits(T: int, O: int, I: int, cus: int = 256) -> int:
    """Number of token slices for the weight gradient ``dy^T x`` ([O, I], K = T).

    Slices x 256x256 output tiles should reach the CU count when the gradient has
    few tiles and half of it otherwise, with slices of >= 2048 tokens and at most 8
    slices (more only adds fp32 partial traffic).  Measured on MI355X at T = 32768:
    1024x1024 -> 8 (77 us), 2048x1024 -> 8 (126 us), 3072x1024 -> 4 (191 us)."""
    tiles = -(-O // 256) * -(-I // 256)
    target = cus if tiles <= 32 else cus // 2
    s = 1
    while tiles * s < target and s < 8 and T % (2 * s) == 0 and T // (2 * s) >= 2048:
        s *= 2
    return s


def _wgrad(dy2, x2):
    T, O = dy2.shape
    I = x2.shape[1]
    s = wgrad_splits(T, O, I)
    if s == 1:
        return dy2.t() @ x2
    part = torch.bmm(dy2.view(s, T // s, O).transpose(1, 2), x2.view(s, T // s, I), out_dtype=torch.float32)
    if (O * I) % 8 == 0:
        return N.splitk_sum(part)
    return part.sum(0).to(dy2.dtype)


class _LinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return F.linear(x, w)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1])
        dx = (dy2 @ w).view(x.shape) if ctx.needs_input_grad[0] else None
        dw = _wgrad(dy2, x.reshape(-1, x.shape[-1])) if ctx.needs_input_grad[1] else None
        return dx, dw


def _need_bf16(*ts):
    for t in ts:
        if not t.is_cuda:
            raise N.LighthouseHipError("block ops need GPU tensors (no CPU path)")
        if t.dtype != torch.bfloat16:
            raise TypeError(f"block ops compute in bfloat16; got {t.dtype}")


@graph_break
def linear(x, w):
    """``x @ w^T`` (bf16, no bias)."""
    _need_bf16(x, w)
    return _LinearFn.apply(x, w)


class _RopeQKVFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, freqs, Hq, Hkv, D):
        ctx.save_for_backward(freqs)
        ctx.geo = (Hq, Hkv, D)
        return N.rope_qkv_fwd(x, freqs, Hq, Hkv, D)

    @staticmethod
    def backward(ctx, dq, dk, dv):
        (freqs,) = ctx.saved_tensors
        Hq, Hkv, D = ctx.geo
        ref = next(g for g in (dq, dk, dv) if g is not None)
        B, S = ref.shape[:2]

        def z(g, h):
            if g is None:
                return torch.zeros(B, S, h, D, dtype=torch.bfloat16, device=ref.device)
            return g if g.stride(3) == 1 else g.contiguous()

        return N.rope_qkv_bwd(z(dq, Hq), z(dk, Hkv), z(dv, Hkv), freqs, Hq, Hkv, D), None, None, None, None


@graph_break
def rope_qkv(x, freqs, Hq: int, Hkv: int, D: int):
    """Fused projection output ``x`` [B, S, (Hq+2Hkv)*D] -> rotated q, rotated k, v,
    each [B, S, H, D] contiguous.  ``freqs``: fp32 [>=S, D/2, 2] (cos, sin), e.g.
    ``torch.view_as_real(freqs_cis)``."""
    _need_bf16(x)
    return _RopeQKVFn.apply(x, freqs, Hq, Hkv, D)


class _RMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, eps):
        x = x.contiguous()  # the backward reads the same rows the forward normalised
        y, rstd = N.rmsnorm_fwd(x, w, eps)
        ctx.save_for_backward(x, w, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, rstd = ctx.saved_tensors
        dx, dw = N.rmsnorm_bwd(dy, x, w, rstd)
        return dx, dw, None


@graph_break
def rms_norm(x, w, eps: float):
    _need_bf16(x, w)
    return _RMSNormFn.apply(x, w, eps)


class _AddRMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, r, w, eps):
        h, y, rstd = N.add_rmsnorm_fwd(x, r, w, eps)
        ctx.save_for_backward(h, w, rstd)
        return h, y

    @staticmethod
    def backward(ctx, dh, dy):
        h, w, rstd = ctx.saved_tensors
        if dy is None:
            return dh, dh, None, None
        dx, dw = N.rmsnorm_bwd(dy, h, w, rstd, dres=dh)
        return dx, dx, dw, None


@graph_break
def add_rms_norm(x, r, w, eps: float):
    """``h = x + r`` and ``RMSNorm(h)`` in one pass: returns ``(h, y)``."""
    _need_bf16(x, r, w)
    return _AddRMSNormFn.apply(x, r, w, eps)


class RMSNorm(nn.RMSNorm):
    """``nn.RMSNorm`` (same parameters and state dict) running the native kernels."""

    def forward(self, x):
        return rms_norm(x, self.weight, self.eps if self.eps is not None else torch.finfo(x.dtype).eps)


class _SwiGLUFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h):
        h = h.contiguous()
        ctx.save_for_backward(h)
        return N.swiglu_fwd(h)

    @staticmethod
    def backward(ctx, da):
        (h,) = ctx.saved_tensors
        return N.swiglu_bwd(da, h)


@graph_break
def swiglu(h):
    """``[h1 | h3]`` (last dim 2F) -> ``silu(h1) * h3``."""
    _need_bf16(h)
    return _SwiGLUFn.apply(h)
