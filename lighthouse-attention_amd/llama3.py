"""Llama3 transformer with Lighthouse selection attention, for one MI355X.

This is torchtitan's Llama3 model as the Lighthouse patch wires it
(``lighthouse-attention.patch:551-769``), restated for this build: the
attention of every layer runs on the gfx950 kernels of this package — the
Lighthouse layer (``LighthouseLocal``) on the selection layers, the dense
causal kernel (``ScaledDotProductAttention``) on ``lighthouse_full_attn_layers``
and on models without selection.  The rest of the block runs on this
package's kernels too (``block_ops``: fused rotary embedding + q/k/v split,
RMSNorm, SwiGLU); the projections are hipBLASLt GEMMs, fused per input
(``[wq; wk; wv]``, ``[w1; w3]``) with the parameters kept as torchtitan names
them, and weight gradients split along the token axis.

torchtitan itself is not vendored with the reference (upstream dependency; the
patch applies to its ``llama3`` package).  Its unchanged parts are restated
from the published torchtitan source of the patch's base revision:
``precompute_freqs_cis`` with Llama-3.1 frequency scaling, ``apply_rotary_emb``
on interleaved pairs, ``repeat_kv``, ``FeedForward`` (hidden width
``int(2*h/3)`` rounded up to ``multiple_of``), ``nn.RMSNorm`` everywhere, the
depth-scaled truncated-normal initialisation and the block layout.

``Trainer`` is the one-GPU equivalent of torchtitan's step under FSDP mixed
precision (bf16 parameters for compute, fp32 master weights, fp32 gradient
reduction): forward + backward in bf16, cross entropy in fp32, global-norm
clipping and fused AdamW on the fp32 masters (``configs/scorer/norm.toml:25-49``).
"""
from __future__ import annotations

import copy
import math
from dataclasses import dataclass, field

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import block_ops as ops
from .dense_attention import ScaledDotProductAttention
from .lighthouse_selection import (
    DialatedLighthouseNormScorer,
    DialatedLighthouseNormScorerCP,
    DilatedLighthouseGLAScorer,
    DilatedLighthouseScorer,
    LighthouseCP,
    LighthouseLocal,
)

__all__ = [
    "RoPEScalingArgs", "TransformerModelArgs", "llama3_args", "precompute_freqs_cis", "apply_rotary_emb",
    "repeat_kv", "Attention", "FeedForward", "TransformerBlock", "Transformer", "Trainer",
    "ffn_hidden_dim", "num_params", "cast_params_",
]


@dataclass
class RoPEScalingArgs:
    """Llama-3.1 RoPE frequency scaling (torchtitan ``RoPEScalingArgs`` defaults)."""
    scaling_factor: float = 8.0
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    original_max_position_embeddings: int = 8192


@dataclass
class TransformerModelArgs:
    """torchtitan's ``TransformerModelArgs`` with the patch's fields
    (``lighthouse-attention.patch:555-578``).  ``lighthouse_tie_break`` and
    ``lighthouse_strict`` are this build's selection options (see
    ``LighthouseLocal``); their defaults reproduce the reference."""
    dim: int = 4096
    n_layers: int = 32
    n_heads: int = 32
    n_kv_heads: int | None = None
    vocab_size: int = 128256
    multiple_of: int = 256
    ffn_dim_multiplier: float | None = None
    hidden_dim: int | None = None
    norm_eps: float = 1e-5
    rope_theta: float = 10000
    rope_scaling_args: RoPEScalingArgs = field(default_factory=RoPEScalingArgs)

    dilation: int = 4
    max_seq_len: int = 131072
    depth_init: bool = True
    use_flex_attn: bool = False
    attn_mask_type: str = "causal"
    eos_id: int = 0

    use_selection_lighthouse: bool = False
    use_lighthouse_cp: bool = False
    lighthouse_num_levels: int = 3
    lighthouse_pooling_factor: int = 16
    lighthouse_topk: int = 16
    lighthouse_scorer: str = "norm"
    lighthouse_full_attn_layers: list[int] | None = None

    lighthouse_tie_break: str = "reference"
    lighthouse_strict: bool = True

    def update_from_config(self, seq_len: int | None = None, vocab_size: int | None = None) -> None:
        """The parts of torchtitan's ``update_from_config`` a model needs: the
        tokenizer's vocabulary and a ``max_seq_len`` covering the training length."""
        if vocab_size is not None:
            self.vocab_size = int(vocab_size)
        if seq_len is not None and seq_len > self.max_seq_len:
            self.max_seq_len = int(seq_len)


# The patch's flavors (``lighthouse-attention.patch:77-533``).  Every 270M
# Lighthouse flavor shares the same trunk and differs in (levels, pooling,
# top-k, full-attention layers, context parallel); that table is kept here as
# data.  Upstream's 70B/405B entries, which the patch leaves in place, are
# not part of this build.
_TRUNK_270M = dict(dim=1024, n_layers=30, hidden_dim=1536, n_heads=8, n_kv_heads=8, rope_theta=10000)
_FULL = [0, 1, 28, 29]
_LIGHTHOUSE_270M = {
    # name: (levels, pooling, topk, context-parallel, full-attention layers)
    "ablation_270m_lighthouse": (2, 2, 8192, False, _FULL),
    "ablation_270m_lighthouse_topk4096": (2, 2, 4096, False, _FULL),
    "ablation_270m_lighthouse_topk8192": (2, 2, 8192, False, _FULL),
    "ablation_270m_lighthouse_topk16384": (2, 2, 16384, False, _FULL),
    "ablation_270m_lighthouse_topk8192_pool4": (2, 4, 8192, False, _FULL),
    "ablation_270m_lighthouse_topk4096_pool4": (2, 4, 4096, False, _FULL),
    "ablation_270m_lighthouse_topk2048_pool4": (2, 4, 2048, False, _FULL),
    "ablation_270m_lighthouse_topk8192_lvl3": (3, 2, 8192, False, _FULL),
    "ablation_270m_lighthouse_topk4096_lvl3": (3, 2, 4096, False, _FULL),
    "ablation_270m_lighthouse_topk1536_lvl3": (3, 2, 1536, False, _FULL),
    "ablation_270m_lighthouse_topk2048_lvl3": (3, 2, 2048, False, _FULL),
    "ablation_270m_lighthouse_topk3072_lvl3": (3, 2, 3072, False, _FULL),
    "ablation_270m_lighthouse_topk6144_lvl3": (3, 2, 6144, False, _FULL),
    "ablation_270m_lighthouse_topk2048_pool4_lvl3": (3, 4, 2048, False, _FULL),
    "ablation_270m_lighthouse_topk1536_pool4_lvl3": (3, 4, 1536, False, _FULL),
    "ablation_270m_lighthouse_topk4096_pool4_lvl3_cp": (3, 4, 4096, True, _FULL),
    "ablation_270m_lighthouse_topk4096_pool4_lvl4_cp_1m": (4, 4, 4096, True, []),
    "ablation_270m_lighthouse_topk6144_pool4_lvl4_cp": (4, 4, 6144, True, _FULL),
    "ablation_270m_lighthouse_topk16384_pool4_lvl3_cp": (3, 4, 16384, True, _FULL),
    "ablation_270m_lighthouse_topk1536_pool4_lvl3_cp": (3, 4, 1536, True, _FULL),
    "ablation_270m_lighthouse_topk2048_pool4_lvl3_cp": (3, 4, 2048, True, _FULL),
    "ablation_270m_lighthouse_topk1536_pool8_lvl3": (3, 8, 1536, False, _FULL),
    "ablation_270m_lighthouse_topk768_pool4_lvl3": (3, 4, 768, False, _FULL),
    "ablation_270m_lighthouse_topk768_pool8_lvl3": (3, 8, 768, False, _FULL),
    "ablation_270m_lighthouse_topk2048_lvl4": (4, 2, 2048, False, _FULL),
    "ablation_270m_lighthouse_topk1536_lvl4": (4, 2, 1536, False, _FULL),
    "ablation_270m_lighthouse_topk2048_lvl5": (5, 2, 2048, False, _FULL),
    "ablation_270m_lighthouse_topk1536_lvl5": (5, 2, 1536, False, _FULL),
}

llama3_args: dict[str, TransformerModelArgs] = {
    "ablation_270m": TransformerModelArgs(dim=576, n_layers=30, hidden_dim=1536, n_heads=8, n_kv_heads=8,
                                          rope_theta=10000),
    "ablation_270m_topk1536_pool4_lvl3_sdpa": TransformerModelArgs(**_TRUNK_270M),
    "ablation_2b": TransformerModelArgs(dim=2048, n_layers=24, hidden_dim=8192, n_heads=32, n_kv_heads=32,
                                        rope_theta=10000),
    "llama_8b": TransformerModelArgs(dim=4096, n_layers=32, hidden_dim=14336, n_heads=32, n_kv_heads=8,
                                     rope_theta=10000),
}
for _name, (_lv, _pf, _k, _cp, _full) in _LIGHTHOUSE_270M.items():
    llama3_args[_name] = TransformerModelArgs(
        **_TRUNK_270M, use_selection_lighthouse=True, use_lighthouse_cp=_cp, lighthouse_num_levels=_lv,
        lighthouse_pooling_factor=_pf, lighthouse_topk=_k, dilation=4, lighthouse_full_attn_layers=list(_full))


# ---------------------------------------------------------------------------
# rotary embedding
# ---------------------------------------------------------------------------
def precompute_freqs_cis(dim: int, end: int, theta: float = 10000.0,
                         scaling_args: RoPEScalingArgs = RoPEScalingArgs()) -> torch.Tensor:
    """``exp(i * t * f_j)`` for ``t < end``, ``j < dim/2`` (complex64 ``[end, dim/2]``).

    ``f_j = theta^(-2j/dim)``, then the Llama-3.1 rule on wavelength ``w = 2*pi/f``:
    ``w < L/high`` kept, ``w > L/low`` divided by ``scaling_factor``, and in between
    ``(1-s) f/scaling_factor + s f`` with ``s = (L/w - low)/(high - low)``
    (L = ``original_max_position_embeddings``)."""
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2)[: dim // 2].float() / dim))
    sf, lo, hi = scaling_args.scaling_factor, scaling_args.low_freq_factor, scaling_args.high_freq_factor
    L0 = scaling_args.original_max_position_embeddings
    wavelen = 2 * math.pi / freqs
    high_w, low_w = L0 / hi, L0 / lo
    freqs = torch.where(wavelen > low_w, freqs / sf, freqs)
    smooth = (L0 / wavelen - lo) / (hi - lo)
    smoothed = (1 - smooth) * freqs / sf + smooth * freqs
    medium = ~(wavelen < high_w) & ~(wavelen > low_w)
    freqs = torch.where(medium, smoothed, freqs)
    t = torch.arange(end, device=freqs.device)
    ang = torch.outer(t, freqs).float()
    return torch.polar(torch.ones_like(ang), ang)


def apply_rotary_emb(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor):
    """Rotate adjacent pairs ``(x[2j], x[2j+1])`` of ``[B, S, H, D]`` q and k by the
    position's angle, in fp32, and round back to the input dtype."""
    S = xq.shape[1]
    fc = freqs_cis[:S].view(1, S, 1, -1)
    q_ = torch.view_as_complex(xq.float().reshape(*xq.shape[:-1], -1, 2))
    k_ = torch.view_as_complex(xk.float().reshape(*xk.shape[:-1], -1, 2))
    return (torch.view_as_real(q_ * fc).flatten(3).type_as(xq),
            torch.view_as_real(k_ * fc).flatten(3).type_as(xk))


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """``[B, S, KVH, D] -> [B, S, KVH*n_rep, D]``, each kv head repeated ``n_rep`` times."""
    if n_rep == 1:
        return x
    b, s, kvh, d = x.shape
    return x[:, :, :, None, :].expand(b, s, kvh, n_rep, d).reshape(b, s, kvh * n_rep, d)


# ---------------------------------------------------------------------------
# modules
# ---------------------------------------------------------------------------
def _build_lighthouse_scorer(args: TransformerModelArgs, head_dim: int):
    """Scorer by name, as ``lighthouse-attention.patch:34-71``: returns (scorer, needs_gate)."""
    name = (args.lighthouse_scorer or "norm").lower()
    if args.use_lighthouse_cp and name != "norm":
        raise ValueError(f"lighthouse_scorer='{name}' is not supported under context parallelism; "
                         "set lighthouse_scorer='norm' or disable use_lighthouse_cp.")
    common = dict(pooling_factor=args.lighthouse_pooling_factor, levels=args.lighthouse_num_levels)
    if name == "norm":
        cls = DialatedLighthouseNormScorerCP if args.use_lighthouse_cp else DialatedLighthouseNormScorer
        return cls(**common), False
    if name == "dilated":
        return DilatedLighthouseScorer(head_dim=head_dim, dilation=args.dilation, **common), False
    if name == "gla":
        return DilatedLighthouseGLAScorer(head_dim=head_dim, dilation=args.dilation, **common), True
    raise ValueError(f"Unknown lighthouse_scorer={name!r}; expected one of {{'norm', 'dilated', 'gla'}}.")


class Attention(nn.Module):
    """Multi-head attention block (torchtitan ``Attention`` + ``lighthouse-attention.patch:245-360``)."""

    def __init__(self, args: TransformerModelArgs):
        super().__init__()
        if args.use_flex_attn:
            raise NotImplementedError("flex attention (block-causal document masks) is not part of this build")
        self.n_heads = args.n_heads
        self.n_kv_heads = args.n_heads if args.n_kv_heads is None else args.n_kv_heads
        self.n_rep = self.n_heads // self.n_kv_heads
        self.head_dim = args.dim // args.n_heads
        self.wq = nn.Linear(args.dim, args.n_heads * self.head_dim, bias=False)
        self.wk = nn.Linear(args.dim, self.n_kv_heads * self.head_dim, bias=False)
        self.wv = nn.Linear(args.dim, self.n_kv_heads * self.head_dim, bias=False)
        self.wo = nn.Linear(args.n_heads * self.head_dim, args.dim, bias=False)
        self.use_flex_attn = False
        self.inner_attention = ScaledDotProductAttention()

        self.use_selection_lighthouse = args.use_selection_lighthouse
        self.use_lighthouse_cp = args.use_lighthouse_cp
        self._use_lighthouse = self.use_selection_lighthouse
        self.pooling_factor = args.lighthouse_pooling_factor
        self.num_levels = args.lighthouse_num_levels
        self.topk = args.lighthouse_topk
        self.dilation = args.dilation
        self.scorer, self._needs_gate = _build_lighthouse_scorer(args, self.head_dim)
        if self._needs_gate:
            self.wg = nn.Linear(args.dim, self.n_heads, bias=True)
            self.gate_logit_normalizer = 16
        if self.use_lighthouse_cp:
            self.selection_attn = LighthouseCP(attention=self.inner_attention, scorer=self.scorer,
                                               num_levels=self.num_levels, pooling_factor=self.pooling_factor,
                                               topk=self.topk)
        else:
            self.selection_attn = LighthouseLocal(scorer=self.scorer, num_levels=self.num_levels,
                                                  pooling_factor=self.pooling_factor, topk=self.topk,
                                                  attention=self.inner_attention,
                                                  tie_break=args.lighthouse_tie_break,
                                                  strict=args.lighthouse_strict)
            # the output goes straight into wo: store it sequence-major, so the
            # transpose below is free in both directions
            self.selection_attn.out_seq_major = True

    def init_weights(self, init_std: float):
        for lin in (self.wq, self.wk, self.wv):
            nn.init.trunc_normal_(lin.weight, mean=0.0, std=0.02)
        nn.init.trunc_normal_(self.wo.weight, mean=0.0, std=init_std)
        if self._needs_gate:
            nn.init.trunc_normal_(self.wg.weight, mean=0.0, std=0.02)
            nn.init.zeros_(self.wg.bias)

    def _fuses_rope(self) -> bool:
        return (not self._needs_gate and self.n_kv_heads == self.n_heads and self.head_dim == 128
                and isinstance(self.selection_attn, LighthouseLocal) and self.selection_attn.fuses_rope())

    def set_use_lighthouse(self, use_lighthouse: bool):
        self._use_lighthouse = use_lighthouse

    def set_cp_info(self, rank: int, world_size: int, cp_group):
        if self.use_lighthouse_cp:
            self.selection_attn.set_cp_info(rank, world_size, cp_group)

    def forward(self, x: torch.Tensor, freqs_cis: torch.Tensor, attention_masks=None):
        bs, seqlen, _ = x.shape
        # one projection GEMM for [q | k | v]; rotary embedding and the split in one pass
        wqkv = torch.cat([self.wq.weight, self.wk.weight, self.wv.weight])
        xqkv = ops.linear(x, wqkv)
        if attention_masks is not None:
            raise NotImplementedError("document masks need flex attention, which is not part of this build")
        lighthouse = self.use_selection_lighthouse and self._use_lighthouse
        if lighthouse and self._fuses_rope():
            # the norm-scorer layer rotates q and k inside its pyramid pass
            out = self.selection_attn.forward_rope(xqkv, torch.view_as_real(freqs_cis), self.n_heads)
            out = out.transpose(1, 2).contiguous().view(bs, seqlen, -1)
            return ops.linear(out, self.wo.weight)
        xq, xk, xv = ops.rope_qkv(xqkv, torch.view_as_real(freqs_cis), self.n_heads, self.n_kv_heads, self.head_dim)
        if lighthouse:
            if self._needs_gate:
                gk = F.logsigmoid(self.wg(x)) / self.gate_logit_normalizer
                out = self.selection_attn(xq, xk, xv, gk=gk)
            else:
                out = self.selection_attn(xq, xk, xv)
        else:
            keys = repeat_kv(xk, self.n_rep)
            values = repeat_kv(xv, self.n_rep)
            out = self.inner_attention(xq.transpose(1, 2), keys.transpose(1, 2), values.transpose(1, 2))
        out = out.transpose(1, 2).contiguous().view(bs, seqlen, -1)
        return ops.linear(out, self.wo.weight)


def _eps(norm: nn.RMSNorm, x: torch.Tensor) -> float:
    return norm.eps if norm.eps is not None else torch.finfo(x.dtype).eps


def ffn_hidden_dim(hidden_dim: int, multiple_of: int, ffn_dim_multiplier: float | None) -> int:
    """torchtitan ``FeedForward`` width: ``int(2*h/3)``, times the multiplier, rounded
    up to ``multiple_of``.  The patch passes ``hidden_dim`` through this rule
    (``lighthouse-attention.patch:745-753``), so ``hidden_dim=1536`` builds 1024."""
    h = int(2 * hidden_dim / 3)
    if ffn_dim_multiplier is not None:
        h = int(ffn_dim_multiplier * h)
    return multiple_of * ((h + multiple_of - 1) // multiple_of)


class FeedForward(nn.Module):
    """SwiGLU MLP ``w2(silu(w1 x) * w3 x)``."""

    def __init__(self, dim: int, hidden_dim: int, multiple_of: int, ffn_dim_multiplier: float | None):
        super().__init__()
        h = ffn_hidden_dim(hidden_dim, multiple_of, ffn_dim_multiplier)
        self.w1 = nn.Linear(dim, h, bias=False)
        self.w2 = nn.Linear(h, dim, bias=False)
        self.w3 = nn.Linear(dim, h, bias=False)

    def forward(self, x):
        # [h1 | h3] from one GEMM, then silu(h1) * h3 in one pass
        h = ops.linear(x, torch.cat([self.w1.weight, self.w3.weight]))
        return ops.linear(ops.swiglu(h), self.w2.weight)

    def init_weights(self, init_std: float):
        nn.init.trunc_normal_(self.w1.weight, mean=0.0, std=0.02)
        for lin in (self.w2, self.w3):
            nn.init.trunc_normal_(lin.weight, mean=0.0, std=init_std)


class TransformerBlock(nn.Module):
    def __init__(self, layer_id: int, args: TransformerModelArgs):
        super().__init__()
        self.n_heads = args.n_heads
        self.dim = args.dim
        self.attention = Attention(args)
        ffn_hidden = args.hidden_dim if args.hidden_dim is not None else 4 * args.dim
        self.feed_forward = FeedForward(args.dim, ffn_hidden, args.multiple_of, args.ffn_dim_multiplier)
        self.attention_norm = ops.RMSNorm(args.dim, eps=args.norm_eps)
        self.ffn_norm = ops.RMSNorm(args.dim, eps=args.norm_eps)
        if args.depth_init:
            self.weight_init_std = 0.02 / (2 * (layer_id + 1)) ** 0.5
        else:
            self.weight_init_std = 0.02 / (2 * args.n_layers) ** 0.5

    def forward(self, x, freqs_cis, attention_masks=None):
        a = self.attention(self.attention_norm(x), freqs_cis, attention_masks)
        h, y = ops.add_rms_norm(x, a, self.ffn_norm.weight, _eps(self.ffn_norm, x))
        return h + self.feed_forward(y)

    def forward_fused(self, h, y, freqs_cis, next_norm, attention_masks=None):
        """The block on a residual stream ``h`` whose ``attention_norm(h)`` is already
        ``y``; returns ``(h_out, next_norm(h_out))`` with both residual adds fused
        into the norms that read them."""
        a = self.attention(y, freqs_cis, attention_masks)
        h, y2 = ops.add_rms_norm(h, a, self.ffn_norm.weight, _eps(self.ffn_norm, h))
        return ops.add_rms_norm(h, self.feed_forward(y2), next_norm.weight, _eps(next_norm, h))

    def init_weights(self):
        for norm in (self.attention_norm, self.ffn_norm):
            norm.reset_parameters()
        self.attention.init_weights(self.weight_init_std)
        self.feed_forward.init_weights(self.weight_init_std)


class Transformer(nn.Module):
    """Token embedding, ``n_layers`` blocks, final RMSNorm and output projection;
    ``lighthouse_full_attn_layers`` switch Lighthouse off on the listed layers
    (``lighthouse-attention.patch:508-519``)."""

    def __init__(self, args: TransformerModelArgs):
        super().__init__()
        self.model_args = args
        self.vocab_size = args.vocab_size
        self.n_layers = args.n_layers
        self.tok_embeddings = nn.Embedding(args.vocab_size, args.dim)
        self.register_buffer("freqs_cis", self._precompute_freqs_cis(), persistent=True)
        self.layers = nn.ModuleDict()
        for layer_id in range(args.n_layers):
            self.layers[str(layer_id)] = TransformerBlock(layer_id, args)
        self._full_attn_layers: set[str] = set()
        for layer_id in args.lighthouse_full_attn_layers or []:
            key = str(layer_id)
            if key in self.layers:
                self.layers[key].attention.set_use_lighthouse(False)
                self._full_attn_layers.add(key)
        self.norm = ops.RMSNorm(args.dim, eps=args.norm_eps)
        self.output = nn.Linear(args.dim, args.vocab_size, bias=False)

    def _precompute_freqs_cis(self):
        a = self.model_args
        return precompute_freqs_cis(a.dim // a.n_heads, a.max_seq_len, a.rope_theta, a.rope_scaling_args)

    def init_weights(self, buffer_device: torch.device | None = None):
        dev = buffer_device or self.freqs_cis.device
        with torch.device(dev):
            self.freqs_cis = self._precompute_freqs_cis()
        nn.init.normal_(self.tok_embeddings.weight)
        for layer in self.layers.values():
            layer.init_weights()
        self.norm.reset_parameters()
        std = self.model_args.dim ** -0.5
        nn.init.trunc_normal_(self.output.weight, mean=0.0, std=std, a=-3 * std, b=3 * std)

    def forward(self, tokens: torch.Tensor, attention_masks=None):
        h = self.tok_embeddings(tokens)
        blocks = list(self.layers.values())
        if not blocks:
            return ops.linear(self.norm(h), self.output.weight)
        # each residual add runs inside the RMSNorm that reads its result (the next
        # block's attention_norm, or the final norm)
        y = blocks[0].attention_norm(h)
        for i, layer in enumerate(blocks):
            nxt = blocks[i + 1].attention_norm if i + 1 < len(blocks) else self.norm
            h, y = layer.forward_fused(h, y, self.freqs_cis, nxt, attention_masks)
        return ops.linear(y, self.output.weight)


def cast_params_(model: nn.Module, dtype: torch.dtype) -> nn.Module:
    """Cast the parameters only (``Module.to(dtype)`` would also turn the complex
    ``freqs_cis`` buffer real)."""
    for p in model.parameters():
        p.data = p.data.to(dtype)
    return model


def num_params(model: nn.Module, exclude_embedding: bool = False) -> int:
    n = sum(p.numel() for p in model.parameters())
    if exclude_embedding:
        n -= model.tok_embeddings.weight.numel()
    return n


# ---------------------------------------------------------------------------
# training step
# ---------------------------------------------------------------------------
class Trainer:
    """One-GPU training step with FSDP-style mixed precision.

    ``master`` holds fp32 parameters and the AdamW state; ``model`` is its bf16
    copy that runs forward and backward.  A step: refresh the bf16 weights from
    the masters, forward, fp32 cross entropy (mean over tokens), backward, bf16
    gradients widened to the masters' fp32 ``.grad``, global-norm clip, fused
    AdamW, linear warm-up of the learning rate (torchtitan's ``warmup_steps``
    schedule, factor ``(step+1)/(warmup+1)``)."""

    def __init__(self, args: TransformerModelArgs, device, lr: float = 2e-3, betas=(0.9, 0.95), eps: float = 1e-8,
                 weight_decay: float = 0.1, max_norm: float = 1.0, warmup_steps: int = 2000, seed: int = 0):
        device = torch.device(device)
        torch.manual_seed(seed)
        with torch.device(device):
            self.master = Transformer(args)
        self.master.init_weights(device)
        self.model = cast_params_(copy.deepcopy(self.master), torch.bfloat16)
        self._mp = list(self.master.parameters())
        self._bp = list(self.model.parameters())
        for p in self._mp:  # fp32 gradient buffers, overwritten every step
            p.grad = torch.zeros_like(p)
        self.optimizer = torch.optim.AdamW(self._mp, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                                           fused=device.type == "cuda")
        self.base_lr = lr
        self.warmup_steps = warmup_steps
        self.max_norm = max_norm
        self.step_count = 0

    def _lr(self) -> float:
        if self.step_count < self.warmup_steps:
            return self.base_lr * (self.step_count + 1) / (self.warmup_steps + 1)
        return self.base_lr

    def step(self, tokens: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
        with torch.no_grad():
            torch._foreach_copy_(self._bp, self._mp)
        logits = self.model(tokens)
        loss = F.cross_entropy(logits.flatten(0, 1).float(), labels.flatten(0, 1))
        loss.backward()
        with torch.no_grad():
            torch._foreach_copy_([p.grad for p in self._mp], [p.grad for p in self._bp])
            grad_norm = torch.nn.utils.clip_grad_norm_(self._mp, self.max_norm, foreach=True)
        for group in self.optimizer.param_groups:
            group["lr"] = self._lr()
        self.optimizer.step()
        for p in self._bp:
            p.grad = None
        self.step_count += 1
        self.last_grad_norm = grad_norm
        return loss.detach()
