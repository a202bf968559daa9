"""CPU oracle for the Lighthouse selection-attention layer.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg use it, and only as the checker (or as the timed CPU restatement).

It restates, on the CPU, what the reference computes for one Lighthouse layer
(all citations are relative to the reference repository root):

=====================================  =============================================
function here                          reference it restates
=====================================  =============================================
``level_lengths`` / ``level_offsets``  ``src/lighthouse_selection.py:601-614`` (cat order)
                                       ``src/lighthouse_selection_cuda.py:163-175``
``compute_output_indices_selection``   ``src/lighthouse_selection_cuda.py:346-357``
``tile_geometry``                      ``src/lighthouse_selection_cuda.py:370-397``
``bitonic_sort128``                    ``src/lighthouse_selection_cuda.py:41-110``
``select_indices``                     ``src/lighthouse_selection_cuda.py:114-331,399-427``
``norm_scorer``                        ``src/lighthouse_selection.py:589-616``
``dilated_scorer``                     ``src/lighthouse_selection.py:635-689``
``gla_scorer``, ``simple_gla``         ``src/lighthouse_selection.py:692-755`` (+ fla's
                                       ``chunk_simple_gla``, restated from its
                                       published recurrence)
``sdpa_causal``                        ``src/lighthouse_selection.py:815`` (causal SDPA)
``scatter_fwd`` / ``scatter_bwd``      ``src/lighthouse_selection.py:408-514,517-576``
``lighthouse_layer``                   ``src/lighthouse_selection.py:789-825``
=====================================  =============================================

Integer/index work (geometry, the selection network, key ordering) is numpy;
floating-point work (scorers, attention, scatter, autograd for the backward)
is PyTorch on the CPU in float32/float64.

How each function is pinned (checked against something other than itself) is
listed in ``tests/test_oracle.py``; the selection is additionally cross-checked
against the slot-literal C restatement in ``oracle/select_ref.c``.

Tie semantics.  ``tie="reference"`` is the reference network: compare-exchange
on strict inequality only, so tied scores keep their network positions.
``tie="lower_index"`` orders by (score descending, level-local index
ascending); on distinct scores both modes agree.

Domain.  Scores must be finite and greater than -1e6 (the reference's own
"empty" sentinel, ``src/lighthouse_selection_cuda.py:191,227``).  Norm scores
are >= 0, so every scorer output is in the domain.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

try:  # torch is only needed by the floating-point half of the oracle
    import torch
    import torch.nn.functional as F
except Exception:  # pragma: no cover - torch is present in this image
    torch = None
    F = None

SENTINEL = np.float32(-1e6)
TOPK_PER_TILE = 128
HALF = 64


# --------------------------------------------------------------------------
# geometry
# --------------------------------------------------------------------------
def level_lengths(S: int, L: int, p: int) -> list[int]:
    """Length of pyramid level l=1..L: ``S // p**(l-1)``.

    Follows the per-level ``level_len = s // pf`` of
    ``src/lighthouse_selection.py:601-608``.
    """
    return [S // p ** (l - 1) for l in range(1, L + 1)]


def level_offsets(S: int, L: int, p: int) -> list[int]:
    """Offset of level l=1..L in the base-first concatenation
    (``torch.cat(levels, dim=1)``, ``src/lighthouse_selection.py:610-614``)."""
    offs, acc = [], 0
    for n in level_lengths(S, L, p):
        offs.append(acc)
        acc += n
    return offs


def closed_form_offset(S: int, level: int, p: int) -> float:
    """The reference kernel's closed form ``N*(p - p**(2-l))/(p-1)``
    (``src/lighthouse_selection_cuda.py:168-175``), in exact rationals."""
    if level <= 1:
        return 0.0
    from fractions import Fraction
    return Fraction(S) * (p - Fraction(p) ** (2 - level)) / (p - 1)


def compute_output_indices_selection(N: int, num_levels: int, pooling_factor: int, topk: int) -> int:
    """``src/lighthouse_selection_cuda.py:346-357``: coarsest level kept whole,
    ``pooling_factor*topk`` slots for every finer level."""
    total = 0
    for level in range(num_levels, 0, -1):
        c_l = pooling_factor ** (level - 1)
        total += N // c_l if level == num_levels else pooling_factor * topk
    return total


@dataclass(frozen=True)
class TileGeometry:
    S: int
    L: int
    p: int
    topk: int
    T: int            # tiles per (b, h) = topk // 128
    NCC: int          # coarsest nodes per tile
    per_tile: int     # entries emitted per tile (structural count)
    S_sel: int        # T * per_tile
    strict_ok: bool   # inside the reference kernel's well-defined domain
    reason: str       # why not, when strict_ok is False


def tile_geometry(S: int, L: int, p: int, topk: int) -> TileGeometry:
    """Tiling of ``src/lighthouse_selection_cuda.py:383-397`` plus the count of
    entries each tile emits.

    Per tile, level L contributes its NCC coarsest nodes; every finer level
    contributes the p children of each parent selected one level up, and a
    level selects ``min(candidates, 128)`` parents.  Inside the strict domain
    this equals the reference's slot count ``NCC + (L-1)*p*128``.
    """
    if topk % TOPK_PER_TILE != 0 or topk < TOPK_PER_TILE:
        raise AssertionError("topk must be a multiple of 128")
    if p & (p - 1) != 0 or p < 2:
        raise AssertionError("pf must be power of 2")
    if topk // 2 < p:
        raise AssertionError("topk // 2 >= pooling_factor")
    if L < 2:
        # with one level the reference kernel's leaf loop reads parents that were
        # never set (src/lighthouse_selection_cuda.py:293-308) and emits nothing
        raise AssertionError("num_levels must be >= 2")
    T = topk // TOPK_PER_TILE
    coarsest = S // p ** (L - 1)
    NCC = coarsest // T
    n = [0] * (L + 1)
    n[L] = NCC
    for lvl in range(L - 1, 0, -1):
        n[lvl] = p * min(n[lvl + 1], TOPK_PER_TILE)
    per_tile = sum(n[1:])
    reasons = []
    if NCC < TOPK_PER_TILE:
        reasons.append(f"N_CHUNK_COARSEST={NCC} must be >= TOPK_PER_TILE={TOPK_PER_TILE}")
    if NCC % HALF != 0:
        reasons.append(f"N_CHUNK_COARSEST={NCC} is not a multiple of 64 (tiles would overrun their slots)")
    if coarsest % T != 0:
        reasons.append(f"coarsest level length {coarsest} is not a multiple of the tile count {T}")
    if S % p ** (L - 1) != 0:
        reasons.append(f"S={S} is not a multiple of pooling_factor**(num_levels-1)={p ** (L - 1)}")
    return TileGeometry(S, L, p, topk, T, NCC, per_tile, T * per_tile, not reasons, "; ".join(reasons))


# --------------------------------------------------------------------------
# the 128-wide bitonic network
# --------------------------------------------------------------------------
_STAGES = []
_k = 2
while _k <= TOPK_PER_TILE:
    _j = _k // 2
    while _j >= 1:
        _STAGES.append((_k, _j))
        _j //= 2
    _k *= 2
_POS = np.arange(TOPK_PER_TILE)
_BIG_ID = np.int64(1) << 40


def bitonic_sort128(scores: np.ndarray, ids: np.ndarray, tie: str = "reference"):
    """Descending 128-element bitonic sort, one row per sort.

    ``src/lighthouse_selection_cuda.py:41-110``: for k = 2..128 and
    j = k/2..1, positions i < i^j are compared; the block is descending iff
    ``(i & k) == 0``; the pair is exchanged only when strictly out of order,
    so equal scores never move relative to each other within one
    compare-exchange.  The payload travels with its score.
    """
    s = np.array(scores, dtype=np.float32, copy=True)
    x = np.array(ids, dtype=np.int64, copy=True)
    assert s.shape[-1] == TOPK_PER_TILE and x.shape == s.shape
    for k, j in _STAGES:
        lo = _POS[(_POS & j) == 0]
        hi = lo | j
        desc = (lo & k) == 0
        a_s, b_s = s[..., lo], s[..., hi]
        a_x, b_x = x[..., lo], x[..., hi]
        if tie == "reference":
            swap = np.where(desc, a_s < b_s, a_s > b_s)
        elif tie == "lower_index":
            ak = np.where(a_x < 0, _BIG_ID, a_x)
            bk = np.where(b_x < 0, _BIG_ID, b_x)
            b_better = (b_s > a_s) | ((b_s == a_s) & (bk < ak))
            a_better = (a_s > b_s) | ((a_s == b_s) & (ak < bk))
            swap = np.where(desc, b_better, a_better)
        else:
            raise ValueError(f"unknown tie mode {tie!r}")
        s[..., lo] = np.where(swap, b_s, a_s)
        s[..., hi] = np.where(swap, a_s, b_s)
        x[..., lo] = np.where(swap, b_x, a_x)
        x[..., hi] = np.where(swap, a_x, b_x)
    return s, x


# --------------------------------------------------------------------------
# selection (structural formulation)
# --------------------------------------------------------------------------
def _stream_select(cand: np.ndarray, sqk_row, skq_row, tie: str):
    """Streaming top-64(qk) + top-64(kq of the qk rejects) over 64-wide batches,
    ``src/lighthouse_selection_cuda.py:189-258``.

    cand: [N, n] level-local candidate ids (-1 = invalid); sqk_row/skq_row map
    ids to scores (callables on [N, m] int arrays).  Returns the 128 selected
    ids per row in the reference's ``[TQ | TK]`` order (:324-327).
    """
    N, n = cand.shape
    nb = (n + HALF - 1) // HALF
    pad = nb * HALF - n
    if pad:
        cand = np.concatenate([cand, np.full((N, pad), -1, dtype=cand.dtype)], axis=1)
    tq_s = np.full((N, HALF), SENTINEL, dtype=np.float32)
    tq_x = np.full((N, HALF), -1, dtype=np.int64)
    tk_s = tq_s.copy()
    tk_x = tq_x.copy()
    for b in range(nb):
        c = cand[:, b * HALF:(b + 1) * HALF]
        cs = sqk_row(c)
        s, x = bitonic_sort128(np.concatenate([tq_s, cs], 1), np.concatenate([tq_x, c], 1), tie)
        tq_s, tq_x = s[:, :HALF], x[:, :HALF]
        rej = x[:, HALF:]
        ks = skq_row(rej)
        s2, x2 = bitonic_sort128(np.concatenate([tk_s, ks], 1), np.concatenate([tk_x, rej], 1), tie)
        tk_s, tk_x = s2[:, :HALF], x2[:, :HALF]
    return np.concatenate([tq_x, tk_x], axis=1)


def select_tiles(scores_qk: np.ndarray, scores_kq: np.ndarray, num_levels: int,
                 pooling_factor: int, topk: int, S: int, tie: str = "reference"):
    """Per-tile, per-level candidates and selected sets.

    Returns ``(geom, levels)`` where ``levels[l]`` (l = 1..L) is a pair
    ``(cand, selected)``: ``cand`` [B*H*T, n_l] level-local ids (-1 invalid)
    and ``selected`` [B*H*T, 128] ids in ``[TQ | TK]`` order (None for l = 1).
    """
    L, p = num_levels, pooling_factor
    g = tile_geometry(S, L, p, topk)
    sqk = np.asarray(scores_qk, dtype=np.float32)
    skq = np.asarray(scores_kq, dtype=np.float32)
    B, H, S_tot = sqk.shape
    assert sqk.shape == skq.shape
    offs = level_offsets(S, L, p)
    lens = level_lengths(S, L, p)
    assert S_tot >= offs[-1] + lens[-1]
    T, NCC = g.T, g.NCC
    N = B * H * T
    row_bh = np.repeat(np.arange(B * H), T)
    tile = np.tile(np.arange(T), B * H)
    flat_qk = sqk.reshape(B * H, S_tot)
    flat_kq = skq.reshape(B * H, S_tot)

    levels: dict[int, tuple[np.ndarray, np.ndarray | None]] = {}
    parents = None
    for lvl in range(L, 0, -1):
        off, ln = offs[lvl - 1], lens[lvl - 1]
        if lvl == L:
            cand = tile[:, None].astype(np.int64) * NCC + np.arange(NCC, dtype=np.int64)[None, :]
        else:
            a = np.arange(p * TOPK_PER_TILE)
            par = parents[:, a // p]
            cand = np.where(par >= 0, par * p + (a % p)[None, :], -1)
            cand = np.where(cand < ln, cand, -1)

        def _gather(tab, ids, off=off):
            safe = np.where(ids >= 0, ids + off, 0)
            v = np.take_along_axis(tab[row_bh], safe, axis=1)
            return np.where(ids >= 0, v, SENTINEL).astype(np.float32)

        if lvl > 1:
            sel = _stream_select(cand, lambda ids: _gather(flat_qk, ids), lambda ids: _gather(flat_kq, ids), tie)
            parents = sel
            levels[lvl] = (cand, sel)
        else:
            levels[lvl] = (cand, None)
    return g, levels


def entry_keys(level: np.ndarray, idx: np.ndarray, selected: np.ndarray, L: int, p: int) -> np.ndarray:
    """Causal order key of each emitted entry, scaled by 2**(L-1) to an integer.

    ``src/lighthouse_selection_cuda.py:16-25``: an entry at level l with local
    index i sorts at ``c_l*i`` (its span start) unless it was selected, then at
    ``c_l*(i+1) - 2**(1-l)`` (just before its span end, after all of its
    descendants).  Multiplying by 2**(L-1) makes every key an exact integer.
    """
    c = np.asarray(p, dtype=np.int64) ** (level.astype(np.int64) - 1)
    scale = np.int64(1) << (L - 1)
    unsel = c * idx * scale
    sel = c * (idx + 1) * scale - (np.int64(1) << (L - level.astype(np.int64)))
    return np.where(selected, sel, unsel)


def select_indices(scores_qk, scores_kq, num_levels: int, pooling_factor: int, topk: int,
                   actual_seq_len: int, tie: str = "reference", strict: bool = True) -> np.ndarray:
    """Selected pyramid indices ``int32 [B, H, S_sel]`` in causal (key) order.

    Restates ``LighthouseSelectionQkKqChunkedTopkNvrtc.forward``
    (``src/lighthouse_selection_cuda.py:359-428``).  Every valid candidate of
    every level is emitted exactly once by the reference kernel (as a kq
    reject after the two warm-up batches, as one of the final ``[TQ | TK]``,
    or as a level-1 leaf), so the output is "all candidates, keyed by their
    selected flag, sorted by key".  Tiles cover disjoint key ranges, so the
    result is tile-major.  ``strict=True`` raises where the reference asserts
    or is undefined.
    """
    L, p, S = num_levels, pooling_factor, actual_seq_len
    g = tile_geometry(S, L, p, topk)
    if strict and not g.strict_ok:
        raise AssertionError(g.reason)
    g, levels = select_tiles(scores_qk, scores_kq, L, p, topk, S, tie)
    B, H = np.asarray(scores_qk).shape[:2]
    offs = level_offsets(S, L, p)
    keys, vals = [], []
    for lvl in range(1, L + 1):
        cand, sel = levels[lvl]
        if sel is None:
            flag = np.zeros_like(cand, dtype=bool)
        else:
            flag = (cand[:, :, None] == sel[:, None, :]).any(-1) & (cand >= 0)
        k = entry_keys(np.full_like(cand, lvl), cand, flag, L, p)
        keys.append(np.where(cand >= 0, k, np.iinfo(np.int64).max))
        vals.append(np.where(cand >= 0, cand + offs[lvl - 1], -1))
    keys = np.concatenate(keys, axis=1)
    vals = np.concatenate(vals, axis=1)
    order = np.argsort(keys, axis=1, kind="stable")
    vals = np.take_along_axis(vals, order, axis=1)[:, :g.per_tile]
    assert (vals >= 0).all(), "structural count disagrees with the valid-candidate count"
    return vals.reshape(B, H, g.S_sel).astype(np.int32)


def inverse_map(indices: np.ndarray, S_tot: int) -> np.ndarray:
    """``inv[b, h, pyramid_index] = position in the selected sequence`` or -1."""
    B, H, S_sel = indices.shape
    inv = np.full((B, H, S_tot), -1, dtype=np.int32)
    bi, hi, si = np.meshgrid(np.arange(B), np.arange(H), np.arange(S_sel), indexing="ij")
    inv[bi, hi, indices] = si
    return inv


# --------------------------------------------------------------------------
# floating-point half (PyTorch CPU)
# --------------------------------------------------------------------------
def norm_scorer(xq, xk, xv, pooling_factor: int = 4, levels: int = 3):
    """``DialatedLighthouseNormScorer.forward`` (``src/lighthouse_selection.py:589-616``).

    Returns ``(scores_qk_cat, scores_kq_cat, xq_cat, xk_cat, xv_cat)`` with the
    reference's shapes: scores ``[B, H, S_tot]`` and pyramids ``[B, H, S_tot, D]``
    (transposed views of base-first concatenations).
    """
    b, s, h, d = xq.shape
    sqk = torch.linalg.vector_norm(xq, dim=-1)
    skq = torch.linalg.vector_norm(xk, dim=-1)
    ql, kl, vl, al, bl = [xq], [xk], [xv], [sqk], [skq]
    for level in range(1, levels):
        pf = pooling_factor ** level
        n = s // pf
        ql.append(xq[:, :n * pf].reshape(b, n, pf, h, d).mean(2))
        kl.append(xk[:, :n * pf].reshape(b, n, pf, h, d).mean(2))
        vl.append(xv[:, :n * pf].reshape(b, n, pf, h, d).mean(2))
        al.append(sqk[:, :n * pf].reshape(b, n, pf, h).amax(2))
        bl.append(skq[:, :n * pf].reshape(b, n, pf, h).amax(2))
    cat = lambda xs: torch.cat(xs, dim=1).transpose(1, 2)
    return cat(al), cat(bl), cat(ql), cat(kl), cat(vl)


_ATTN_CHUNK_ELEMS = 1 << 27  # score elements held at once by the chunked form (512 MiB fp32)


def sdpa_causal(q, k, v, scale: float | None = None, chunk: int | None = None):
    """Causal softmax attention ``softmax(q k^T * scale + mask) v`` on
    ``[..., n, D]`` tensors (the torchtitan SDPA wrapper with ``is_causal``,
    ``src/lighthouse_selection.py:815``), written out explicitly.

    Long sequences go through ``_ChunkedCausalAttn`` (query blocks of
    ``chunk`` rows, default sized to ``_ATTN_CHUNK_ELEMS``), which is the same
    formula evaluated block by block with a hand-written backward, so memory
    stays bounded at the benchmark sizes."""
    n, dh = q.shape[-2], q.shape[-1]
    scale = 1.0 / math.sqrt(dh) if scale is None else scale
    if chunk is None:
        rows = max(1, q.numel() // (n * dh)) if n else 1
        chunk = max(64, _ATTN_CHUNK_ELEMS // max(1, rows * n))
    if chunk < n:
        return _ChunkedCausalAttn.apply(q, k, v, scale, chunk)
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    mask = torch.ones(n, k.shape[-2], dtype=torch.bool, device=q.device).tril()
    s = s.masked_fill(~mask, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v)


def _causal_block_scores(q, k, i0, i1, scale):
    """Scaled, causally masked scores of queries [i0, i1) against keys [0, i1)."""
    s = torch.matmul(q[..., i0:i1, :], k[..., :i1, :].transpose(-1, -2).contiguous()) * scale
    above = torch.arange(i1, device=q.device)[None, :] > torch.arange(i0, i1, device=q.device)[:, None]
    return s.masked_fill(above, float("-inf"))


class _ChunkedCausalAttn(torch.autograd.Function if torch is not None else object):
    """``sdpa_causal`` by query blocks: forward keeps the row log-sum-exp,
    backward recomputes each block's probabilities from it
    (dV += P^T dO, dP = dO V^T, dS = P (dP - rowsum(dO o O)) * scale,
    dQ = dS K, dK += dS^T Q)."""

    @staticmethod
    def forward(ctx, q, k, v, scale, chunk):
        n = q.shape[-2]
        o = torch.empty_like(q)
        lse = q.new_empty(q.shape[:-1])
        for i0 in range(0, n, chunk):
            i1 = min(n, i0 + chunk)
            s = _causal_block_scores(q, k, i0, i1, scale)
            m = s.amax(-1, keepdim=True)
            e = torch.exp(s - m)
            den = e.sum(-1, keepdim=True)
            o[..., i0:i1, :] = torch.matmul(e, v[..., :i1, :]) / den
            lse[..., i0:i1] = (m + torch.log(den)).squeeze(-1)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale, ctx.chunk = scale, chunk
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        scale, chunk = ctx.scale, ctx.chunk
        n = q.shape[-2]
        delta = (do * o).sum(-1, keepdim=True)
        dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
        for i0 in range(0, n, chunk):
            i1 = min(n, i0 + chunk)
            pr = torch.exp(_causal_block_scores(q, k, i0, i1, scale) - lse[..., i0:i1, None])
            doc = do[..., i0:i1, :]
            dv[..., :i1, :] += torch.matmul(pr.transpose(-1, -2).contiguous(), doc)
            dp = torch.matmul(doc, v[..., :i1, :].transpose(-1, -2).contiguous())
            ds = pr * (dp - delta[..., i0:i1, :]) * scale
            dq[..., i0:i1, :] = torch.matmul(ds, k[..., :i1, :])
            dk[..., :i1, :] += torch.matmul(ds.transpose(-1, -2).contiguous(), q[..., i0:i1, :])
        return dq, dk, dv, None, None


def dilated_scorer(xq, xk, xv, dilation: int = 4, pooling_factor: int = 4, levels: int = 3,
                   attention=None):
    """``DilatedLighthouseScorer.forward`` (``src/lighthouse_selection.py:635-689``).

    Token t of head h is position ``t // dil`` of virtual head
    ``(t % dil) * H + h``; scores are the L2 norms of two causal attentions
    (q->k and k->q, both with v) over those virtual heads.  The pyramid of
    Q/K/V is the same as the norm scorer's.
    """
    attention = attention or sdpa_causal
    b, s, h, d = xq.shape
    sd = s // dilation

    def virt(x):  # [b, s, h, d] -> [b, dil*h, s/dil, d]
        return x.reshape(b, sd, dilation * h, d).transpose(1, 2)

    def unvirt(o):  # [b, dil*h, s/dil, d] -> [b, s, h, d]
        return o.transpose(1, 2).reshape(b, s, h, d)

    with torch.no_grad():  # scores only feed the (integer) selection
        out_qk = unvirt(attention(virt(xq), virt(xk), virt(xv)))
        out_kq = unvirt(attention(virt(xk), virt(xq), virt(xv)))
    sqk = torch.linalg.vector_norm(out_qk, dim=-1)
    skq = torch.linalg.vector_norm(out_kq, dim=-1)
    ql, kl, vl, al, bl = [xq], [xk], [xv], [sqk], [skq]
    for level in range(1, levels):
        pf = pooling_factor ** level
        n = s // pf
        ql.append(xq[:, :n * pf].reshape(b, n, pf, h, d).mean(2))
        kl.append(xk[:, :n * pf].reshape(b, n, pf, h, d).mean(2))
        vl.append(xv[:, :n * pf].reshape(b, n, pf, h, d).mean(2))
        al.append(sqk[:, :n * pf].reshape(b, n, pf, h).amax(2))
        bl.append(skq[:, :n * pf].reshape(b, n, pf, h).amax(2))
    cat = lambda xs: torch.cat(xs, dim=1).transpose(1, 2)
    return cat(al), cat(bl), cat(ql), cat(kl), cat(vl)


def simple_gla(q, k, v, g, scale: float):
    """Simple gated linear attention, quadratic form: for each head of
    ``[B, T, H, D]`` inputs and log gates ``g`` ``[B, T, H]``,
    ``o_t = scale * sum_{s <= t} exp(G_t - G_s) (q_t . k_s) v_s`` with
    ``G = cumsum(g)`` along T.  This is the output of ``fla``'s
    ``chunk_simple_gla(q, k, v, g, scale)`` (flash-linear-attention 0.4.x,
    pinned by ``requirements.txt``; not vendored with the reference), i.e. the
    recurrence ``h_t = exp(g_t) h_{t-1} + k_t^T v_t``, ``o_t = scale q_t h_t``
    from a zero state.  Computed in float64."""
    qd, kd, vd = (x.double().transpose(1, 2) for x in (q, k, v))  # [B, H, T, D]
    G = torch.cumsum(g.double().transpose(1, 2), dim=-1)          # [B, H, T]
    T = qd.shape[2]
    diff = G[..., :, None] - G[..., None, :]                        # G_t - G_s
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    decay = torch.where(causal, torch.exp(torch.where(causal, diff, torch.zeros_like(diff))),
                        torch.zeros_like(diff))
    a = (qd @ kd.transpose(-1, -2)) * decay * scale
    return (a @ vd).transpose(1, 2)                                  # [B, T, H, D]


def simple_gla_recurrent(q, k, v, g, scale: float):
    """The same output by the token-by-token recurrence (float64, tiny shapes)."""
    B, T, H, D = q.shape
    out = torch.zeros(B, T, H, D, dtype=torch.float64)
    for b in range(B):
        for hd in range(H):
            st = torch.zeros(D, D, dtype=torch.float64)
            for t in range(T):
                st = math.exp(float(g[b, t, hd])) * st + torch.outer(k[b, t, hd].double(), v[b, t, hd].double())
                out[b, t, hd] = scale * (q[b, t, hd].double() @ st)
    return out


def gla_scorer(xq, xk, xv, gk, dilation: int = 4, pooling_factor: int = 4, levels: int = 3,
               scale: float | None = None, round_bf16: bool = False, round_to=None):
    """``DilatedLighthouseGLAScorer.forward`` (``src/lighthouse_selection.py:713-755``).

    Token t of head h is position ``t // dil`` of virtual head ``(t % dil) * H + h``
    (the reference's ``.view(b, s // dil, dil * h, d)``, :722-725); the scores are the
    L2 norms of two simple-GLA outputs over those virtual heads, q->k and k->q, both
    with v and the gate ``gk`` [B, S, H] viewed the same way (:727-734).  The Q/K/V
    pyramid and the max-pooled score levels are the norm scorer's (:736-755).
    ``round_bf16`` rounds the GLA outputs to bfloat16 before the norm and the norm
    after it, as the reference's bf16 tensors do; ``round_to`` (a torch dtype)
    does the same for another 16-bit type."""
    if round_bf16:
        round_to = torch.bfloat16
    b, s, h, d = xq.shape
    sd = s // dilation
    scale = d ** -0.5 if scale is None else scale

    def virt(x):
        return x.reshape(b, sd, dilation * h, *x.shape[3:])

    g = gk.float().reshape(b, sd, dilation * h)
    with torch.no_grad():
        o_qk = simple_gla(virt(xq), virt(xk), virt(xv), g, scale).reshape(b, s, h, d)
        o_kq = simple_gla(virt(xk), virt(xq), virt(xv), g, scale).reshape(b, s, h, d)
        if round_to is not None:
            o_qk, o_kq = o_qk.to(round_to).double(), o_kq.to(round_to).double()
        sqk = torch.linalg.vector_norm(o_qk, dim=-1).float()
        skq = torch.linalg.vector_norm(o_kq, dim=-1).float()
        if round_to is not None:
            sqk, skq = sqk.to(round_to).float(), skq.to(round_to).float()
    ql, kl, vl, al, bl = [xq], [xk], [xv], [sqk], [skq]
    for level in range(1, levels):
        pf = pooling_factor ** level
        n = s // pf
        ql.append(xq[:, :n * pf].reshape(b, n, pf, h, d).mean(2))
        kl.append(xk[:, :n * pf].reshape(b, n, pf, h, d).mean(2))
        vl.append(xv[:, :n * pf].reshape(b, n, pf, h, d).mean(2))
        al.append(sqk[:, :n * pf].reshape(b, n, pf, h).amax(2))
        bl.append(skq[:, :n * pf].reshape(b, n, pf, h).amax(2))
    cat = lambda xs: torch.cat(xs, dim=1).transpose(1, 2)  # noqa: E731
    return cat(al), cat(bl), cat(ql), cat(kl), cat(vl)


def fanout_spans(indices, S: int, L: int, p: int):
    """For each selected entry: (first base position, fan-out c_l) of the span
    it is added to, ``[(i+1)c_l - 1, (i+2)c_l - 2]`` clipped to ``[0, S)``
    (``src/lighthouse_selection.py:428-451``)."""
    idx = torch.as_tensor(np.asarray(indices)).long()
    offs = level_offsets(S, L, p)
    lens = level_lengths(S, L, p)
    start = torch.zeros_like(idx)
    fan = torch.ones_like(idx)
    for lvl in range(1, L + 1):
        c = p ** (lvl - 1)
        inl = (idx >= offs[lvl - 1]) & (idx < offs[lvl - 1] + lens[lvl - 1])
        local = idx - offs[lvl - 1]
        start = torch.where(inl, local * c + (c - 1), start)
        fan = torch.where(inl, torch.full_like(idx, c), fan)
    return start, fan


def scatter_fwd(attn_out, indices, S: int, L: int, p: int, N_total: int | None = None):
    """``_ScatterToBaseAutograd.forward`` with ``rank_ids = 0`` and ``N_shard = S``
    (``src/lighthouse_selection.py:817-823`` uses ``N_total = S`` too):
    ``out[b,h,t] = sum of attn_out[b,h,s]`` over entries s whose span holds t,
    for ``t < N_total``."""
    N_total = S if N_total is None else N_total
    B, H, S_sel, D = attn_out.shape
    start, fan = fanout_spans(indices, S, L, p)
    out = torch.zeros(B, H, N_total, D, dtype=attn_out.dtype)
    cmax = p ** (L - 1)
    for u in range(cmax):
        pos = start + u
        ok = (u < fan) & (pos < N_total)
        tgt = torch.where(ok, pos, torch.zeros_like(pos))
        src = attn_out * ok[..., None].to(attn_out.dtype)
        out = out.scatter_add(2, tgt[..., None].expand(B, H, S_sel, D), src)
    return out


def scatter_bwd(grad_out, indices, S: int, L: int, p: int):
    """``_ScatterToBaseAutograd.backward`` (``src/lighthouse_selection.py:462-514,552-576``):
    ``grad_attn[b,h,s] = sum of grad_out[b,h,t]`` over t in the span of entry s
    (``t < N_total``, the length of ``grad_out``)."""
    B, H, N_total, D = grad_out.shape
    start, fan = fanout_spans(indices, S, L, p)
    S_sel = start.shape[-1]
    acc = torch.zeros(B, H, S_sel, D, dtype=grad_out.dtype)
    for u in range(p ** (L - 1)):
        pos = start + u
        ok = (u < fan) & (pos < N_total)
        tgt = torch.where(ok, pos, torch.zeros_like(pos))
        g = torch.gather(grad_out, 2, tgt[..., None].expand(B, H, S_sel, D))
        acc = acc + g * ok[..., None].to(grad_out.dtype)
    return acc


class _ScatterFn(torch.autograd.Function if torch is not None else object):
    @staticmethod
    def forward(ctx, attn_out, indices, S, L, p):
        ctx.save_for_backward(indices)
        ctx.geo = (S, L, p)
        return scatter_fwd(attn_out, indices, S, L, p)

    @staticmethod
    def backward(ctx, g):
        (indices,) = ctx.saved_tensors
        return scatter_bwd(g, indices, *ctx.geo), None, None, None, None


def lighthouse_layer(xq, xk, xv, num_levels: int, pooling_factor: int, topk: int,
                     scorer: str = "norm", dilation: int = 4, indices=None,
                     tie: str = "reference", strict: bool = True, gk=None):
    """``LighthouseLocal.forward`` (``src/lighthouse_selection.py:789-825``) on
    the CPU, differentiable through torch autograd.

    ``indices`` (int32 ``[B, H, S_sel]``) may be supplied to share one selected
    set with the device path; otherwise they are computed by ``select_indices``
    from this oracle's own scores.  Returns ``(out [B,H,S,D], indices)``.
    """
    L, p = num_levels, pooling_factor
    b, s, h, d = xq.shape
    if scorer == "norm":
        sqk, skq, qc, kc, vc = norm_scorer(xq, xk, xv, p, L)
    elif scorer == "dilated":
        sqk, skq, qc, kc, vc = dilated_scorer(xq, xk, xv, dilation, p, L)
    elif scorer == "gla":
        sqk, skq, qc, kc, vc = gla_scorer(xq, xk, xv, gk, dilation, p, L)
    else:
        raise ValueError(scorer)
    if indices is None:
        indices = select_indices(sqk.detach().float().numpy(), skq.detach().float().numpy(),
                                 L, p, topk, s, tie=tie, strict=strict)
    idx = torch.as_tensor(np.asarray(indices)).long()
    gi = idx[..., None].expand(-1, -1, -1, d)
    sq = torch.gather(qc, 2, gi)
    sk = torch.gather(kc, 2, gi)
    sv = torch.gather(vc, 2, gi)
    attn = sdpa_causal(sq, sk, sv)
    out = _ScatterFn.apply(attn, idx, s, L, p)
    return out, np.asarray(indices)
