"""ctypes binding of ``liblighthouse_hip.so`` (the gfx950 kernels behind the C ABI
declared in ``include/lighthouse_hip.h``) and thin tensor-level wrappers.

PyTorch is used only for device memory and the current HIP stream: every
wrapper allocates its outputs with ``torch.empty`` and passes raw pointers,
sizes and strides to the library, which launches on the caller's stream.
There is no fallback: if the library is missing or a tensor is not on a GPU,
the call raises.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblighthouse_hip.so")
CSRC = os.path.join(_HERE, "csrc")
D_SUPPORTED = 128

TIE_MODES = {"reference": 0, "lower_index": 1}

_lib = None
_lock = threading.Lock()

_c = ctypes
_P = _c.c_void_p
_I = _c.c_int
_L = _c.c_int64
_F = _c.c_float

_SIGS = {
    "lh_strerror": (_c.c_char_p, [_I]),
    "lh_abi_version": (_I, []),
    "lh_select_geometry": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P]),
    "lh_pyramid_fwd": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _P, _L, _L, _L, _P, _P,
                            _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "lh_dilated_scores": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _P]),
    "lh_gla_scores": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _P, _L, _I, _P]),
    "lh_gla_workspace_bytes": (_L, [_I, _I, _I, _I, _I, _I]),
    "lh_select_topk": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "lh_build_inverse": (_I, [_P, _I, _P, _I, _I, _I, _P]),
    "lh_check_indices": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "lh_attn_fwd": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _P, _L, _L, _L, _I, _P,
                         _I, _I, _I, _I, _F, _P, _P, _I, _P]),
    "lh_attn_bwd": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _P, _L, _L, _L, _I, _P,
                         _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _I, _P]),
    "lh_attn_bwd_dkdv": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _P, _L, _L, _L, _I, _P,
                              _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _I, _P]),
    "lh_attn_bwd_dq": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _P, _L, _L, _L, _I, _P,
                            _I, _I, _I, _I, _F, _P, _P, _P, _P, _I, _P]),
    "lh_attn_status": (_I, [_P]),
    "lh_attn_queue_slot": (_I, [_P, _P]),
    "lh_attn_set_schedule": (_I, [_I, _P]),
    "lh_scatter_fwd": (_I, [_P, _P, _P, _L, _L, _L, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "lh_scatter_bwd": (_I, [_P, _L, _L, _L, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "lh_pyramid_bwd": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "lh_rope_pyramid_fwd": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _P, _L, _L, _L, _P, _P, _P, _L, _L, _L,
                                 _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "lh_pyramid_rope_bwd": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _P, _P, _P, _L, _L, _L,
                                 _I, _I, _I, _I, _I, _I, _P]),
    "lh_rope_qkv_fwd": (_I, [_P, _L, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "lh_rope_qkv_bwd": (_I, [_P, _P, _P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P]),
    "lh_rmsnorm_fwd": (_I, [_P, _P, _P, _P, _L, _I, _F, _P]),
    "lh_add_rmsnorm_fwd": (_I, [_P, _P, _P, _P, _P, _P, _L, _I, _F, _P]),
    "lh_rmsnorm_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _P]),
    "lh_rmsnorm_bwd_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _L, _I, _P]),
    "lh_swiglu_fwd": (_I, [_P, _P, _L, _I, _P]),
    "lh_swiglu_bwd": (_I, [_P, _P, _P, _L, _I, _P]),
    "lh_splitk_sum": (_I, [_P, _P, _I, _L, _P]),
}
EXPORTED = tuple(_SIGS)


def build(force: bool = True, jobs: int = 5) -> str:
    """Compile ``liblighthouse_hip.so`` for gfx950 with hipcc (``csrc/Makefile``)."""
    if force:
        subprocess.run(["make", "-s", "-C", CSRC, "clean"], check=True)
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", CSRC], check=True)
    return LIB_PATH


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build it with `make -C {CSRC}` "
                        "(or __graft_entry__.build()); there is no non-native fallback")
                h = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in _SIGS.items():
                    f = getattr(h, name)
                    f.restype = res
                    f.argtypes = args
                _lib = h
    return _lib


class LighthouseHipError(RuntimeError):
    pass


def _check(rc: int, what: str):
    if rc != 0:
        msg = lib().lh_strerror(rc).decode()
        raise LighthouseHipError(f"{what}: {msg} (code {rc})")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise LighthouseHipError("lighthouse_hip kernels need GPU tensors (no CPU path)")


# Row element types of the native kernels (LH_DTYPE_* of the C ABI).
ROW_DTYPES = {torch.bfloat16: 0, torch.float16: 1}


def _need_rows(what, *ts, dtypes=ROW_DTYPES):
    """16-bit float storage (bf16 or fp16, one type for all rows of a call) with a
    contiguous last (head) dimension: what every row-reading kernel of the
    library assumes.  Returns the dtype code (LH_DTYPE_BF16 / LH_DTYPE_F16)."""
    code, first = None, None
    for t in ts:
        if t is None:
            continue
        if t.dtype not in dtypes:
            names = " or ".join(str(d).replace("torch.", "") for d in dtypes)
            raise TypeError(f"{what}: the native kernels read and write {names} rows; got {t.dtype}")
        if first is not None and t.dtype != first:
            raise TypeError(f"{what}: all rows of one call must share a dtype; got {first} and {t.dtype}")
        first, code = t.dtype, dtypes[t.dtype]
        if t.dim() and t.stride(-1) != 1:
            raise ValueError(f"{what}: the head dimension must be contiguous (stride(-1) == 1)")
    return 0 if code is None else code


BF16_ONLY = {torch.bfloat16: 0}


def _need_dtype(what, dtype, *ts):
    for t in ts:
        if t is not None and t.dtype != dtype:
            raise TypeError(f"{what}: expected {dtype}, got {t.dtype}")


# Index validation before every launch that reads caller indices: off by default,
# on with LH_CHECK_INDICES=1 in the environment or set_check_indices(True).  Each
# check synchronizes the stream (debug aid, not for timed runs), so the checks
# are skipped while the current stream is being captured into a graph.
_check_indices = os.environ.get("LH_CHECK_INDICES", "0") not in ("", "0")


def set_check_indices(on: bool) -> bool:
    """Turn the index check mode on or off; returns the previous setting."""
    global _check_indices
    prev, _check_indices = _check_indices, bool(on)
    return prev


def check_indices(indices, lo: int, hi: int, unique: bool = True, what: str = "indices"):
    """Raise ``IndexError`` unless every entry of ``indices`` [B, H, n] lies in
    ``[lo, hi)`` and (``unique``) no (b, h) names a row twice.  Synchronizes."""
    _need_gpu(indices)
    _need_dtype(what, torch.int32, indices)
    idx = indices.contiguous()
    B, H, n = idx.shape
    dev = idx.device
    counts = torch.empty(2, dtype=torch.int32, device=dev)
    marks = torch.empty(B, H, hi - lo, dtype=torch.int32, device=dev) if unique else None
    with torch.cuda.device(dev):
        rc = lib().lh_check_indices(_ptr(idx), B, H, n, lo, hi, _ptr(marks), _ptr(counts), _stream(dev))
    _check(rc, "lh_check_indices")
    bad, dup = (int(c) for c in counts.cpu())
    if bad:
        raise IndexError(f"{what}: {bad} entries outside [{lo}, {hi})")
    if dup:
        raise IndexError(f"{what}: {dup} duplicate entries (indices must be unique per (batch, head))")


def geometry(S: int, L: int, p: int, topk: int, strict: bool = True):
    """``(num_tiles, nodes_per_tile, per_tile, S_sel)``; raises like the reference outside
    its domain when ``strict``."""
    out = [ctypes.c_int() for _ in range(4)]
    rc = lib().lh_select_geometry(S, L, p, topk, int(bool(strict)), *[ctypes.byref(o) for o in out])
    if rc == 2:
        raise AssertionError(
            f"selection geometry S={S}, num_levels={L}, pooling_factor={p}, topk={topk} is outside the "
            "reference kernel's domain (N_CHUNK_COARSEST must be >= 128 and a multiple of 64, tiles must "
            "divide the coarsest level); pass strict=False for per-tile compaction")
    _check(rc, "lh_select_geometry")
    return tuple(o.value for o in out)


def pyramid_lengths(S: int, L: int, p: int):
    lens = [S // p ** l for l in range(L)]
    offs = [sum(lens[:l]) for l in range(L)]
    return lens, offs, sum(lens)


# ---------------------------------------------------------------------------
# op wrappers (tensor in, tensor out; all on the current stream)
# ---------------------------------------------------------------------------
def pyramid_fwd(xq, xk, xv, L: int, p: int, scores=None, pooled_out=None):
    """Norm scores + pooled Q/K/V.  ``xq/xk/xv`` bf16 or fp16 [B, S, H, D] with D contiguous.

    Returns ``(pq, pk, pv, scores_qk, scores_kq)`` with pooled rows of the input
    dtype [B, Sp, H, D] and scores fp32 [B, H, S_tot].  If ``scores`` is given
    (dilated scorer), its base level is kept and only pooled.
    ``pooled_out`` may supply three pooled destinations (any strides, D contiguous).
    """
    _need_gpu(xq, xk, xv)
    dt = _need_rows("pyramid_fwd", xq, xk, xv)
    B, S, H, D = xq.shape
    assert xk.shape == xq.shape and xv.shape == xq.shape
    assert xq.stride() == xk.stride() == xv.stride(), "q/k/v must share strides"
    lens, offs, S_tot = pyramid_lengths(S, L, p)
    Sp = S_tot - S
    dev = xq.device
    if pooled_out is None:
        pq, pk, pv = (torch.empty(B, Sp, H, D, dtype=xq.dtype, device=dev) for _ in range(3))
    else:
        pq, pk, pv = pooled_out
        _need_rows("pyramid_fwd pooled_out", xq, pq, pk, pv)
    if scores is None:
        sqk = torch.empty(B, H, S_tot, dtype=torch.float32, device=dev)
        skq = torch.empty_like(sqk)
        given = 0
    else:
        sqk, skq = scores
        given = 1
    sb, ss, sh, _ = xq.stride()
    pb, ps, ph, _ = pq.stride()
    with torch.cuda.device(dev):
        rc = lib().lh_pyramid_fwd(_ptr(xq), _ptr(xk), _ptr(xv), sb, ss, sh, _ptr(pq), _ptr(pk), _ptr(pv),
                                  pb, ps, ph, _ptr(sqk), _ptr(skq), B, S, H, D, L, p, given, dt, _stream(dev))
    _check(rc, "lh_pyramid_fwd")
    return pq, pk, pv, sqk, skq


def _check_freqs(freqs, S: int, D: int):
    assert freqs.dtype == torch.float32 and freqs.is_contiguous() and tuple(freqs.shape[1:]) == (D // 2, 2) \
        and freqs.shape[0] >= S, "freqs must be fp32 [>= S, D/2, 2] contiguous"


def rope_pyramid_fwd(xqkv, freqs, H: int, L: int, p: int, D: int = D_SUPPORTED):
    """Rotary embedding fused into the pyramid pass.

    ``xqkv`` bf16 [B, S, 3*H*D]: the fused [q | k | v] projection output (row
    stride may exceed the width; D contiguous), q and k unrotated.  Returns
    ``(xr, pq, pk, pv, scores_qk, scores_kq)``: ``xr`` [B, S, 3*H*D] with the
    rotated q and k rows in its first two column blocks (the third block is left
    unwritten; v rows are read from ``xqkv``), so q, k (from ``xr``) and v (from
    ``xqkv``) share one set of strides; the rest as ``pyramid_fwd``."""
    _need_gpu(xqkv, freqs)
    B, S, W = xqkv.shape
    _need_rows("rope_pyramid_fwd", xqkv, dtypes=BF16_ONLY)
    assert W == 3 * H * D, "xqkv must hold [q | k | v] heads"
    assert xqkv.stride(2) == 1 and xqkv.stride(0) == S * xqkv.stride(1), "rows of xqkv must be evenly strided"
    _check_freqs(freqs, S, D)
    lens, offs, S_tot = pyramid_lengths(S, L, p)
    dev = xqkv.device
    xr = torch.empty_strided(xqkv.shape, xqkv.stride(), dtype=torch.bfloat16, device=dev)
    pq, pk, pv = (torch.empty(B, S_tot - S, H, D, dtype=torch.bfloat16, device=dev) for _ in range(3))
    sqk = torch.empty(B, H, S_tot, dtype=torch.float32, device=dev)
    skq = torch.empty_like(sqk)
    rs = xqkv.stride(1)
    base = xqkv.data_ptr()
    e = xqkv.element_size()
    with torch.cuda.device(dev):
        rc = lib().lh_rope_pyramid_fwd(base, base + H * D * e, base + 2 * H * D * e, S * rs, rs, D,
                                       _ptr(freqs), xr.data_ptr(), xr.data_ptr() + H * D * e, S * rs, rs, D,
                                       _ptr(pq), _ptr(pk), _ptr(pv), *pq.stride()[:3], _ptr(sqk), _ptr(skq),
                                       B, S, H, D, L, p, _stream(dev))
    _check(rc, "lh_rope_pyramid_fwd")
    return xr, pq, pk, pv, sqk, skq


def dilated_scores(xq, xk, xv, dilation: int, S_tot: int, scale: float | None = None):
    """Base-level dilated scores into fresh fp32 [B, H, S_tot] buffers (pooled levels unset)."""
    _need_gpu(xq, xk, xv)
    dt = _need_rows("dilated_scores", xq, xk, xv)
    B, S, H, D = xq.shape
    for t in (xq, xk, xv):
        assert t.is_contiguous()
    dev = xq.device
    sqk = torch.empty(B, H, S_tot, dtype=torch.float32, device=dev)
    skq = torch.empty_like(sqk)
    with torch.cuda.device(dev):
        rc = lib().lh_dilated_scores(_ptr(xq), _ptr(xk), _ptr(xv), _ptr(sqk), _ptr(skq), B, S, H, D, dilation,
                                     S_tot, float(scale or 0.0), dt, _stream(dev))
    _check(rc, "lh_dilated_scores")
    _check_queues(dev, "lh_dilated_scores")
    return sqk, skq


def gla_scores(xq, xk, xv, gk, dilation: int, S_tot: int, scale: float | None = None, segments: int = 0):
    """Base-level GLA scores into fresh fp32 [B, H, S_tot] buffers (pooled levels unset).
    ``gk`` [B, S, H] log gates (any float dtype; taken in fp32, as fla does).
    ``segments``: sequence segments walked in parallel (0: chosen from the
    sequence length alone; 1: one sequential walk).  Rows bf16 or fp16; the
    scores are rounded to the row type."""
    dt = _need_rows("gla_scores", xq, xk, xv)
    _need_gpu(xq, xk, xv, gk)
    B, S, H, D = xq.shape
    for t in (xq, xk, xv):
        assert t.is_contiguous()
    if tuple(gk.shape) != (B, S, H):
        raise ValueError(f"gk must be [B, S, H] = {(B, S, H)}, got {tuple(gk.shape)}")
    g = gk.float().contiguous()
    dev = xq.device
    sqk = torch.empty(B, H, S_tot, dtype=torch.float32, device=dev)
    skq = torch.empty_like(sqk)
    scale = D ** -0.5 if scale is None else scale
    nbytes = lib().lh_gla_workspace_bytes(B, S, H, D, dilation, int(segments))
    if nbytes < 0:
        raise ValueError(f"gla_scores: invalid geometry B={B} S={S} H={H} D={D} dilation={dilation}")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev) if nbytes else None
    with torch.cuda.device(dev):
        rc = lib().lh_gla_scores(_ptr(xq), _ptr(xk), _ptr(xv), _ptr(g), _ptr(sqk), _ptr(skq), B, S, H, D, dilation,
                                 S_tot, float(scale), int(segments), _ptr(ws), nbytes, dt,
                                 _stream(dev))
    _check(rc, "lh_gla_scores")
    return sqk, skq


def select_topk(scores_qk, scores_kq, S: int, L: int, p: int, topk: int, tie: str = "reference",
                strict: bool = True, with_inverse: bool = True):
    """int32 indices [B, H, S_sel] (+ inverse map [B, H, S_tot] or None)."""
    _need_gpu(scores_qk, scores_kq)
    assert scores_qk.dtype == torch.float32 and scores_kq.dtype == torch.float32
    assert scores_qk.shape == scores_kq.shape
    if tie not in TIE_MODES:
        raise ValueError(f"tie_break must be one of {sorted(TIE_MODES)}, got {tie!r}")
    B, H, S_tot = scores_qk.shape
    _, _, S_tot_expected = pyramid_lengths(S, L, p)
    assert S_tot >= S_tot_expected, "scores are shorter than the pyramid"
    sqk = scores_qk.contiguous()
    skq = scores_kq.contiguous()
    _, _, _, S_sel = geometry(S, L, p, topk, strict)
    dev = sqk.device
    idx = torch.empty(B, H, S_sel, dtype=torch.int32, device=dev)
    inv = torch.empty(B, H, S_tot, dtype=torch.int32, device=dev) if with_inverse else None
    if with_inverse and S_tot != S_tot_expected:
        raise AssertionError("inverse map needs scores of exactly the pyramid length")
    with torch.cuda.device(dev):
        rc = lib().lh_select_topk(_ptr(sqk), _ptr(skq), _ptr(idx), _ptr(inv), B, H, S, L, p, topk,
                                  TIE_MODES[tie], int(bool(strict)), _stream(dev))
    _check(rc, "lh_select_topk")
    return idx, inv


def build_inverse(indices, S_tot: int, validate: bool = False):
    """Inverse map of ``indices`` [B, H, n]; with ``validate`` (or the check mode)
    the indices are first checked to lie in [0, S_tot) or be -1 (an empty slot,
    skipped) and to name no row twice per (b, h)."""
    _need_dtype("build_inverse indices", torch.int32, indices)
    _need_gpu(indices)
    if validate or _check_mode():
        check_indices(indices, -1, S_tot, unique=True, what="indices")
    idx = indices.contiguous()
    B, H, n = idx.shape
    inv = torch.empty(B, H, S_tot, dtype=torch.int32, device=idx.device)
    with torch.cuda.device(idx.device):
        rc = lib().lh_build_inverse(_ptr(idx), n, _ptr(inv), S_tot, B, H, _stream(idx.device))
    _check(rc, "lh_build_inverse")
    return inv


def attn_status(device=None) -> int:
    """Work-queue faults of the persistent attention launches on ``device``
    since the last call: 0 when every launch's blocks added up, else the number
    of counter slots found not cleared at launch (blocks skipped or repeated),
    which are reset.  Synchronizes the device."""
    f = ctypes.c_int(0)
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        rc = lib().lh_attn_status(ctypes.byref(f))
    _check(rc, "lh_attn_status")
    return f.value


SCHED_NO_PLAN = 1   # LH_SCHED_NO_PLAN
SCHED_NO_QUEUE = 2  # LH_SCHED_NO_QUEUE


def set_attention_schedule(plans: bool = True, queues: bool = True):
    """Let the attention launches of this process use packed query-block plans
    and per-XCD work queues where their shape calls for them (the default), or
    keep them from it, for A/B measurement; outputs are bit-identical either
    way.  Returns the previous setting as ``(plans, queues)``."""
    prev = ctypes.c_int(0)
    flags = (0 if plans else SCHED_NO_PLAN) | (0 if queues else SCHED_NO_QUEUE)
    _check(lib().lh_attn_set_schedule(flags, ctypes.byref(prev)), "lh_attn_set_schedule")
    return (not prev.value & SCHED_NO_PLAN, not prev.value & SCHED_NO_QUEUE)


def _check_mode() -> bool:
    """Check mode is on and the current stream can synchronize (not capturing)."""
    return _check_indices and torch.cuda.is_available() and not torch.cuda.is_current_stream_capturing()


def _check_queues(dev, what: str):
    """In check mode, raise if an attention launch found its work-queue counters dirty."""
    if _check_mode():
        n = attn_status(dev)
        if n:
            raise LighthouseHipError(
                f"{what}: {n} work-queue counter slot(s) were not cleared at launch, so blocks were skipped "
                "or repeated and the outputs are not to be trusted; the slots are reset now")


class Rows:
    """Where row r of (b, h) lives: ``base`` [.., r, .., D] for r < split,
    else ``pool`` at r - split.  Strides are in elements, D contiguous."""

    def __init__(self, q, k, v, base_strides, qp=None, kp=None, vp=None, pool_strides=(0, 0, 0), split=None,
                 limit=None):
        self.dtype_code = _need_rows("attention rows", q, k, v, qp, kp, vp)
        self.dtype = q.dtype
        self.q, self.k, self.v = q, k, v
        self.qp, self.kp, self.vp = qp, kp, vp
        self.bs = tuple(int(s) for s in base_strides)
        self.ps = tuple(int(s) for s in pool_strides)
        self.split = int(split) if split is not None else 2 ** 31 - 1
        # number of addressable rows (split + pooled rows), for the index check mode
        self.limit = int(limit) if limit is not None else None

    def check(self, indices):
        if _check_mode() and indices is not None and self.limit is not None:
            check_indices(indices, 0, self.limit, unique=False, what="attention row indices")

    def args(self):
        return (_ptr(self.q), _ptr(self.k), _ptr(self.v), *self.bs,
                _ptr(self.qp), _ptr(self.kp), _ptr(self.vp), *self.ps, self.split)


def _bwd_args_check(rows, indices, dout, lse, delta):
    _need_dtype("attention backward indices", torch.int32, indices)
    _need_rows("attention backward dout", dout)
    _need_dtype("attention backward dout", rows.dtype, dout)
    _need_dtype("attention backward lse/delta", torch.float32, lse, delta)
    _need_gpu(rows.q, dout, lse, delta, indices)
    rows.check(indices)


def attn_fwd(rows: Rows, indices, B: int, H: int, n: int, D: int = D_SUPPORTED, scale: float | None = None):
    """Causal attention over the rows named by ``indices`` [B, H, n] (None = identity).

    Returns ``(O [B, H, n, D] of the rows' dtype, lse fp32 [B, H, n])`` (lse in the
    exp2 domain)."""
    _need_dtype("attn_fwd indices", torch.int32, indices)
    _need_gpu(rows.q, indices)
    rows.check(indices)
    dev = rows.q.device
    scale = D ** -0.5 if scale is None else scale
    idx = indices.contiguous() if indices is not None else None
    out = torch.empty(B, H, n, D, dtype=rows.dtype, device=dev)
    lse = torch.empty(B, H, n, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = lib().lh_attn_fwd(*rows.args(), _ptr(idx), B, H, n, D, scale, _ptr(out), _ptr(lse), rows.dtype_code,
                               _stream(dev))
    _check(rc, "lh_attn_fwd")
    _check_queues(dev, "lh_attn_fwd")
    return out, lse


def attn_bwd_dkdv(rows: Rows, indices, B: int, H: int, n: int, dout, lse, delta, D: int = D_SUPPORTED,
                  scale: float | None = None):
    """dK, dV of the gathered rows (key-stationary kernel): two [B, H, n, D] of the rows' dtype."""
    _bwd_args_check(rows, indices, dout, lse, delta)
    dev = rows.q.device
    scale = D ** -0.5 if scale is None else scale
    idx = indices.contiguous() if indices is not None else None
    dk, dv = (torch.empty(B, H, n, D, dtype=rows.dtype, device=dev) for _ in range(2))
    with torch.cuda.device(dev):
        rc = lib().lh_attn_bwd_dkdv(*rows.args(), _ptr(idx), B, H, n, D, scale, _ptr(dout.contiguous()),
                                    _ptr(lse), _ptr(delta), _ptr(dk), _ptr(dv), rows.dtype_code, _stream(dev))
    _check(rc, "lh_attn_bwd_dkdv")
    _check_queues(dev, "lh_attn_bwd_dkdv")
    return dk, dv


def attn_bwd_dq(rows: Rows, indices, B: int, H: int, n: int, dout, lse, delta, D: int = D_SUPPORTED,
                scale: float | None = None):
    """dQ of the gathered rows (query-stationary kernel): [B, H, n, D] of the rows' dtype."""
    _bwd_args_check(rows, indices, dout, lse, delta)
    dev = rows.q.device
    scale = D ** -0.5 if scale is None else scale
    idx = indices.contiguous() if indices is not None else None
    dq = torch.empty(B, H, n, D, dtype=rows.dtype, device=dev)
    with torch.cuda.device(dev):
        rc = lib().lh_attn_bwd_dq(*rows.args(), _ptr(idx), B, H, n, D, scale, _ptr(dout.contiguous()),
                                  _ptr(lse), _ptr(delta), _ptr(dq), rows.dtype_code, _stream(dev))
    _check(rc, "lh_attn_bwd_dq")
    _check_queues(dev, "lh_attn_bwd_dq")
    return dq


def attn_bwd(rows: Rows, indices, B: int, H: int, n: int, dout, lse, delta, D: int = D_SUPPORTED,
             scale: float | None = None):
    """Gradients w.r.t. the gathered q, k, v rows: three [B, H, n, D] of the rows' dtype."""
    _bwd_args_check(rows, indices, dout, lse, delta)
    dev = rows.q.device
    scale = D ** -0.5 if scale is None else scale
    idx = indices.contiguous() if indices is not None else None
    dout = dout.contiguous()
    dq, dk, dv = (torch.empty(B, H, n, D, dtype=rows.dtype, device=dev) for _ in range(3))
    with torch.cuda.device(dev):
        rc = lib().lh_attn_bwd(*rows.args(), _ptr(idx), B, H, n, D, scale, _ptr(dout), _ptr(lse), _ptr(delta),
                               _ptr(dq), _ptr(dk), _ptr(dv), rows.dtype_code, _stream(dev))
    _check(rc, "lh_attn_bwd")
    _check_queues(dev, "lh_attn_bwd")
    return dq, dk, dv


def scatter_fwd(attn, inverse, S: int, S_out: int, L: int, p: int, seq_major: bool = False):
    """Fan-out of the selected rows onto the base sequence: ``[B, H, S_out, D]``.

    ``seq_major`` stores the result as ``[B, S_out, H, D]`` and returns its
    ``[B, H, S_out, D]`` view (transposing it back is then free)."""
    dt = _need_rows("scatter_fwd attn", attn)
    _need_dtype("scatter_fwd inverse", torch.int32, inverse)
    _need_gpu(attn, inverse)
    attn = attn.contiguous()
    B, H, n, D = attn.shape
    if _check_mode():
        check_indices(inverse, -1, n, unique=False, what="scatter_fwd inverse map")
    if seq_major:
        out = torch.empty(B, S_out, H, D, dtype=attn.dtype, device=attn.device).transpose(1, 2)
    else:
        out = torch.empty(B, H, S_out, D, dtype=attn.dtype, device=attn.device)
    ob, oh, os_, od = out.stride()
    with torch.cuda.device(attn.device):
        rc = lib().lh_scatter_fwd(_ptr(attn), _ptr(inverse), _ptr(out), ob, oh, os_, B, H, S, S_out, n, D, L, p,
                                  dt, _stream(attn.device))
    _check(rc, "lh_scatter_fwd")
    return out


def scatter_bwd(dout, indices, o, S: int, L: int, p: int):
    """``(dattn [B, H, n, D] of dout's dtype, delta fp32 [B, H, n] or None)``; ``dout``
    may have any (batch, head, seq) strides with D contiguous."""
    dt = _need_rows("scatter_bwd", dout, o)
    _need_dtype("scatter_bwd indices", torch.int32, indices)
    _need_gpu(dout, indices, o)
    if _check_mode():
        check_indices(indices, 0, pyramid_lengths(S, L, p)[2], unique=True, what="scatter_bwd indices")
    if dout.stride(3) != 1 or any(st % 8 for st in dout.stride()[:3]) or dout.data_ptr() % 16:
        dout = dout.contiguous()
    B, H, S_out, D = dout.shape
    n = indices.shape[-1]
    dattn = torch.empty(B, H, n, D, dtype=dout.dtype, device=dout.device)
    delta = torch.empty(B, H, n, dtype=torch.float32, device=dout.device) if o is not None else None
    oc = o.contiguous() if o is not None else None
    db, dh, ds, _ = dout.stride()
    with torch.cuda.device(dout.device):
        rc = lib().lh_scatter_bwd(_ptr(dout), db, dh, ds, _ptr(indices.contiguous()), _ptr(oc), _ptr(dattn),
                                  _ptr(delta), B, H, S, S_out, n, D, L, p, dt, _stream(dout.device))
    _check(rc, "lh_scatter_bwd")
    return dattn, delta


def pyramid_bwd(gq, gk, gv, inverse, B: int, S: int, H: int, L: int, p: int, D: int = D_SUPPORTED):
    """Base-row gradients [B, S, H, D] (the grads' dtype) from selected-space (or
    pyramid-row) grads ``g*`` indexed [b, h, s, :] with any strides (D contiguous)."""
    dt = _need_rows("pyramid_bwd grads", gq, gk, gv)
    _need_dtype("pyramid_bwd inverse", torch.int32, inverse)
    ref = next(g for g in (gq, gk, gv) if g is not None)
    _need_gpu(ref, inverse)
    if _check_mode() and inverse is not None:
        check_indices(inverse, -1, ref.shape[2], unique=False, what="pyramid_bwd inverse map")
    dev = ref.device
    outs = [torch.empty(B, S, H, D, dtype=ref.dtype, device=dev) if g is not None else None
            for g in (gq, gk, gv)]
    gb, gh, gs, _ = ref.stride()
    for g in (gq, gk, gv):
        assert g is None or tuple(g.stride()) == (gb, gh, gs, 1), "selected grads must share strides"
    with torch.cuda.device(dev):
        rc = lib().lh_pyramid_bwd(_ptr(gq), _ptr(gk), _ptr(gv), gb, gh, gs, _ptr(inverse),
                                  _ptr(outs[0]), _ptr(outs[1]), _ptr(outs[2]), B, S, H, D, L, p, dt, _stream(dev))
    _check(rc, "lh_pyramid_bwd")
    return tuple(outs)


def pyramid_rope_bwd(gq, gk, gv, inverse, freqs, B: int, S: int, H: int, L: int, p: int, D: int = D_SUPPORTED):
    """``pyramid_bwd`` with the rotary embedding's backward fused in: returns the
    gradient of the fused projection output, bf16 [B, S, 3*H*D] ([dq | dk | dv],
    dq and dk rotated back by -theta)."""
    _need_rows("pyramid_rope_bwd grads", gq, gk, gv, dtypes=BF16_ONLY)
    _need_gpu(gq, gk, gv)
    _check_freqs(freqs, S, D)
    gb, gh, gs, _ = gq.stride()
    for g in (gk, gv):
        assert tuple(g.stride()) == (gb, gh, gs, 1), "selected grads must share strides"
    dev = gq.device
    W = 3 * H * D
    dx = torch.empty(B, S, W, dtype=torch.bfloat16, device=dev)
    base, e = dx.data_ptr(), dx.element_size()
    with torch.cuda.device(dev):
        rc = lib().lh_pyramid_rope_bwd(_ptr(gq), _ptr(gk), _ptr(gv), gb, gh, gs, _ptr(inverse), _ptr(freqs),
                                       base, base + H * D * e, base + 2 * H * D * e, S * W, W, D,
                                       B, S, H, D, L, p, _stream(dev))
    _check(rc, "lh_pyramid_rope_bwd")
    return dx


# ---------------------------------------------------------------------------
# transformer-block ops (rotary embedding, RMSNorm, SwiGLU)
# ---------------------------------------------------------------------------
def rope_qkv_fwd(x, freqs, Hq: int, Hkv: int, D: int = D_SUPPORTED):
    """Split the fused projection output ``x`` [B, S, (Hq+2Hkv)*D] (row stride may
    exceed the width; D contiguous) into q, k, v [B, S, H, D] contiguous, with q and
    k rotated by ``freqs`` (fp32 [>=S, D/2, 2] = cos, sin)."""
    _need_gpu(x, freqs)
    _need_dtype("rope_qkv_fwd (bf16 only)", torch.bfloat16, x)
    B, S, W = x.shape
    assert x.stride(2) == 1 and x.stride(0) == S * x.stride(1), "rows of x must be evenly strided"
    assert W == (Hq + 2 * Hkv) * D, "x must hold [q | k | v] heads"
    assert freqs.dtype == torch.float32 and freqs.is_contiguous() and tuple(freqs.shape[1:]) == (D // 2, 2) \
        and freqs.shape[0] >= S, "freqs must be fp32 [>= S, D/2, 2] contiguous"
    dev = x.device
    q = torch.empty(B, S, Hq, D, dtype=torch.bfloat16, device=dev)
    k = torch.empty(B, S, Hkv, D, dtype=torch.bfloat16, device=dev)
    v = torch.empty(B, S, Hkv, D, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        rc = lib().lh_rope_qkv_fwd(_ptr(x), x.stride(1), _ptr(freqs), _ptr(q), _ptr(k), _ptr(v), B, S, Hq, Hkv, D,
                                   _stream(dev))
    _check(rc, "lh_rope_qkv_fwd")
    return q, k, v


def rope_qkv_bwd(dq, dk, dv, freqs, Hq: int, Hkv: int, D: int = D_SUPPORTED):
    """Adjoint of ``rope_qkv_fwd``: grads of q, k, v ([B, S, H, D], any strides with D
    contiguous) -> grad of the fused projection output [B, S, (Hq+2Hkv)*D]."""
    _need_gpu(dq, dk, dv, freqs)
    _need_dtype("rope_qkv_bwd (bf16 only)", torch.bfloat16, dq, dk, dv)
    B, S = dq.shape[:2]
    assert tuple(dq.shape) == (B, S, Hq, D) and tuple(dk.shape) == (B, S, Hkv, D) == tuple(dv.shape)
    assert freqs.dtype == torch.float32 and freqs.is_contiguous() and tuple(freqs.shape[1:]) == (D // 2, 2) \
        and freqs.shape[0] >= S, "freqs must be fp32 [>= S, D/2, 2] contiguous"
    dev = dq.device
    dx = torch.empty(B, S, (Hq + 2 * Hkv) * D, dtype=torch.bfloat16, device=dev)
    st = (ctypes.c_int64 * 9)(*[int(s) for g in (dq, dk, dv) for s in g.stride()[:3]])
    for g in (dq, dk, dv):
        assert g.stride(3) == 1, "head dimension must be contiguous"
    with torch.cuda.device(dev):
        rc = lib().lh_rope_qkv_bwd(_ptr(dq), _ptr(dk), _ptr(dv), ctypes.cast(st, _P), _ptr(freqs), _ptr(dx),
                                   dx.stride(1), B, S, Hq, Hkv, D, _stream(dev))
    _check(rc, "lh_rope_qkv_bwd")
    return dx


def rmsnorm_fwd(x, w, eps: float):
    """``y = (x * rsqrt(mean(x^2) + eps)) * w`` over the last dim; returns (y, rstd fp32)."""
    _need_gpu(x, w)
    _need_dtype("rmsnorm_fwd (bf16 only)", torch.bfloat16, x, w)
    x = x.contiguous()
    dim = x.shape[-1]
    assert w.shape == (dim,) and w.is_contiguous(), "weight must be [dim]"
    rows = x.numel() // dim
    y = torch.empty_like(x)
    rstd = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib().lh_rmsnorm_fwd(_ptr(x), _ptr(w), _ptr(y), _ptr(rstd), rows, dim, float(eps), _stream(x.device))
    _check(rc, "lh_rmsnorm_fwd")
    return y, rstd


def add_rmsnorm_fwd(x, r, w, eps: float):
    """``h = x + r`` (bf16) and ``y = RMSNorm(h)``; returns ``(h, y, rstd)``."""
    _need_gpu(x, r, w)
    _need_dtype("add_rmsnorm_fwd (bf16 only)", torch.bfloat16, x, r, w)
    x, r = x.contiguous(), r.contiguous()
    dim = x.shape[-1]
    rows = x.numel() // dim
    assert r.shape == x.shape and w.shape == (dim,) and w.is_contiguous()
    h = torch.empty_like(x)
    y = torch.empty_like(x)
    rstd = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib().lh_add_rmsnorm_fwd(_ptr(x), _ptr(r), _ptr(w), _ptr(h), _ptr(y), _ptr(rstd), rows, dim, float(eps),
                                      _stream(x.device))
    _check(rc, "lh_add_rmsnorm_fwd")
    return h, y, rstd


RMSNORM_BWD_PARTS = 512


def rmsnorm_bwd(dy, x, w, rstd, dres=None):
    """Grads of RMSNorm: ``(dx bf16 like x, dw bf16 like w)``; ``dres`` (optional) is
    added to dx (a residual branch's gradient)."""
    _need_gpu(dy, x, w, rstd)
    _need_dtype("rmsnorm_bwd (bf16 only)", torch.bfloat16, dy, x, w)
    dy, x, rstd = dy.contiguous(), x.contiguous(), rstd.contiguous()
    if dres is not None:
        dres = dres.contiguous()
    dim = x.shape[-1]
    rows = x.numel() // dim
    dx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    dw = torch.empty(w.shape, dtype=w.dtype, device=w.device)
    parts = min(RMSNORM_BWD_PARTS, rows)
    part = torch.empty(dim, parts, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib().lh_rmsnorm_bwd(_ptr(dy), _ptr(x), _ptr(w), _ptr(rstd), _ptr(dres), _ptr(dx), _ptr(dw),
                                  _ptr(part), parts, rows, dim, _stream(x.device))
    _check(rc, "lh_rmsnorm_bwd")
    return dx, dw


def swiglu_fwd(h):
    """``h`` [..., 2F] = [h1 | h3] -> ``silu(h1) * h3`` [..., F] (torch's roundings)."""
    _need_gpu(h)
    _need_dtype("swiglu_fwd (bf16 only)", torch.bfloat16, h)
    h = h.contiguous()
    F2 = h.shape[-1]
    rows = h.numel() // F2
    a = torch.empty(*h.shape[:-1], F2 // 2, dtype=torch.bfloat16, device=h.device)
    with torch.cuda.device(h.device):
        rc = lib().lh_swiglu_fwd(_ptr(h), _ptr(a), rows, F2 // 2, _stream(h.device))
    _check(rc, "lh_swiglu_fwd")
    return a


def swiglu_bwd(da, h):
    _need_gpu(da, h)
    _need_dtype("swiglu_bwd (bf16 only)", torch.bfloat16, da, h)
    da, h = da.contiguous(), h.contiguous()
    F2 = h.shape[-1]
    rows = h.numel() // F2
    dh = torch.empty(h.shape, dtype=h.dtype, device=h.device)
    with torch.cuda.device(h.device):
        rc = lib().lh_swiglu_bwd(_ptr(da), _ptr(h), _ptr(dh), rows, F2 // 2, _stream(h.device))
    _check(rc, "lh_swiglu_bwd")
    return dh


def splitk_sum(part):
    """``part`` fp32 [s, ...] -> bf16 sum over s (one rounding)."""
    _need_gpu(part)
    part = part.contiguous()
    out = torch.empty(part.shape[1:], dtype=torch.bfloat16, device=part.device)
    with torch.cuda.device(part.device):
        rc = lib().lh_splitk_sum(_ptr(part), _ptr(out), part.shape[0], out.numel(), _stream(part.device))
    _check(rc, "lh_splitk_sum")
    return out
