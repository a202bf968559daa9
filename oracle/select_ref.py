"""ctypes binding of ``oracle/select_ref.c`` (test infrastructure only).

The C file restates the reference selection kernel slot by slot
(``src/lighthouse_selection_cuda.py:41-331,383-427``); see its header.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liblh_select_ref.so")
_lib = None

_ERR = {-1: "bad arguments", -2: "outside the reference's strict domain",
        -3: "slot overrun", -4: "output length mismatch", -5: "allocation failure"}


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        f = lib.lh_ref_select
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                      ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        _lib = lib
    return _lib


def select_indices_c(scores_qk, scores_kq, num_levels: int, pooling_factor: int, topk: int,
                     actual_seq_len: int, out_len: int, tie: str = "reference",
                     strict: bool = True) -> np.ndarray:
    """int32 ``[B, H, out_len]`` selected pyramid indices in causal order."""
    sq = np.ascontiguousarray(scores_qk, dtype=np.float32)
    sk = np.ascontiguousarray(scores_kq, dtype=np.float32)
    assert sq.shape == sk.shape and sq.ndim == 3
    B, H, S_tot = sq.shape
    out = np.empty((B, H, out_len), dtype=np.int32)
    rc = _load().lh_ref_select(sq.ctypes.data, sk.ctypes.data, B * H, S_tot, actual_seq_len,
                               num_levels, pooling_factor, topk, int(tie == "lower_index"),
                               0 if strict else 1, out.ctypes.data, out_len)
    if rc != 0:
        raise AssertionError(f"lh_ref_select: {_ERR.get(rc, rc)}")
    return out
