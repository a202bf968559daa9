"""Writes the committed selection fixtures in this directory from the CPU oracle.

    python tests/golden/make_golden.py

cfg1_selection.npz     benchmark config 1: B=1, H=8, D=128, S=4096, fp32 N(0,1) q/k/v
                       (torch seed 0), norm scorer, L=3, p=4, topk=1536 (outside the
                       reference kernel's domain, so per-tile compaction); scores and
                       the selected-index dump for both tie modes.
ties_4096_k256.npz     bf16 N(0,1) q/k (seed 1), H=4, S=4096, L=3, p=4, topk=256
                       (strict domain); bf16-rounded norms are tie-heavy.

The reference's own code is not run: it needs CUDA/NVRTC.  These vectors pin the
oracle against regressions; its correctness is pinned by tests/test_oracle.py.
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import lh_oracle as O  # noqa: E402


def case(name, S, H, L, p, k, strict, dtype, seed, manifest):
    g = torch.Generator().manual_seed(seed)
    xq = torch.randn(1, S, H, 128, generator=g)
    xk = torch.randn(1, S, H, 128, generator=g)
    xv = torch.randn(1, S, H, 128, generator=g)
    if dtype == "bf16":
        xq, xk, xv = (x.bfloat16() for x in (xq, xk, xv))
    sqk, skq, *_ = O.norm_scorer(xq, xk, xv, p, L)
    sqk = sqk.float().numpy()
    skq = skq.float().numpy()
    out = {"scores_qk": sqk, "scores_kq": skq}
    meta = {"S": S, "H": H, "L": L, "p": p, "topk": k, "strict": strict, "dtype": dtype, "seed": seed}
    for tie in ("reference", "lower_index"):
        idx = O.select_indices(sqk, skq, L, p, k, S, tie=tie, strict=strict)
        out[f"indices_{tie}"] = idx
        meta[f"sha256_{tie}"] = hashlib.sha256(idx.tobytes()).hexdigest()
    np.savez_compressed(os.path.join(HERE, name), **out)
    manifest[name] = meta


if __name__ == "__main__":
    manifest = {}
    case("cfg1_selection.npz", 4096, 8, 3, 4, 1536, False, "fp32", 0, manifest)
    case("ties_4096_k256.npz", 4096, 4, 3, 4, 256, True, "bf16", 1, manifest)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print(json.dumps(manifest, indent=1))
