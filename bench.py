"""Lighthouse layer forward+backward throughput on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 200] [--workload cfg2] [--no-cpu-baseline]

A step is one forward + backward of one Lighthouse layer over one batch of
seeded synthetic N(0,1) bf16 tensors already resident in HBM: pyramid + scores
(norm, or dilated attention scores) -> top-k selection -> gathered causal
attention -> fan-out, then fan-out adjoint -> attention backward -> pyramid
backward.  The default workload is cfg2 (S=32768, H=8, k=2048, L=3, p=4,
norm scorer), the configuration the metric is quoted on; the other workloads
are the remaining benchmark configurations at their full sizes.  The model
workload cfg5 times one training step of the Llama3 270M Lighthouse model
instead (forward, backward, gradient clipping, AdamW).

Prints one JSON line.  `value` is tokens/s = B*S*steps / timed seconds.
`roofline` is for the kernel with the largest share of the step, timed with
HIP events recorded on the launch stream between consecutive native ops inside
the timed region.  `cpu_baseline` times the CPU oracle (a restatement of the
reference path, fp32) on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Lighthouse layer fwd+bwd tokens/s at S=32K,k=2048 bf16; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
MODEL_METRIC = "Llama3 270M Lighthouse training step tokens/s (fwd+bwd+AdamW), S=32K, bf16"

WORKLOADS = {
    # benchmark configs 2-4 and the Lighthouse-layer shape of config 5 (config 1 is the CPU-only case).
    # heavy_keys: fraction of key positions (the same for every head) scaled by 4, from a seeded draw.
    "cfg2": dict(B=1, H=8, S=32768, L=3, p=4, topk=2048, strict=True, scorer="norm"),
    "cfg3_k1536": dict(B=1, H=8, S=65536, L=3, p=4, topk=1536, strict=False, scorer="norm", heavy_keys=0.05),
    "cfg3_k3072": dict(B=1, H=8, S=65536, L=3, p=4, topk=3072, strict=False, scorer="norm", heavy_keys=0.05),
    "cfg3_k6144": dict(B=1, H=8, S=65536, L=3, p=4, topk=6144, strict=False, scorer="norm", heavy_keys=0.05),
    "cfg4": dict(B=1, H=8, S=131072, L=5, p=2, topk=1536, strict=False, scorer="dilated", dilation=4),
    "cfg5_layer": dict(B=1, H=8, S=32768, L=3, p=4, topk=1536, strict=False, scorer="norm"),
    # the reference's GLA scorer config (configs/scorer/gla.toml: k=2048, p=4, L=3) at the cfg2 shape,
    # gate logsigmoid(N(0,1)) / 16 as the patch's logsigmoid(wg(x)) / 16
    "gla": dict(B=1, H=8, S=32768, L=3, p=4, topk=2048, strict=True, scorer="gla", dilation=4),
}
D = 128
# Model workloads: one training step (forward, backward, clip, AdamW) of the Llama3 model.
MODEL_WORKLOADS = {
    # benchmark config 5: the 270M flavor with Lighthouse (norm, L=3, p=4, k=1536) on layers 2-27,
    # dense causal attention on layers 0, 1, 28, 29; byte-level vocabulary; batch 1 x 32768 tokens.
    "cfg5": dict(flavor="ablation_270m_lighthouse_topk1536_pool4_lvl3", B=1, S=32768, vocab=256,
                 layer="cfg5_layer"),
}


def make_inputs(w, torch, device, seed=1234, heads=None):
    """Seeded synthetic layer inputs of workload `w`: bf16 q, k, v [B, S, H, D]
    and upstream grad [B, H, S, D], drawn N(0,1) in fp32 and cast.  `heads`
    keeps a subset of the H heads (the draw is the same as for all heads)."""
    B, H, S = w["B"], w["H"], w["S"]
    g = torch.Generator(device=device).manual_seed(seed)
    xs = [torch.randn(B, S, H, D, device=device, generator=g) for _ in range(3)]
    if w.get("heavy_keys"):
        pos = torch.randperm(S, device=device, generator=g)[: int(round(w["heavy_keys"] * S))]
        xs[1][:, pos] *= 4.0
    dout = torch.randn(B, H, S, D, device=device, generator=g)
    gk = None
    if w["scorer"] == "gla":
        gk = torch.nn.functional.logsigmoid(torch.randn(B, S, H, device=device, generator=g)) / 16
    if heads is not None:
        hs = torch.as_tensor(heads, device=device)
        xs = [x.index_select(2, hs) for x in xs]
        dout = dout.index_select(1, hs)
        gk = gk.index_select(2, hs) if gk is not None else None
    xs = [x.bfloat16() for x in xs]
    if gk is not None:
        return xs, dout.bfloat16(), gk.bfloat16()
    return xs, dout.bfloat16()


def make_layer(w, pkg):
    """LighthouseLocal for workload `w`, built as the reference model builds it."""
    if w["scorer"] == "dilated":
        scorer = pkg.DilatedLighthouseScorer(head_dim=D, dilation=w["dilation"], pooling_factor=w["p"],
                                             levels=w["L"])
    elif w["scorer"] == "gla":
        scorer = pkg.DilatedLighthouseGLAScorer(head_dim=D, dilation=w["dilation"], pooling_factor=w["p"],
                                                levels=w["L"])
    else:
        scorer = pkg.DialatedLighthouseNormScorer(pooling_factor=w["p"], levels=w["L"])
    return pkg.LighthouseLocal(attention=None, scorer=scorer, num_levels=w["L"], pooling_factor=w["p"],
                               topk=w["topk"], strict=w["strict"])


def algorithmic_work(w, S_sel):
    """Per-launch algorithmic work of each native op: (kind, amount) with kind
    'bytes' (HBM-bound) or 'flop' (MFMA-bound).  bf16 = 2 bytes, fp32 = 4."""
    B, H, S, L, p = w["B"], w["H"], w["S"], w["L"], w["p"]
    S_tot = sum(S // p ** l for l in range(L))
    pairs = S_sel * (S_sel + 1) / 2 * B * H  # causal (query, key) pairs
    e = 2
    if w["scorer"] in ("dilated", "gla"):
        # base scores come in (fp32, two tensors); pooled levels of rows and scores go out
        pyr = 3 * S * H * D * e + 3 * (S_tot - S) * H * D * e + 2 * S * H * 4 + 2 * (S_tot - S) * H * 4
    else:
        pyr = 3 * S * H * D * e + 3 * (S_tot - S) * H * D * e + 2 * S_tot * H * 4
    work = {
        "pyramid": ("bytes", pyr * B),
        "select": ("bytes", (2 * S_sel * H * 4 + S_sel * H * 4 + S_tot * H * 4) * B),
        "attn_fwd": ("flop", 4 * D * pairs),            # S = Q K^T and O = P V
        "scatter_fwd": ("bytes", ((S_sel + S) * H * D * e + S_tot * H * 4) * B),
        "scatter_bwd": ("bytes", ((S_sel + S) * H * D * e + S_sel * H * D * e + S_sel * H * 4 * 2) * B),
        "attn_bwd_dkdv": ("flop", 8 * D * pairs),       # S, dP, dV, dK passes
        "attn_bwd_dq": ("flop", 2 * D * pairs),         # the dQ pass (S and dP are recomputed)
        "pyramid_bwd": ("bytes", (3 * S_sel * H * D * e + 3 * S * H * D * e + S_tot * H * 4) * B),
    }
    if w["scorer"] == "dilated":
        sd = S // w["dilation"]
        # two dense causal attentions (q->k, k->q) over dil*H virtual heads of length S/dil
        work["dilated_scores"] = ("flop", 2 * 4 * D * (w["dilation"] * H) * sd * (sd + 1) / 2 * B)
    if w["scorer"] == "gla":
        # chunked simple GLA, both directions, per 64-token chunk of each virtual head:
        # Q K^T and A V (64 x 64 x D each), Q H and K^T V (64 x D x D each)
        chunks = -(-(S // w["dilation"]) // 64) * w["dilation"] * H * B
        work["gla_scores"] = ("flop", 2 * chunks * 2 * (2 * 64 * 64 * D + 2 * 64 * D * D))
    return work


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE and WRITE_SIZE, each scaled by what the counter reads
    for a plain copy of known size), or None if that kernel was not profiled."""
    try:
        with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
            return json.load(f)["bytes_per_launch"].get(workload, {}).get(kernel)
    except (OSError, ValueError, KeyError):
        return None


def run_gpu(args, pkg, torch):
    w = WORKLOADS[args.workload]
    B, H, S, L, p, k, strict = (w[n] for n in ("B", "H", "S", "L", "p", "topk", "strict"))
    dev = torch.device("cuda:0")
    xs, dout, *gate = make_inputs(w, torch, dev)
    xs = [x.requires_grad_() for x in xs]
    kw = {"gk": gate[0]} if gate else {}
    layer = make_layer(w, pkg)
    S_sel = pkg._native.geometry(S, L, p, k, strict)[3]

    def step():
        for x in xs:
            x.grad = None
        out = layer(*xs, **kw)
        out.backward(dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    marks = []

    def hook(name):
        ev = torch.cuda.Event(enable_timing=True)
        st = torch.cuda.current_stream()
        ev.record(st)
        marks.append((name, ev, st.cuda_stream))

    sel_mod = pkg.lighthouse_selection
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    sel_mod.set_op_hook(hook)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    sel_mod.set_op_hook(None)

    ms_step = start.elapsed_time(end) / args.steps
    wall_ms_step = (t1 - t0) * 1e3 / args.steps
    kernels = op_stats(marks, algorithmic_work(w, S_sel))
    dom = max(kernels, key=lambda n: kernels[n]["ms"])
    roofline = roofline_of(kernels, dom, args.workload)
    tokens_per_s = B * S / (ms_step * 1e-3)
    cfg = {"workload": f"lighthouse_layer_fwd_bwd_{args.workload}", "B": B, "H": H, "D": D, "S": S,
           "num_levels": L, "pooling_factor": p, "topk": k, "scorer": w["scorer"], "S_sel": S_sel,
           "strict": strict, "parallelism": "single GPU"}
    if w["scorer"] == "dilated":
        cfg["dilation"] = w["dilation"]
    if w.get("heavy_keys"):
        cfg["heavy_keys"] = w["heavy_keys"]
    # the backward pair (dK/dV + dQ kernels) against the attention backward's algorithmic
    # work, 2.5x the forward's (S, dP, dV, dK and dQ products; the dQ kernel's recomputed
    # S and dP are not counted); with the two-stream schedule the kernels overlap, and
    # the pair's time is the longer of the two
    kd, kq = kernels["attn_bwd_dkdv"], kernels["attn_bwd_dq"]
    two = sel_mod._bwd_streams >= 2
    pair_ms = max(kd["ms"], kq["ms"]) if two else kd["ms"] + kq["ms"]
    pair_work = kd["work"] + kq["work"]
    sched = "two streams" if two else "one stream, dK/dV then dQ"
    pair = {"ms": round(pair_ms, 4), "algorithmic_tflop": round(pair_work / 1e12, 4),
            "achieved": round(pair_work / (pair_ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
            "frac": round(pair_work / (pair_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "schedule": sched}
    return {
        "tokens_per_s": tokens_per_s, "ms_step": ms_step, "wall_ms_step": wall_ms_step, "config": cfg,
        "roofline": roofline, "kernels": kernels, "backward_pair": pair,
    }


def op_stats(marks, work):
    """Per-op average launch time from (name, event, stream) marks: each op is timed
    from the previous mark on its own stream, and a ``*_start`` mark opens a run of
    consecutive ops on its stream (ops on a side stream are timed on that stream)."""
    per_op = {}
    prev = {}
    for name, ev, st in marks:
        if name.endswith("_start"):
            prev[st] = ev
            continue
        per_op.setdefault(name, []).append(prev[st].elapsed_time(ev))
        prev[st] = ev
    kernels = {}
    for name, ts in per_op.items():
        avg_ms = sum(ts) / len(ts)
        kind, amount = work[name]
        if kind == "flop":
            ach, peak, unit = amount / (avg_ms * 1e-3) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"
        else:
            ach, peak, unit = amount / (avg_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        kernels[name] = {"ms": round(avg_ms, 4), "achieved": round(ach, 2), "unit": unit,
                         "frac": round(ach / peak, 4), "work": amount, "launches": len(ts)}
    return kernels


def profiled_counters(workload, kernel):
    """Matrix-core busy share and effective clock of `kernel` from the committed
    rocprofv3 counter summary (SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "mfma_counters.json")) as f:
            return json.load(f)["per_kernel"].get(workload, {}).get(kernel)
    except (OSError, ValueError, KeyError):
        return None


def roofline_of(kernels, dom, workload):
    kd = kernels[dom]
    mfma = kd["unit"] == "TFLOP/s"
    r = {"kernel": dom, "bound": "mfma" if mfma else "hbm", "achieved": kd["achieved"],
         "peak": BF16_PEAK_TFLOPS if mfma else HBM_PEAK_GBS, "unit": kd["unit"], "frac": kd["frac"],
         "traffic": measured_traffic(workload, dom)}
    if r["traffic"] is not None:
        r["traffic_source"] = ("profiles/hbm_traffic.json: rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 per launch "
                               "(copy-calibrated) of an earlier run of this command, not measured in this run")
    c = profiled_counters(workload, dom) if mfma else None
    if c is not None:
        r["mfma_busy_pct_profiled"] = c["mfma_busy_pct"]
        r["clock_ghz_profiled"] = c["clock_ghz"]
        r["counters_source"] = ("profiles/mfma_counters.json: rocprofv3 SQ_VALU_MFMA_BUSY_CYCLES / "
                                "(GRBM_GUI_ACTIVE per XCD x 1024 SIMDs) of an earlier run of this command")
    return r


def run_model(args, pkg, torch):
    """One training step of the Llama3 model per step (MODEL_WORKLOADS)."""
    import dataclasses
    m = MODEL_WORKLOADS[args.workload]
    wl = WORKLOADS[m["layer"]]
    L3 = pkg.llama3
    B, S = m["B"], m["S"]
    margs = dataclasses.replace(L3.llama3_args[m["flavor"]], vocab_size=m["vocab"], lighthouse_strict=wl["strict"])
    margs.update_from_config(seq_len=S)
    dev = torch.device("cuda:0")
    trainer = L3.Trainer(margs, dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(1234)
    tok = torch.randint(0, m["vocab"], (B, S + 1), device=dev, generator=g)
    x, y = tok[:, :-1].contiguous(), tok[:, 1:].contiguous()
    for _ in range(args.warmup):
        trainer.step(x, y)
    torch.cuda.synchronize()
    marks = []

    def hook(name):
        ev = torch.cuda.Event(enable_timing=True)
        st = torch.cuda.current_stream()
        ev.record(st)
        marks.append((name, ev, st.cuda_stream))

    sel_mod = pkg.lighthouse_selection
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    sel_mod.set_op_hook(hook)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        loss = trainer.step(x, y)
    end.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    sel_mod.set_op_hook(None)
    ms_step = start.elapsed_time(end) / args.steps
    S_sel = pkg._native.geometry(S, wl["L"], wl["p"], wl["topk"], wl["strict"])[3]
    work = algorithmic_work(dict(wl, B=B), S_sel)
    H = margs.n_heads
    if wl["scorer"] == "norm":
        # the model's norm-scorer layers rotate q and k inside the pyramid pass,
        # which also writes the rotated rows (read by the attention gathers)
        kind, amount = work["pyramid"]
        work["pyramid"] = (kind, amount + 2 * S * H * D * 2 * B)
    dense_pairs = S * (S + 1) / 2 * B * H
    work["dense_attn_fwd"] = ("flop", 4 * D * dense_pairs)
    work["dense_attn_bwd"] = ("flop", 10 * D * dense_pairs)   # dK/dV (4 products) + dQ (1), as in the layer
    kernels = op_stats(marks, work)
    for k in kernels.values():
        k["ms_per_step"] = round(k["ms"] * k["launches"] / args.steps, 3)
    dom = max(kernels, key=lambda n: kernels[n]["ms_per_step"])
    native_ms = sum(k["ms_per_step"] for k in kernels.values())
    n_light = sum(1 for b in trainer.model.layers.values() if b.attention._use_lighthouse)
    cfg = {"workload": f"llama3_train_step_{args.workload}", "flavor": m["flavor"], "B": B, "S": S,
           "vocab_size": margs.vocab_size, "dim": margs.dim, "n_layers": margs.n_layers, "n_heads": H,
           "ffn_hidden": L3.ffn_hidden_dim(margs.hidden_dim, margs.multiple_of, margs.ffn_dim_multiplier),
           "lighthouse_layers": n_light, "dense_layers": margs.n_layers - n_light,
           "num_levels": wl["L"], "pooling_factor": wl["p"], "topk": wl["topk"], "S_sel": S_sel,
           "strict": wl["strict"], "params": L3.num_params(trainer.master),
           "optimizer": "AdamW fp32 masters, bf16 compute, clip 1.0", "parallelism": "single GPU"}
    return {"tokens_per_s": B * S / (ms_step * 1e-3), "ms_step": ms_step,
            "wall_ms_step": (t1 - t0) * 1e3 / args.steps, "config": cfg,
            "roofline": roofline_of(kernels, dom, args.workload), "kernels": kernels,
            "native_ms_per_step": round(native_ms, 3), "final_loss": round(loss.item(), 4)}


def _cpu_model():
    """Host CPU model name (lscpu's "Model name"), or None."""
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, ValueError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def run_cpu_baseline(args, torch):
    """CPU oracle (fp32, the reference path restated) on a bounded sample: the same
    workload with `--cpu-heads` of its H heads (2 for the norm scorer, 1 for the
    dilated one), scaled to all heads.  One warm-up run, then the median of
    `--cpu-runs` timed runs each of the forward alone and of forward + backward."""
    import statistics
    from oracle import lh_oracle as O
    w = WORKLOADS[args.workload]
    B, H, S, L, p, k, strict = (w[n] for n in ("B", "H", "S", "L", "p", "topk", "strict"))
    hs = max(1, min(args.cpu_heads if args.cpu_heads else (1 if w["scorer"] in ("dilated", "gla") else 2), H))
    xs0, dout, *gate = make_inputs(w, torch, torch.device("cpu"), seed=99, heads=list(range(hs)))
    dout = dout.float()
    gk = gate[0].float() if gate else None

    def run(backward):
        xs = [x.float().requires_grad_(backward) for x in xs0]
        t0 = time.perf_counter()
        out, _ = O.lighthouse_layer(*xs, L, p, k, scorer=w["scorer"], dilation=w.get("dilation", 4), strict=strict,
                                    gk=gk)
        if backward:
            out.backward(dout)
        return time.perf_counter() - t0

    run(True)  # warm-up
    t_fb = statistics.median(run(True) for _ in range(args.cpu_runs))
    with torch.no_grad():
        t_f = statistics.median(run(False) for _ in range(args.cpu_runs))
    scale = H / hs
    tok = lambda t: round(B * S / (t * scale), 2)  # noqa: E731
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count()
    return {"value": tok(t_fb), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "fwd_value": tok(t_f), "nproc": nproc, "cpu_model": _cpu_model(),
            "sample": f"oracle layer fp32 on {hs} of {H} heads (B={B}, S={S}): 1 warm-up, median of "
                      f"{args.cpu_runs} runs, fwd+bwd {t_fb:.2f} s, fwd {t_f:.2f} s; scaled x{H // hs} to all "
                      "heads; value = fwd+bwd, fwd_value = fwd only"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps before the timed ones (default: 200 for the layer workloads, about "
                         "0.6 s at cfg2, since the GPU clock settles over the first fraction of a second of "
                         "load and the timed steps should see it settled; 5 for the model step)")
    ap.add_argument("--workload", default="cfg2", choices=sorted(WORKLOADS) + sorted(MODEL_WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=0,
                    help="heads in the CPU sample (0: 2 for the norm scorer, 1 for the dilated one)")
    ap.add_argument("--cpu-runs", type=int, default=3, help="timed CPU runs per figure (median reported)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB five times (reference kernel of known "
                         "traffic for the FETCH_SIZE / WRITE_SIZE counters) and exit")
    ap.add_argument("--schedule", default="auto", choices=["auto", "noplan", "noqueue", "plain"],
                    help="attention launch scheduling, for A/B runs: auto (plans and work queues where the "
                         "shape calls for them), noplan, noqueue, or plain (one block per workgroup)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU per process and has no multi-GPU path; "
              f"--gpus {args.gpus} is not supported (use --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import torch
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 5}))
        return
    import __graft_entry__ as G
    pkg = G.load_package()
    if args.schedule != "auto":
        pkg._native.set_attention_schedule(plans=args.schedule not in ("noplan", "plain"),
                                           queues=args.schedule not in ("noqueue", "plain"))
    model = args.workload in MODEL_WORKLOADS
    if args.warmup is None:
        args.warmup = 5 if model else 200
    r = run_model(args, pkg, torch) if model else run_gpu(args, pkg, torch)
    # the CPU oracle covers the layer; a CPU training step of the 270M model is not sampled
    cpu = None if (args.no_cpu_baseline or model) else run_cpu_baseline(args, torch)
    line = {
        "metric": MODEL_METRIC if model else METRIC,
        "value": round(r["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": ("synthetic: uniform random token ids [B, S+1] (inputs and shifted labels), random-init weights"
                 if model else
                 "synthetic: seeded N(0,1) bf16 q/k/v [B,S,H,D] and upstream grad [B,H,S,D], resident in HBM"
                 + ("; 5% of key positions x4" if WORKLOADS[args.workload].get("heavy_keys") else "")),
        "config": r["config"],
        "roofline": r["roofline"],
        "cpu_baseline": cpu,
        "kernels": r["kernels"],
        "wall_ms_per_step": round(r["wall_ms_step"], 4),
    }
    if args.schedule != "auto":
        line["config"]["schedule"] = args.schedule
    for key in ("backward_pair", "native_ms_per_step", "final_loss"):
        if key in r:
            line[key] = r[key]
    print(json.dumps(line))


if __name__ == "__main__":
    main()
