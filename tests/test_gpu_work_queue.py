"""Work queues and block plans of the attention launches.

With more blocks than CUs the attention kernels run one workgroup per CU.  The
query-stationary kernels (forward, dQ) take a host-packed list of query blocks
when B*H is a multiple of 8 and a (b, h) has 1 to 3.5 blocks per CU (lh_attn.hip,
make_plan / plan_first / plan_next); otherwise, and always for dK/dV, the
workgroups take blocks from 8 per-XCD queues through device-scope atomic
counters that the last workgroup clears (wq_first / wq_next / wq_grid).  Which
workgroup runs a block does not change its arithmetic, so results must be
bit-equal to the same heads run one at a time, and every launch must find the
counters cleared by the one before (each test launches many times on one
stream; one case runs on two streams).  B*H below 8 leaves queues empty, so
those XCDs' workgroups start by taking blocks from the other queues.  Cases:
(9001, 1, 8), (12345, 2, 4), (8448, 1, 16) and the dilated scorer use plans for
the forward and dQ; (30000, 1, 3) and dense (30000, 1, 8) use queues for all
three kernels.  The oracle checks at full size (test_gpu_configs.py) run
with whichever applies.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rand(shape, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).bfloat16().to(dev)


def _per_head(pkg, xs, pxs, idx, split, B, H, n, do, lse_all, delta_all):
    """O, lse, dq, dk, dv of every (b, h) computed alone (B = H = 1)."""
    N = pkg._native
    outs = {k: [] for k in ("o", "lse", "dq", "dk", "dv")}
    for b in range(B):
        for h in range(H):
            sl = [x[b:b + 1, :, h:h + 1] for x in xs]
            if pxs is None:
                rows = N.Rows(*sl, (sl[0].stride(0), sl[0].stride(1), sl[0].stride(2)))
                ix = None
            else:
                psl = [x[b:b + 1, :, h:h + 1] for x in pxs]
                rows = N.Rows(*sl, (sl[0].stride(0), sl[0].stride(1), sl[0].stride(2)), *psl,
                              (psl[0].stride(0), psl[0].stride(1), psl[0].stride(2)), split=split)
                ix = idx[b:b + 1, h:h + 1].contiguous()
            o, lse = N.attn_fwd(rows, ix, 1, 1, n)
            d = do[b:b + 1, h:h + 1].contiguous()
            dq, dk, dv = N.attn_bwd(rows, ix, 1, 1, n, d, lse_all[b:b + 1, h:h + 1].contiguous(),
                                    delta_all[b:b + 1, h:h + 1].contiguous())
            for k, v in zip(("o", "lse", "dq", "dk", "dv"), (o, lse, dq, dk, dv)):
                outs[k].append(v)
    return {k: torch.cat(v, 1).reshape(B, H, *v[0].shape[2:]) for k, v in outs.items()}


@pytest.mark.parametrize("n,B,H", [(9001, 1, 8), (12345, 2, 4), (8448, 1, 16), (30000, 1, 3)])
def test_queue_gathered_bit_equal(pkg, dev, n, B, H):
    """Gathered rows (random distinct base and pooled rows), ragged n (partial last block)."""
    print(f"queues gathered n={n} B={B} H={H}", flush=True)
    N = pkg._native
    S, Sp = n, n // 3
    xs = [_rand((B, S, H, 128), 10 + i, dev) for i in range(3)]
    pxs = [_rand((B, Sp, H, 128), 20 + i, dev) for i in range(3)]
    g = torch.Generator().manual_seed(n)
    idx = torch.stack([torch.stack([torch.randperm(S + Sp, generator=g)[:n] for _ in range(H)])
                       for _ in range(B)]).int().to(dev)
    rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)), *pxs,
                  (pxs[0].stride(0), pxs[0].stride(1), pxs[0].stride(2)), split=S)
    o, lse = N.attn_fwd(rows, idx, B, H, n)
    do = _rand((B, H, n, 128), 30, dev)
    delta = (do.float() * o.float()).sum(-1)
    dq, dk, dv = N.attn_bwd(rows, idx, B, H, n, do, lse, delta)
    ref = _per_head(pkg, xs, pxs, idx, S, B, H, n, do, lse, delta)
    for name, got in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.equal(got, ref[name]), f"{name} differs from the per-head result"


@pytest.mark.parametrize("n,B,H", [(10000, 2, 4), (30000, 1, 8)])
def test_queue_dense_bit_equal(pkg, dev, n, B, H):
    """Identity row map (the dense layers' path)."""
    print(f"queues dense n={n} B={B} H={H}", flush=True)
    N = pkg._native
    xs = [_rand((B, n, H, 128), 40 + i, dev) for i in range(3)]
    rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)))
    o, lse = N.attn_fwd(rows, None, B, H, n)
    do = _rand((B, H, n, 128), 50, dev)
    delta = (do.float() * o.float()).sum(-1)
    dq, dk, dv = N.attn_bwd(rows, None, B, H, n, do, lse, delta)
    ref = _per_head(pkg, xs, None, None, None, B, H, n, do, lse, delta)
    for name, got in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.equal(got, ref[name]), f"{name} differs from the per-head result"


def test_queue_dilated_scores_bit_equal(pkg, dev):
    """Dilated scorer: 8 heads x dilation 4 = 32 virtual heads of 16 query blocks (512 blocks)."""
    S, H, dil, L, p = 16384, 8, 4, 3, 4
    print(f"queues dilated S={S} H={H} dil={dil}", flush=True)
    N = pkg._native
    xs = [_rand((1, S, H, 128), 60 + i, dev) for i in range(3)]
    _, _, S_tot = N.pyramid_lengths(S, L, p)
    sqk, skq = N.dilated_scores(*xs, dil, S_tot)
    for h in range(H):
        sl = [x[:, :, h:h + 1].contiguous() for x in xs]
        rq, rk = N.dilated_scores(*sl, dil, S_tot)
        assert torch.equal(sqk[:, h:h + 1, :S], rq[..., :S]), f"head {h}: qk scores differ"
        assert torch.equal(skq[:, h:h + 1, :S], rk[..., :S]), f"head {h}: kq scores differ"


def test_queue_two_streams(pkg, dev):
    """The same launches on the default stream and a second stream (separate counter slots), three times each."""
    n, B, H = 20000, 1, 8
    print(f"queues two streams n={n} B={B} H={H}", flush=True)
    N = pkg._native
    xs = [_rand((B, n, H, 128), 70 + i, dev) for i in range(3)]
    rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)))
    o, lse = N.attn_fwd(rows, None, B, H, n)
    do = _rand((B, H, n, 128), 80, dev)
    delta = (do.float() * o.float()).sum(-1)
    ref = (o, lse) + N.attn_bwd(rows, None, B, H, n, do, lse, delta)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    got = []
    for r in range(3):
        with torch.cuda.stream(side):
            a = N.attn_fwd(rows, None, B, H, n) + N.attn_bwd(rows, None, B, H, n, do, lse, delta)
        b = N.attn_fwd(rows, None, B, H, n) + N.attn_bwd(rows, None, B, H, n, do, lse, delta)
        got += [a, b]
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    for i, g in enumerate(got):
        for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), g, ref):
            assert torch.equal(x, y), f"launch {i}: {name} differs"


def test_queue_graph_replay(pkg, dev):
    """Attention fwd + bwd captured into a graph (queues for all three kernels at B*H = 3),
    replayed three times with eager attention calls and synchronizations between the
    replays; every replay bit-equal to the eager result.  The counters are cleared by the
    kernels themselves, so the graph holds no memset nodes."""
    n, B, H = 30000, 1, 3
    print(f"queues graph replay n={n} B={B} H={H}", flush=True)
    N = pkg._native
    xs = [_rand((B, n, H, 128), 90 + i, dev) for i in range(3)]
    rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)))
    o, lse = N.attn_fwd(rows, None, B, H, n)
    do = _rand((B, H, n, 128), 95, dev)
    delta = (do.float() * o.float()).sum(-1)
    ref = (o, lse) + N.attn_bwd(rows, None, B, H, n, do, lse, delta)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm-up off the capture, as torch recommends
        N.attn_fwd(rows, None, B, H, n)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = N.attn_fwd(rows, None, B, H, n) + N.attn_bwd(rows, None, B, H, n, do, lse, delta)
    for r in range(3):
        for x in got:
            x.zero_()
        torch.cuda.synchronize(dev)
        g.replay()
        eager = N.attn_fwd(rows, None, B, H, n)  # eager launches between replays
        torch.cuda.synchronize(dev)
        for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
            assert torch.equal(x, y), f"replay {r}: {name} differs from the eager result"
        assert torch.equal(eager[0], ref[0]), f"replay {r}: eager o differs"


def _hip_memcpy():
    """hipMemcpy of the HIP runtime torch has loaded (the library binds the same one)."""
    import ctypes
    h = ctypes.CDLL("libamdhip64.so.7")
    f = h.hipMemcpy
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return f


def _slot(pkg, dev):
    import ctypes
    p = ctypes.c_void_p()
    rc = pkg._native.lib().lh_attn_queue_slot(ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream),
                                              ctypes.byref(p))
    assert rc == 0 and p.value
    return p.value


def _slot_words(pkg, dev):
    import ctypes
    buf = (ctypes.c_uint32 * 32)()
    torch.cuda.synchronize(dev)
    assert _hip_memcpy()(ctypes.cast(buf, ctypes.c_void_p), ctypes.c_void_p(_slot(pkg, dev)), 128, 2) == 0
    return list(buf)


def _plant(pkg, dev, word, value):
    import ctypes
    buf = (ctypes.c_uint32 * 1)(value)
    torch.cuda.synchronize(dev)
    assert _hip_memcpy()(ctypes.c_void_p(_slot(pkg, dev) + 4 * word), ctypes.cast(buf, ctypes.c_void_p), 4, 1) == 0


# (word, value, flagged, outputs whole): a queue head past zero skips entries
# (blocks missing: flagged); a drained mask only stops other XCDs from taking
# entries their owners still take (outputs whole, nothing to flag); a done word
# not zero makes an early workgroup clear the counters while others run, and
# they sweep the queues again (outputs whole, flagged); the done word's block
# count off (flagged).  For B = 1, H = 3, queues 2, 5 and 7 hold one head each.
DIRT = [(2, 3, True, False), (8, (1 << 2) | (1 << 5), False, True), (10, 5, True, True), (11, 7, True, True)]


@pytest.mark.parametrize("word,value,flagged,whole", DIRT)
@pytest.mark.parametrize("kernel", ["fwd", "dkdv"])
def test_queue_dirty_slot_detected(pkg, dev, kernel, word, value, flagged, whole):
    """A counter slot planted not clear before a persistent launch: the launch's
    block count says so (lh_attn_status > 0, and check mode raises), the slot
    comes back cleared, and the next launch is bit-equal to a clean one."""
    n, B, H = 30000, 1, 3
    print(f"dirty slot kernel={kernel} word={word} value={value:#x}", flush=True)
    N = pkg._native
    xs = [_rand((B, n, H, 128), 110 + i, dev) for i in range(3)]
    rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)))
    o, lse = N.attn_fwd(rows, None, B, H, n)
    do = _rand((B, H, n, 128), 115, dev)
    delta = (do.float() * o.float()).sum(-1)

    def run():
        if kernel == "fwd":
            return N.attn_fwd(rows, None, B, H, n)
        return N.attn_bwd_dkdv(rows, None, B, H, n, do, lse, delta)

    ref = run()
    assert N.attn_status(dev) == 0, "a clean launch was flagged"
    assert not any(_slot_words(pkg, dev)), "a clean launch left its slot not cleared"
    _plant(pkg, dev, word, value)
    got = run()
    faults = N.attn_status(dev)
    assert (faults > 0) == flagged, f"status {faults}, expected flagged={flagged}"
    if whole:
        for x, y in zip(got, ref):
            assert torch.equal(x, y), "outputs of the dirty launch differ"
    assert not any(_slot_words(pkg, dev)), "the slot was not reset"
    again = run()
    assert N.attn_status(dev) == 0
    for x, y in zip(again, ref):
        assert torch.equal(x, y), "the launch after the reset differs"
    if flagged:  # the same through the Python check mode
        prev = N.set_check_indices(True)
        try:
            _plant(pkg, dev, word, value)
            with pytest.raises(N.LighthouseHipError, match="work-queue"):
                run()
        finally:
            N.set_check_indices(prev)
        assert not any(_slot_words(pkg, dev))
        for x, y in zip(run(), ref):
            assert torch.equal(x, y)


def test_queue_two_graphs_on_two_streams(pkg, dev):
    """Two graphs captured one after the other on torch's shared capture stream,
    then replayed at the same time on two streams (and beside eager launches on
    the default stream): each captured launch has counters of its own, so every
    replay is bit-equal to the eager result and no slot is flagged."""
    n, B, H = 30000, 1, 3
    print(f"two graphs n={n} B={B} H={H}", flush=True)
    N = pkg._native
    xs = [_rand((B, n, H, 128), 120 + i, dev) for i in range(3)]
    rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)))
    o, lse = N.attn_fwd(rows, None, B, H, n)
    do = _rand((B, H, n, 128), 125, dev)
    delta = (do.float() * o.float()).sum(-1)
    ref = (o, lse) + N.attn_bwd(rows, None, B, H, n, do, lse, delta)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm-up off the capture
        N.attn_fwd(rows, None, B, H, n)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graphs, outs = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(N.attn_fwd(rows, None, B, H, n) + N.attn_bwd(rows, None, B, H, n, do, lse, delta))
        graphs.append(g)
    streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    for r in range(3):
        for out in outs:
            for x in out:
                x.zero_()
        torch.cuda.synchronize(dev)
        for g, s in zip(graphs, streams):
            with torch.cuda.stream(s):
                g.replay()
        eager = N.attn_fwd(rows, None, B, H, n)
        torch.cuda.synchronize(dev)
        for i, out in enumerate(outs):
            for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), out, ref):
                assert torch.equal(x, y), f"replay {r}, graph {i}: {name} differs from the eager result"
        assert torch.equal(eager[0], ref[0])
    assert N.attn_status(dev) == 0


@pytest.mark.parametrize("n,B,H,gathered", [(18432, 1, 8, True), (30000, 1, 3, False), (5000, 2, 4, True)])
def test_backward_halves_bit_equal(pkg, dev, n, B, H, gathered):
    """lh_attn_bwd equals its two halves (lh_attn_bwd_dkdv, lh_attn_bwd_dq) bit
    for bit, over repeated launches on one stream's counter slot."""
    print(f"backward halves n={n} B={B} H={H} gathered={gathered}", flush=True)
    N = pkg._native
    S, Sp = n, n // 3
    xs = [_rand((B, S, H, 128), 130 + i, dev) for i in range(3)]
    if gathered:
        pxs = [_rand((B, Sp, H, 128), 140 + i, dev) for i in range(3)]
        g = torch.Generator().manual_seed(n)
        idx = torch.stack([torch.stack([torch.randperm(S + Sp, generator=g)[:n] for _ in range(H)])
                           for _ in range(B)]).int().to(dev)
        rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)), *pxs,
                      (pxs[0].stride(0), pxs[0].stride(1), pxs[0].stride(2)), split=S)
    else:
        idx = None
        rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)))
    o, lse = N.attn_fwd(rows, idx, B, H, n)
    do = _rand((B, H, n, 128), 150, dev)
    delta = (do.float() * o.float()).sum(-1)
    dk, dv = N.attn_bwd_dkdv(rows, idx, B, H, n, do, lse, delta)
    dq = N.attn_bwd_dq(rows, idx, B, H, n, do, lse, delta)
    for r in range(3):
        got = N.attn_bwd(rows, idx, B, H, n, do, lse, delta)
        for name, x, y in zip(("dq", "dk", "dv"), got, (dq, dk, dv)):
            assert torch.equal(x, y), f"launch {r}: {name} differs from the separate kernel's"
    assert N.attn_status(dev) == 0


@pytest.mark.parametrize("n,B,H", [(18432, 1, 8), (18432, 1, 4)])
def test_schedule_switch_bit_equal(pkg, dev, n, B, H):
    """lh_attn_set_schedule: the forward and backward with plans and queues
    off, each off alone and the default all give the same bits (cfg2's shape
    uses plans for the forward and dQ and queues for dK/dV; 4 heads use queues
    for all three)."""
    print(f"schedule switch n={n} B={B} H={H}", flush=True)
    N = pkg._native
    S, Sp = n, n // 3
    xs = [_rand((B, S, H, 128), 160 + i, dev) for i in range(3)]
    pxs = [_rand((B, Sp, H, 128), 170 + i, dev) for i in range(3)]
    g = torch.Generator().manual_seed(n + H)
    idx = torch.stack([torch.stack([torch.randperm(S + Sp, generator=g)[:n] for _ in range(H)])
                       for _ in range(B)]).int().to(dev)
    rows = N.Rows(*xs, (xs[0].stride(0), xs[0].stride(1), xs[0].stride(2)), *pxs,
                  (pxs[0].stride(0), pxs[0].stride(1), pxs[0].stride(2)), split=S)
    do = _rand((B, H, n, 128), 180, dev)

    def run():
        o, lse = N.attn_fwd(rows, idx, B, H, n)
        delta = (do.float() * o.float()).sum(-1)
        return (o, lse) + tuple(N.attn_bwd(rows, idx, B, H, n, do, lse, delta))

    ref = run()
    try:
        for plans, queues in ((False, False), (False, True), (True, False), (True, True)):
            N.set_attention_schedule(plans=plans, queues=queues)
            got = run()
            for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
                assert torch.equal(x, y), f"plans={plans} queues={queues}: {name} differs from the default"
    finally:
        N.set_attention_schedule()
    assert N.attn_status(dev) == 0
