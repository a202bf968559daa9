"""The whole layer (forward + backward) captured into one HIP graph.

A graph records the layer's launches once: the native kernels take their
stream from torch's current stream, every persistent attention launch made
during capture gets a work-queue counter slot of its own, and the output sizes
are known on the host, so nothing in the path synchronizes.  Check mode
(index and work-queue checks, which synchronize) steps aside while the stream
is being captured.  Each replay, with eager work and synchronizations between
replays, must give the same bits as the eager layer on the same inputs.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("scorer", ["norm", "dilated", "gla"])
def test_layer_graph_replay(pkg, dev, scorer):
    B, S, H, L, p, k = 1, 4096, 2, 3, 4, 256
    print(f"layer graph replay scorer={scorer} S={S} H={H} k={k}", flush=True)
    N = pkg._native
    g = torch.Generator().manual_seed(21)
    xs = [torch.randn(B, S, H, 128, generator=g).bfloat16().to(dev) for _ in range(3)]
    dout = torch.randn(B, H, S, 128, generator=g).bfloat16().to(dev)
    kw = {}
    if scorer == "dilated":
        kw = {"dilation": 4}
    elif scorer == "gla":
        kw = {"dilation": 4, "gk": (torch.nn.functional.logsigmoid(torch.randn(B, S, H, generator=g)) / 16).to(dev)}

    def eager():
        xg = [x.clone().requires_grad_() for x in xs]
        out, idx = pkg.lighthouse_layer(*xg, num_levels=L, pooling_factor=p, topk=k, **kw)
        out.backward(dout)
        return out.detach(), idx, [x.grad for x in xg]

    ref_out, ref_idx, ref_grads = eager()

    static = [x.clone().requires_grad_() for x in xs]

    def step():
        out, idx = pkg.lighthouse_layer(*static, num_levels=L, pooling_factor=p, topk=k, **kw)
        out.backward(dout)
        return out, idx

    prev = N.set_check_indices(True)
    try:
        side = torch.cuda.Stream()  # warm-up on a side stream, as torch's capture recipe asks
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                for x in static:
                    x.grad = None
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for x in static:
            x.grad = None
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            g_out, g_idx = step()
    finally:
        N.set_check_indices(prev)

    for r in range(3):
        for x in static:  # the replay writes the gradient buffers whole
            x.grad.zero_()
        graph.replay()
        eager_again = eager()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(g_idx, ref_idx), f"replay {r}: indices differ from the eager layer"
        assert torch.equal(g_out, ref_out), f"replay {r}: output differs from the eager layer"
        for name, a, b in zip("qkv", (x.grad for x in static), ref_grads):
            assert torch.equal(a, b), f"replay {r}: d{name} differs from the eager layer"
        assert torch.equal(eager_again[0], ref_out)
    assert N.attn_status(dev) == 0
