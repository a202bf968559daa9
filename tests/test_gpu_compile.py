"""The layer under torch.compile, as the reference's trainer runs it.

The reference compiles every transformer block with ``fullgraph=False``
(``configs/scorer/norm.toml:64-67``, ``lighthouse-attention.patch:540-548``) and
keeps its selection out of the graph with ``@torch.compiler.disable``.  Here the
layer is a registered custom op with a fake implementation, so dynamo traces
through it; compiled results must equal the eager ones bit for bit (the same
kernels run in the same order).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inductor_usable():
    try:
        import triton  # noqa: F401
        return True
    except Exception:
        return False


def test_layer_op_schema_and_fake(pkg, dev):
    """torch.library.opcheck: schema, fake (meta) implementation and autograd
    registration agree with the real op."""
    B, S, H, D = 1, 2048, 2, 128
    g = torch.Generator(device=dev).manual_seed(0)
    xs = [torch.randn(B, S, H, D, device=dev, generator=g).bfloat16().requires_grad_() for _ in range(3)]
    args = (*xs, 3, 4, 128, "reference", True, 0, False, None, None)
    torch.library.opcheck(torch.ops.lighthouse_amd.layer_fwd.default, args,
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))


@pytest.mark.parametrize("seq_major", [False, True])
def test_layer_compiled_fullgraph_bit_equal(pkg, dev, seq_major):
    B, S, H, D, L, p, k = 1, 4096, 2, 128, 3, 4, 256
    print(f"compiled layer fullgraph S={S} H={H} seq_major={seq_major}", flush=True)
    g = torch.Generator(device=dev).manual_seed(1)
    base = [torch.randn(B, S, H, D, device=dev, generator=g).bfloat16() for _ in range(3)]
    dout = torch.randn(B, H, S, D, device=dev, generator=g).bfloat16()

    def f(q, k_, v):
        out, idx = pkg.lighthouse_layer(q, k_, v, L, p, k, seq_major=seq_major)
        return out * 1.0, idx

    cf = torch.compile(f, fullgraph=True, backend="aot_eager")
    res = []
    for fn in (f, cf):
        xs = [b.clone().requires_grad_() for b in base]
        out, idx = fn(*xs)
        out.backward(dout)
        res.append((out.detach(), idx, [x.grad for x in xs]))
    (o1, i1, g1), (o2, i2, g2) = res
    assert torch.equal(i1, i2)
    assert torch.equal(o1, o2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("backend", ["inductor", "aot_eager"])
def test_block_compiled_like_the_reference(pkg, dev, backend):
    """One Lighthouse TransformerBlock of the 270M flavor (dim 1024, 8 heads of 128,
    norm scorer, L=3, p=4, k=1536), torch.compile(block, fullgraph=False), forward and
    backward at S=4096: output and every gradient bit-equal to the eager block."""
    if backend == "inductor" and not _inductor_usable():
        pytest.skip("inductor needs triton, which is not importable here")
    import dataclasses
    L3 = pkg.llama3
    args = dataclasses.replace(L3.llama3_args["ablation_270m_lighthouse_topk1536_pool4_lvl3"], vocab_size=256,
                               lighthouse_strict=False)
    args.update_from_config(seq_len=4096)
    torch.manual_seed(0)
    with torch.device(dev):
        block = L3.TransformerBlock(5, args)
        fc = L3.precompute_freqs_cis(args.dim // args.n_heads, 4096, args.rope_theta, args.rope_scaling_args)
    block.init_weights()
    L3.cast_params_(block, torch.bfloat16)
    assert block.attention._use_lighthouse and block.attention._fuses_rope()
    S = 4096
    print(f"compiled block backend={backend} S={S}", flush=True)
    g = torch.Generator(device=dev).manual_seed(2)
    x0 = torch.randn(1, S, args.dim, device=dev, generator=g).bfloat16()
    dy = torch.randn(1, S, args.dim, device=dev, generator=g).bfloat16()
    cblock = torch.compile(block, fullgraph=False, backend=backend)
    res = []
    for fn in (block, cblock):
        for prm in block.parameters():
            prm.grad = None
        x = x0.clone().requires_grad_()
        y = fn(x, fc)
        y.backward(dy)
        res.append((y.detach(), x.grad, {n: prm.grad.clone() for n, prm in block.named_parameters()}))
    (y1, dx1, gp1), (y2, dx2, gp2) = res
    assert torch.equal(y1, y2)
    assert torch.equal(dx1, dx2)
    for n in gp1:
        assert torch.equal(gp1[n], gp2[n]), n
