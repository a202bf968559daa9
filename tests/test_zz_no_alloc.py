"""lh_rmsnorm_bwd_noalloc: the RMSNorm backward whose dw partials live in the
library's static device array instead of a caller workspace.

Called through the C ABI (ctypes), twice in a row on one GPU with the second
input smaller (fewer rows, narrower rows, no residual gradient), each call
checked against lh_rmsnorm_bwd with a caller-allocated workspace of the same
partial count (bit-equal: same kernels, same summation order) and against
torch autograd in fp32 (bf16 tolerance)."""
import ctypes

import pytest
import torch

from conftest import assert_close

pytestmark = pytest.mark.gpu

PARTS = 256


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _case(pkg, dev, rows, dim, with_dres, seed):
    lib = pkg._native.lib()
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(rows, dim, device=dev, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(dim, device=dev, generator=g)).bfloat16()
    dy = torch.randn(rows, dim, device=dev, generator=g).bfloat16()
    dres = torch.randn(rows, dim, device=dev, generator=g).bfloat16() if with_dres else None
    _, rstd = pkg._native.rmsnorm_fwd(x, w, 1e-5)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    dx_a, dw_a = torch.empty_like(x), torch.empty_like(w)
    rc = lib.lh_rmsnorm_bwd_noalloc(_ptr(dy), _ptr(x), _ptr(w), _ptr(rstd), _ptr(dres), _ptr(dx_a), _ptr(dw_a),
                                    rows, dim, st)
    assert rc == 0, lib.lh_strerror(rc)
    dx_b, dw_b = torch.empty_like(x), torch.empty_like(w)
    part = torch.empty(dim, PARTS, dtype=torch.float32, device=dev)
    rc = lib.lh_rmsnorm_bwd(_ptr(dy), _ptr(x), _ptr(w), _ptr(rstd), _ptr(dres), _ptr(dx_b), _ptr(dw_b), _ptr(part),
                            PARTS, rows, dim, st)
    assert rc == 0, lib.lh_strerror(rc)
    torch.cuda.synchronize()
    assert torch.equal(dx_a, dx_b)
    assert torch.equal(dw_a, dw_b)
    xr = x.float().requires_grad_()
    wr = w.float().requires_grad_()
    torch.nn.functional.rms_norm(xr, (dim,), wr, 1e-5).backward(dy.float())
    ref_dx = xr.grad + (dres.float() if dres is not None else 0)
    assert_close(dx_a, ref_dx, "dx")
    assert_close(dw_a, wr.grad, "dw")


def test_noalloc_rmsnorm_bwd_two_calls(pkg, dev):
    print("no-alloc rmsnorm bwd: rows 8192 dim 1024 with dres, then rows 1000 dim 512 without", flush=True)
    _case(pkg, dev, 8192, 1024, True, 1)
    _case(pkg, dev, 1000, 512, False, 2)


def test_noalloc_rejects_oversized_rows(pkg, dev):
    lib = pkg._native.lib()
    x = torch.zeros(4, 4104, dtype=torch.bfloat16, device=dev)
    r = torch.zeros(4, dtype=torch.float32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    assert lib.lh_rmsnorm_bwd_noalloc(_ptr(x), _ptr(x), _ptr(x), _ptr(r), None, _ptr(x), _ptr(x), 4, 4104, st) == 4
