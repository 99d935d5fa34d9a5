"""The library's RMSNorm (sparc_rms_norm_forward / _backward, the block
stack's pre-norm and final norm) against float64 autograd of
torch.nn.functional.rms_norm, and against torch's own bf16 RMSNorm."""
import ctypes

import pytest
import torch
import torch.nn.functional as F

from sparc_amd import _lib, stack

pytestmark = pytest.mark.gpu

SHAPES = [(1, 8), (37, 768), (200, 520), (64, 4096), (3, 5, 768)]


def _case(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    D = shape[-1]
    x = (torch.randn(*shape, generator=g, dtype=torch.float64) * 1.7 + 0.3).to(dtype)
    w = (1.0 + 0.5 * torch.randn(D, generator=g, dtype=torch.float64)).to(dtype)
    dy = torch.randn(*shape, generator=g, dtype=torch.float64).to(dtype)
    return x, w, dy


def _reference(x, w, dy, eps):
    xd = x.double().requires_grad_()
    wd = w.double().requires_grad_()
    y = F.rms_norm(xd, (x.shape[-1],), wd, eps)
    y.backward(dy.double())
    return y.detach(), xd.grad, wd.grad


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
def test_rms_norm_against_float64(shape, dtype):
    print(f"[case] rms norm {shape} {dtype}", flush=True)
    eps = 1e-6
    x, w, dy = _case(shape, dtype, seed=len(shape) * 1000 + shape[-1])
    norm = torch.nn.RMSNorm(shape[-1], eps=eps).to(dtype).cuda()
    with torch.no_grad():
        norm.weight.copy_(w)
    xc = x.cuda().requires_grad_()
    y = stack.rms_norm(norm, xc)
    y.backward(dy.cuda())
    ry, rdx, rdw = _reference(x, w, dy, eps)
    if dtype == torch.float32:
        tol = dict(rtol=2e-6, atol=2e-6)
        gtol = dict(rtol=1e-5, atol=1e-5 * rdw.abs().max().item())
    else:  # bf16 outputs: one rounding of the fp32 result (2^-8 relative)
        tol = dict(rtol=8e-3, atol=1e-6)
        gtol = dict(rtol=8e-3, atol=8e-3 * rdw.abs().max().item())
    torch.testing.assert_close(y.detach().cpu().double(), ry, **tol)
    torch.testing.assert_close(xc.grad.cpu().double(), rdx, rtol=tol["rtol"], atol=tol["rtol"] * rdx.abs().max().item())
    torch.testing.assert_close(norm.weight.grad.cpu().double(), rdw, **gtol)


def test_rms_norm_bf16_matches_torch():
    """bf16 at the stack's shape: the same values as torch's RMSNorm up to one
    bf16 rounding step, for y and dx; dweight (one fp32 sum rounded to bf16)
    within a rounding step too."""
    print("[case] rms norm bf16 vs torch", flush=True)
    x, w, dy = _case((512, 768), torch.bfloat16, seed=5)
    norm = torch.nn.RMSNorm(768, eps=1e-6).to(torch.bfloat16).cuda()
    with torch.no_grad():
        norm.weight.copy_(w)
    xa = x.cuda().requires_grad_()
    xb = x.cuda().requires_grad_()
    ya = stack.rms_norm(norm, xa)
    ya.backward(dy.cuda())
    dwa = norm.weight.grad.clone()
    norm.weight.grad = None
    yb = norm(xb)
    yb.backward(dy.cuda())
    dwb = norm.weight.grad.clone()

    def ulps(a, b):
        return ((a.float() - b.float()).abs() / b.float().abs().clamp_min(1e-3)).max().item()

    assert ulps(ya, yb) <= 2 ** -7
    assert ulps(xa.grad, xb.grad) <= 2 ** -6
    assert ulps(dwa, dwb) <= 2 ** -6


def test_rms_norm_backward_deterministic_and_empty():
    print("[case] rms norm determinism, rows = 0", flush=True)
    lib = _lib.load()
    x, w, dy = _case((1000, 768), torch.bfloat16, seed=9)
    x, w, dy = x.cuda(), w.cuda(), dy.cuda()
    rows, D = x.shape
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    P = _lib.ptr
    _lib.check(lib.sparc_rms_norm_forward(rows, D, _lib.SPARC_BF16, P(x), P(w), ctypes.c_float(1e-6), P(y), P(rstd),
                                          st), "forward")
    ws = torch.empty(lib.sparc_rms_norm_workspace_bytes(rows, D), dtype=torch.uint8, device="cuda")
    outs = []
    for _ in range(2):
        dx = torch.empty_like(x)
        dw = torch.full((D,), float("nan"), device="cuda")
        _lib.check(lib.sparc_rms_norm_backward(rows, D, _lib.SPARC_BF16, P(x), P(w), P(rstd), P(dy), P(dx), P(dw),
                                               P(ws), ws.numel(), st), "backward")
        outs.append((dx, dw))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    dw0 = torch.full((D,), float("nan"), device="cuda")
    _lib.check(lib.sparc_rms_norm_backward(0, D, _lib.SPARC_BF16, None, None, None, None, None, P(dw0), None, 0, st),
               "backward, no rows")
    torch.cuda.synchronize()
    assert torch.equal(dw0.cpu(), torch.zeros(D))


def test_rms_norm_rejects_unsupported_shapes():
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    t = torch.zeros(16, 12, device="cuda")
    r = torch.zeros(16, device="cuda")
    P = _lib.ptr
    assert lib.sparc_rms_norm_forward(16, 12, _lib.SPARC_F32, P(t), P(t), ctypes.c_float(1e-6), P(t), P(r), st) != 0
    assert lib.sparc_rms_norm_forward(16, 8192, _lib.SPARC_F32, P(t), P(t), ctypes.c_float(1e-6), P(t), P(r), st) != 0
