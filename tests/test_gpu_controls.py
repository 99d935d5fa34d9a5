"""The controls entry points (make_controls, sparc-kernal/forward/control.py:
129-139) through the C ABI against autograd of the float64 oracle: eta and
delta (fp32 outputs, tolerance 1e-4), the in-place input gradient (1e-4 fp32,
2e-2 bf16) and the direction gradients (fp32, 1e-4)."""

import pytest
import torch

from oracle import sparc_oracle as O
from sparc_amd import _lib

pytestmark = pytest.mark.gpu


def rel_err(got, ref):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    return (got - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)


@pytest.mark.parametrize("rows,width,dtype", [
    (1, 8, torch.float32),
    (37, 24, torch.float32),
    (1000, 768, torch.bfloat16),
    (513, 32768, torch.bfloat16),
    (2049, 1032, torch.float32),
    (8_500_000, 8, torch.float32),  # more than 65535 row blocks: the workgroups loop
    (0, 64, torch.float32),
])
def test_controls_match_oracle(rows, width, dtype):
    print(f"[case] controls rows={rows} width={width} dtype={dtype}", flush=True)
    lib = _lib.load()
    g = torch.Generator().manual_seed(rows + width)
    x = torch.randn(rows, width, generator=g).to(dtype)
    u = 0.5 * torch.randn(2, width + 1, generator=g, dtype=torch.float64) / width ** 0.5
    deta = torch.randn(rows, generator=g)
    ddelta = torch.randn(rows, generator=g)
    dx0 = torch.randn(rows, width, generator=g).to(dtype)
    # oracle (float64 autograd)
    x64 = x.double().requires_grad_()
    u0, u1 = u[0].clone().requires_grad_(), u[1].clone().requires_grad_()
    eta_r, delta_r = O.controls(x64, u0, u1)
    gx, gu0, gu1 = torch.autograd.grad((eta_r * deta.double()).sum() + (delta_r * ddelta.double()).sum(),
                                       [x64, u0, u1])
    # HIP
    dev = torch.device("cuda", 0)
    xd, dxd = x.to(dev), dx0.to(dev)
    ud = u.float().to(dev)
    pd, rd = ud[0].clone(), ud[1].clone()
    eta = torch.empty(rows, device=dev)
    delta = torch.empty(rows, device=dev)
    P = _lib.ptr
    st = _lib.stream_of(dev)
    io = _lib.io_code(dtype)
    _lib.check(lib.sparc_controls_forward(rows, width, io, P(xd), P(pd), P(rd), P(eta), P(delta), st), "fwd")
    dpd = torch.full((width + 1,), float("nan"), device=dev)
    drd = torch.full((width + 1,), float("nan"), device=dev)
    ws = torch.empty(lib.sparc_controls_workspace_bytes(rows, width), dtype=torch.uint8, device=dev)
    detad, ddeltad = deta.to(dev), ddelta.to(dev)  # held until the kernels have run
    _lib.check(lib.sparc_controls_backward(rows, width, io, P(xd), P(pd), P(rd), P(eta), P(delta),
                                           P(detad), P(ddeltad), P(dxd), P(dpd), P(drd), P(ws),
                                           ws.numel(), st), "bwd")
    torch.cuda.synchronize()
    if rows == 0:
        assert (dpd == 0).all() and (drd == 0).all()
        return
    assert rel_err(eta, eta_r) <= 1e-4
    assert rel_err(delta, delta_r) <= 1e-4
    assert rel_err(dxd, dx0.double() + gx) <= (1e-4 if dtype == torch.float32 else 2e-2)
    assert rel_err(dpd, gu0) <= 1e-4
    assert rel_err(drd, gu1) <= 1e-4


def test_make_controls_autograd_matches_oracle():
    """sparc_amd.make_controls (HIP) on a module's parameters: values and the
    gradients of x and both directions."""
    print("[case] make_controls autograd B=2 L=33 width=48 fp32", flush=True)
    from sparc_amd import SPARCMixer, make_controls
    torch.manual_seed(0)
    m = SPARCMixer(48)
    with torch.no_grad():
        m.phase_direction.normal_(0, 0.2)
        m.radial_direction.normal_(0, 0.2)
    x = torch.randn(2, 33, 48)
    w_eta, w_delta = torch.randn(2, 33), torch.randn(2, 33)
    x64 = x.double().requires_grad_()
    pdir = m.phase_direction.detach().double().requires_grad_()
    rdir = m.radial_direction.detach().double().requires_grad_()
    e_r, d_r = O.controls(x64, pdir, rdir)
    ref = torch.autograd.grad((e_r * w_eta.double()).sum() + (d_r * w_delta.double()).sum(), [x64, pdir, rdir])
    m = m.cuda()
    xd = x.cuda().requires_grad_()
    e, d = make_controls(m, xd)
    got = torch.autograd.grad((e * w_eta.cuda()).sum() + (d * w_delta.cuda()).sum(),
                              [xd, m.phase_direction, m.radial_direction])
    assert rel_err(e, e_r) <= 1e-4 and rel_err(d, d_r) <= 1e-4
    for a, b in zip(got, ref):
        assert rel_err(a, b) <= 1e-4
