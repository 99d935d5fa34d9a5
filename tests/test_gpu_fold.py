"""The library's controls fold (sparc_controls_fold / _backward: the
controls' directions folded through the block stack's input projection)
against float64 products, and the stack's projected mixer with and without
it."""
import pytest
import torch

from sparc_amd import _lib

pytestmark = pytest.mark.gpu

SHAPES = [(8, 8), (64, 16), (65, 24), (200, 520), (1536, 768), (24576, 768), (96, 4096)]


def _case(width, dim, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(width, dim, generator=g, dtype=torch.float64) / dim ** 0.5).to(dtype)
    u = torch.randn(2, width + 1, generator=g, dtype=torch.float64).float()
    gf = torch.randn(2, dim + 1, generator=g, dtype=torch.float64).float()
    return w, u, gf


def _fold(w, u):
    lib = _lib.load()
    width, dim = w.shape
    wc, uc = w.cuda(), u.cuda()
    f = torch.full((2, dim + 1), float("nan"), device="cuda")
    fpad = torch.full((2, (dim + 4) // 4 * 4), float("nan"), device="cuda")
    ws = torch.empty(lib.sparc_controls_fold_workspace_bytes(width, dim), dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    P = _lib.ptr
    _lib.check(lib.sparc_controls_fold(width, dim, _lib.io_code(w.dtype), P(wc), P(uc[0]), P(uc[1]), P(fpad[0]),
                                       P(fpad[1]), P(ws), ws.numel(), st), "sparc_controls_fold")
    f.copy_(fpad[:, :dim + 1])
    return f.cpu()


def _unfold(w, gf, u=None, dw=None):
    """(ddirections, dweight after the in-place add, or None)"""
    lib = _lib.load()
    width, dim = w.shape
    wc, gc = w.cuda(), gf.cuda()
    uc = u.cuda() if u is not None else None
    dwc = dw.cuda() if dw is not None else None
    du = torch.full((2, width + 1), float("nan"), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    P = _lib.ptr
    _lib.check(lib.sparc_controls_fold_backward(width, dim, _lib.io_code(w.dtype), P(wc),
                                                P(uc[0]) if uc is not None else None,
                                                P(uc[1]) if uc is not None else None, P(gc[0]), P(gc[1]),
                                                P(du[0]), P(du[1]), P(dwc), st), "sparc_controls_fold_backward")
    return du.cpu(), (dwc.cpu() if dwc is not None else None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{w}x{d}" for w, d in SHAPES])
def test_fold_against_float64(shape, dtype):
    print(f"[case] controls fold {shape} {dtype}", flush=True)
    width, dim = shape
    w, u, gf = _case(width, dim, dtype, seed=width * 7 + dim)
    wd = w.double()
    # forward: f_k = [u_k[:width] W, u_k[width]]
    ref = torch.cat((u[:, :width].double() @ wd, u[:, width:].double()), dim=1)
    got = _fold(w, u).double()
    # fp32 sums of `width` products: error bound ~ width * 2^-24 * sum |u_w W_wd|
    bound = (u[:, :width].double().abs() @ wd.abs()) * (width * 2.0 ** -23) + 1e-30
    err = (got[:, :dim] - ref[:, :dim]).abs()
    assert bool((err <= bound).all()), f"max err {err.max().item()} vs bound {bound.max().item()}"
    assert torch.equal(got[:, dim], ref[:, dim])  # the bias passes through
    # backward: du_k = [W g_k[:dim], g_k[dim]]
    refb = torch.cat((gf[:, :dim].double() @ wd.t(), gf[:, dim:].double()), dim=1)
    for with_dw in (False, True):
        dw0 = (torch.randn(width, dim, generator=torch.Generator().manual_seed(width + dim)) * 0.3).to(dtype)
        gotb, dw = _unfold(w, gf, u if with_dw else None, dw0 if with_dw else None)
        gotb = gotb.double()
        boundb = (gf[:, :dim].double().abs() @ wd.abs().t()) * (dim * 2.0 ** -23) + 1e-30
        errb = (gotb[:, :width] - refb[:, :width]).abs()
        assert bool((errb <= boundb).all()), f"max err {errb.max().item()} vs bound {boundb.max().item()}"
        assert torch.equal(gotb[:, width], refb[:, width])
        if with_dw:
            # dW + u^T g: three fp32 roundings (a product, an fma, the add; 2^-24
            # of the sum's magnitude each), then one to the I/O type (bf16: 2^-9)
            refw = dw0.double() + u[:, :width].double().t() @ gf[:, :dim].double()
            mag = dw0.double().abs() + u[:, :width].double().abs().t() @ gf[:, :dim].double().abs()
            ulp = 2.0 ** -21 if dtype == torch.float32 else 2.0 ** -8
            errw = (dw.double() - refw).abs()
            assert bool((errw <= mag * ulp + 1e-30).all()), f"dW max err {errw.max().item()}"


def test_fold_deterministic():
    """The same bits on repeated calls (fixed-order sums, no atomics)."""
    print("[case] controls fold determinism", flush=True)
    w, u, gf = _case(24576, 768, torch.bfloat16, seed=3)
    a, b = _fold(w, u), _fold(w, u)
    assert torch.equal(a, b)
    assert torch.equal(_unfold(w, gf)[0], _unfold(w, gf)[0])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_projected_mixer_fold_matches_torch_products(dtype, monkeypatch):
    """The stack's projected mixer with the library fold and with torch's
    fp32 products in its place (the path wider models take): the same
    outputs and gradients up to fp32 summation order."""
    print(f"[case] projected mixer fold vs torch products {dtype}", flush=True)
    from sparc_amd import mixer as mx
    from sparc_amd.sparc import SPARCMixer

    torch.manual_seed(11)
    D, M, B, T = 64, 48, 2, 40
    mod = SPARCMixer(2 * M).cuda()
    with torch.no_grad():
        for p in (mod.phase_direction, mod.radial_direction):
            p.normal_(0.0, 0.3)
    w = (torch.randn(2 * M, D, device="cuda") / D ** 0.5).to(dtype).requires_grad_()
    xn = torch.randn(B, T, D, device="cuda").to(dtype).requires_grad_()
    dy = torch.randn(B, T, 2 * M, device="cuda").to(dtype)

    def run():
        for t in (w, xn, mod.phase_direction, mod.radial_direction):
            t.grad = None
        y, (lr, li) = mx.projected_sequence(mod, xn, w)
        (y.float() * dy.float()).sum().add_(lr.sum() + li.sum()).backward()
        return [y.detach().float().clone()] + [t.grad.detach().float().clone() for t in (
            w, xn, mod.phase_direction, mod.radial_direction)]

    a = run()
    monkeypatch.setattr(mx, "_FOLD_MAX_DIM", 0)
    b = run()
    tol = dict(rtol=1e-4, atol=1e-4) if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)
    for name, x, y in zip(("y", "dW", "dxn", "dphase", "dradial"), a, b):
        scale = y.abs().max().item() + 1e-6
        torch.testing.assert_close(x / scale, y / scale, **tol, msg=lambda m: f"{name}: {m}")


def test_projected_mixer_mixed_parameter_dtypes():
    """Module parameters of different dtypes (here the directions in bf16, the
    per-mode vectors in fp32) take the per-tensor casts: outputs and
    gradients match the all-fp32 run with the same (bf16-representable)
    values, and each gradient comes back in its parameter's dtype."""
    print("[case] projected mixer, mixed parameter dtypes", flush=True)
    from sparc_amd import mixer as mx
    from sparc_amd.sparc import SPARCMixer

    torch.manual_seed(12)
    D, M, B, T = 32, 24, 2, 48
    mod = SPARCMixer(2 * M).cuda()
    with torch.no_grad():
        for p in (mod.phase_direction, mod.radial_direction):
            p.copy_((torch.randn_like(p) * 0.3).to(torch.bfloat16).float())
    w = (torch.randn(2 * M, D, device="cuda") / D ** 0.5).requires_grad_()
    xn = torch.randn(B, T, D, device="cuda").requires_grad_()
    dy = torch.randn(B, T, 2 * M, device="cuda")

    def run():
        for t in [w, xn] + list(mod.parameters()):
            t.grad = None
        y, (lr, li) = mx.projected_sequence(mod, xn, w)
        (y * dy).sum().add_(lr.sum() + li.sum()).backward()
        return [y.detach().clone()] + [t.grad.detach().float().clone() for t in (
            w, xn, mod.phase_direction, mod.radial_direction, mod.nu_log, mod.write_log_gain)]

    a = run()
    with torch.no_grad():
        mod.phase_direction.data = mod.phase_direction.data.to(torch.bfloat16)
        mod.radial_direction.data = mod.radial_direction.data.to(torch.bfloat16)
    b = run()
    assert mod.phase_direction.grad.dtype == torch.bfloat16 and mod.nu_log.grad.dtype == torch.float32
    for name, x, y in zip(("y", "dW", "dxn", "dphase", "dradial", "dnu_log", "dwlg"), a, b):
        scale = x.abs().max().item() + 1e-6
        # the direction gradients are rounded to bf16 once; the rest is the same fp32 arithmetic
        tol = 2 ** -7 if name in ("dphase", "dradial") else 1e-5
        torch.testing.assert_close(y / scale, x / scale, rtol=tol, atol=tol, msg=lambda m: f"{name}: {m}")
