"""Pins the CPU oracle (oracle/sparc_oracle.py) by mathematics that a wrong
restatement would break: closed forms of the time-invariant case, independent
scan algorithms, adjoint identities, finite differences, and decode/sequence
agreement.  Golden vectors from the reference's own eager path are checked in
test_golden.py."""
import math

import pytest
import torch

from oracle import sparc_oracle as O



@pytest.fixture(autouse=True)
def _float64_default():
    """float64 by default inside this module only."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _rand_complex_inputs(B=2, T=37, M=5, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = 0.5 + 0.49 * torch.rand(B, T, M, generator=g)
    phi = (torch.rand(B, T, M, generator=g) * 2 - 1) * math.pi
    ar, ai = r * torch.cos(phi), r * torch.sin(phi)
    wr = torch.randn(B, T, M, generator=g)
    wi = torch.randn(B, T, M, generator=g)
    return ar, ai, wr, wi


def test_lti_geometric_series():
    """Constant a and w: h_t = w (1 - a^{t+1}) / (1 - a)."""
    B, T, M = 1, 50, 3
    a = torch.tensor([0.9 * complex(math.cos(0.3), math.sin(0.3)), 0.5 + 0.1j, -0.7j])
    w = torch.tensor([1.0 + 0.5j, -2.0 + 0.0j, 0.25 - 1.0j])
    ar = a.real.expand(B, T, M).clone()
    ai = a.imag.expand(B, T, M).clone()
    wr = w.real.expand(B, T, M).clone()
    wi = w.imag.expand(B, T, M).clone()
    (hr, hi), _ = O.complex_scan(ar, ai, wr, wi)
    t = torch.arange(T, dtype=torch.float64)[:, None]
    expect = w * (1 - a[None] ** (t + 1)) / (1 - a[None])
    assert torch.allclose(hr[0], expect.real, atol=1e-12)
    assert torch.allclose(hi[0], expect.imag, atol=1e-12)


def test_impulse_response_is_product_of_transitions():
    ar, ai, _, _ = _rand_complex_inputs(T=20)
    wr = torch.zeros_like(ar)
    wi = torch.zeros_like(ar)
    wr[:, 0] = 1.0
    (hr, hi), _ = O.complex_scan(ar, ai, wr, wi)
    a = torch.complex(ar, ai)
    prod = torch.cumprod(a[:, 1:], dim=1)
    assert torch.allclose(hr[:, 1:], prod.real, atol=1e-12)
    assert torch.allclose(hi[:, 1:], prod.imag, atol=1e-12)


@pytest.mark.parametrize("T", [1, 2, 3, 7, 16, 37, 64])
def test_associative_scans_match_sequential(T):
    ar, ai, wr, wi = _rand_complex_inputs(T=T)
    (hr, hi), _ = O.complex_scan(ar, ai, wr, wi)
    er, ei = O.associative_scan_oddeven(ar, ai, wr, wi)
    assert torch.allclose(er, hr, atol=1e-12) and torch.allclose(ei, hi, atol=1e-12)
    sr, si = O.hillis_steele_scan(ar, ai, wr, wi)
    assert torch.allclose(sr, hr, atol=1e-12) and torch.allclose(si, hi, atol=1e-12)


def test_real_equals_complex_with_zero_phase():
    g = torch.Generator().manual_seed(3)
    a = 0.9 + 0.09 * torch.rand(2, 40, 6, generator=g)
    b = torch.randn(2, 40, 6, generator=g)
    h, last = O.real_scan(a, b)
    (hr, hi), _ = O.complex_scan(a, torch.zeros_like(a), b, torch.zeros_like(b))
    assert torch.allclose(h, hr, atol=1e-14) and hi.abs().max() == 0
    assert torch.allclose(last, h[:, -1])


def test_explicit_adjoint_matches_autograd_with_resets_and_h0():
    ar, ai, wr, wi = _rand_complex_inputs(T=23, M=4, seed=5)
    B, T, M = wr.shape
    h0 = (torch.randn(B, M), torch.randn(B, M))
    seg = torch.ones(B, T, dtype=torch.int32)
    seg[0, 7] = 0
    seg[1, 0] = 0
    resets = O.reset_mask(B, T, seg)
    leaves = [t.clone().requires_grad_() for t in (ar, ai, wr, wi, h0[0], h0[1])]
    (hr, hi), last = O.complex_scan(*leaves[:4], h0=(leaves[4], leaves[5]), resets=resets)
    g = torch.Generator().manual_seed(9)
    dyr, dyi = torch.randn(B, T, M, generator=g), torch.randn(B, T, M, generator=g)
    dl = (torch.randn(B, M, generator=g), torch.randn(B, M, generator=g))
    loss = (hr * dyr).sum() + (hi * dyi).sum() + (last[0] * dl[0]).sum() + (last[1] * dl[1]).sum()
    auto = torch.autograd.grad(loss, leaves)
    dar, dai, dwr, dwi, dh0 = O.complex_scan_adjoint(ar, ai, hr.detach(), hi.detach(), dyr, dyi,
                                                     dlast=dl, h0=h0, resets=resets)
    for mine, ref in zip((dar, dai, dwr, dwi, dh0[0], dh0[1]), auto):
        assert torch.allclose(mine, ref, atol=1e-12)


def test_mixer_gradcheck_finite_differences():
    """The oracle's P1 layer is differentiable as restated: autograd gradients
    of every parameter and the input agree with central differences."""
    g = torch.Generator().manual_seed(1)
    p = O.init_params(6, generator=g)
    p.phase_direction = 0.3 * torch.randn(7, generator=g)
    p.radial_direction = 0.3 * torch.randn(7, generator=g)
    p.write_phase_response = torch.randn(3, generator=g)
    p.write_radial_response = torch.randn(3, generator=g)
    x = torch.randn(1, 5, 6, generator=g)
    names = ["nu_log", "theta_log", "phase_direction", "radial_direction", "write_log_gain",
             "write_phase_response", "write_radial_response"]

    def f(x_, *params):
        q = O.MixerParams(**dict(zip(names, params)))
        y, last = O.mixer_forward(q, x_, return_cache=True)
        return y.sum() + 0.3 * last[0].sum() - 0.2 * last[1].sum()

    inputs = [x.requires_grad_()] + [getattr(p, n).clone().requires_grad_() for n in names]
    assert torch.autograd.gradcheck(f, inputs, eps=1e-6, atol=1e-6, rtol=1e-5)


def test_write_dtype_rounds_write_value_and_gradient():
    """``mixer_forward(write_dtype=bf16)`` (the reference's cast of the write
    to x's dtype): the outputs equal the scan of the write rounded to bf16 by
    hand, and the parameter gradients equal the two-stage chain rule with the
    scan's gradient of the write rounded to bf16 before the write's backward."""
    g = torch.Generator().manual_seed(5)
    M, names = 6, ["nu_log", "theta_log", "phase_direction", "radial_direction", "write_log_gain",
                   "write_phase_response", "write_radial_response"]
    p = O.init_params(2 * M, generator=g)
    p.phase_direction = 0.3 * torch.randn(2 * M + 1, generator=g)
    p.radial_direction = 0.3 * torch.randn(2 * M + 1, generator=g)
    p.write_phase_response = torch.randn(M, generator=g)
    p.write_radial_response = torch.randn(M, generator=g)
    x = torch.randn(2, 9, 2 * M, generator=g)
    dy = torch.randn(2, 9, 2 * M, generator=g)
    params = [getattr(p, n).clone().requires_grad_() for n in names]
    q = O.MixerParams(**dict(zip(names, params)))
    y, _ = O.mixer_forward(q, x, write_dtype=torch.bfloat16)
    got = torch.autograd.grad((y * dy).sum(), params)
    # by hand: the write, its bf16 rounding as a fresh leaf, the scan
    eta, delta = O.controls(x, q.phase_direction, q.radial_direction)
    wr, wi = O.write(x, eta, delta, q.nu_log, q.write_log_gain, q.write_phase_response,
                     q.write_radial_response)
    lr = wr.detach().to(torch.bfloat16).double().requires_grad_()
    li = wi.detach().to(torch.bfloat16).double().requires_grad_()
    ar, ai = O.p1_transition(eta[..., None], delta[..., None], q.nu_log, q.theta_log)
    (hr, hi), _ = O.complex_scan(ar, ai, lr, li)
    y2 = torch.cat((hr, hi), -1).relu()
    assert torch.equal(y.detach(), y2.detach())
    loss = (y2 * dy).sum()
    gw = torch.autograd.grad(loss, [lr, li], retain_graph=True)
    direct = torch.autograd.grad(loss, params, allow_unused=True, retain_graph=True)  # transition, controls
    via_write = torch.autograd.grad([wr, wi], params, [gw[0].to(torch.bfloat16).double(),
                                                       gw[1].to(torch.bfloat16).double()], allow_unused=True)
    for n, a, b, c in zip(names, got, direct, via_write):
        ref = (b if b is not None else 0.0) + (c if c is not None else 0.0)
        assert torch.allclose(a, ref, rtol=1e-12, atol=1e-12), n
    # and the rounding changes the gradient (the model is not a no-op)
    y0, _ = O.mixer_forward(q, x)
    exact = torch.autograd.grad((y0 * dy).sum(), params)
    assert (got[4] - exact[4]).abs().max() > 1e-6


def test_controls_and_write_formulas_at_default_init():
    """Zero directions and responses (the module's init): eta = delta = 0,
    a_m = exp(-nu_m + i theta_m) and w = exp(wlg) tanh(x) exactly (ratio = 1,
    gate = 1): the LTI system of sparc-kernal/sparc.py:59-88."""
    g = torch.Generator().manual_seed(2)
    p = O.init_params(8, generator=g)
    x = torch.randn(2, 4, 8, generator=g)
    eta, delta = O.controls(x, p.phase_direction, p.radial_direction)
    assert eta.abs().max() == 0 and delta.abs().max() == 0
    wr, wi = O.write(x, eta, delta, p.nu_log, p.write_log_gain, p.write_phase_response,
                     p.write_radial_response)
    gamma = torch.exp(p.write_log_gain)
    assert torch.allclose(wr, gamma * torch.tanh(x[..., :4]), atol=1e-14)
    assert torch.allclose(wi, gamma * torch.tanh(x[..., 4:]), atol=1e-14)
    ar, ai = O.p1_transition(eta[..., None], delta[..., None], p.nu_log, p.theta_log)
    nu, th = torch.exp(p.nu_log), torch.exp(p.theta_log)
    assert torch.allclose(ar, torch.exp(-nu) * torch.cos(th), atol=1e-14)
    assert torch.allclose(ai, torch.exp(-nu) * torch.sin(th), atol=1e-14)
    # init: gain = sqrt(1 - e^{-2 nu}) + 1e-8 and |a| = sqrt(U)
    assert torch.allclose(gamma, torch.sqrt(1 - torch.exp(-2 * nu)) + 1e-8, rtol=1e-6)


def test_controls_select_phase_and_radial_rows():
    """delta follows the phase direction, eta the radial one."""
    p = O.init_params(4)
    p.phase_direction = torch.tensor([1.0, 0, 0, 0, 0.0])
    p.radial_direction = torch.tensor([0, 0, 0, 0, 0.5])
    x = torch.tensor([[[0.7, 0, 0, 0]]])
    eta, delta = O.controls(x, p.phase_direction, p.radial_direction)
    assert torch.allclose(delta, torch.tensor([[O.HALF_PI * math.tanh(0.7)]]))
    assert torch.allclose(eta, torch.tensor([[O.LOG16 * math.tanh(0.5)]]))


def test_decode_steps_match_sequence_forward():
    g = torch.Generator().manual_seed(4)
    p = O.init_params(10, generator=g)
    p.phase_direction = 0.2 * torch.randn(11, generator=g)
    p.radial_direction = 0.2 * torch.randn(11, generator=g)
    p.write_phase_response = torch.randn(5, generator=g)
    x = torch.randn(3, 9, 10, generator=g)
    y_seq, last = O.mixer_forward(p, x[:, :4], return_cache=True)
    state = last
    ys = []
    for t in range(4, 9):
        y, state = O.decode_step(p, x[:, t], state)
        ys.append(y)
    y_full, last_full = O.mixer_forward(p, x, return_cache=True)
    assert torch.allclose(torch.stack(ys, 1), y_full[:, 4:], atol=1e-12)
    assert torch.allclose(state[0], last_full[0], atol=1e-12)
    assert torch.allclose(y_seq, y_full[:, :4], atol=1e-14)


def test_grouped_gates_expand_per_mode():
    g = torch.Generator().manual_seed(6)
    r = torch.rand(2, 5, 3, generator=g)
    phi = torch.rand(2, 5, 3, generator=g)
    ar, ai = O.polar_transition(r, phi, 12)
    assert ar.shape == (2, 5, 12)
    for m in range(12):
        assert torch.equal(ar[..., m], r[..., m // 4] * torch.cos(phi[..., m // 4]))
