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


def test_decode_step_write_dtype_rounds_only_the_write():
    """decode_step(write_dtype=bf16) is the sequence forward with the same
    write rounding, step by step; the write is the only rounded quantity (the
    new state differs from the unrounded one by exactly the rounding of w)."""
    g = torch.Generator().manual_seed(63)
    p = O.init_params(12, generator=g)
    p.phase_direction = 0.3 * torch.randn(13, generator=g)
    p.radial_direction = 0.3 * torch.randn(13, generator=g)
    x = torch.randn(2, 5, 12, generator=g, dtype=torch.float64)
    _, last = O.mixer_forward(p, x[:, :3], return_cache=True, write_dtype=torch.bfloat16)
    state = last
    for t in range(3, 5):
        y, state = O.decode_step(p, x[:, t], state, write_dtype=torch.bfloat16)
    y_full, last_full = O.mixer_forward(p, x, return_cache=True, write_dtype=torch.bfloat16)
    assert torch.allclose(y, y_full[:, 4], atol=1e-12) and torch.allclose(state[0], last_full[0], atol=1e-12)
    s0 = (torch.randn(2, 6, generator=g, dtype=torch.float64), torch.randn(2, 6, generator=g, dtype=torch.float64))
    _, (rr, ri) = O.decode_step(p, x[:, 0], s0, write_dtype=torch.bfloat16)
    _, (er, ei) = O.decode_step(p, x[:, 0], s0)
    eta, delta = O.controls(x[:, :1], p.phase_direction, p.radial_direction)
    wr, wi = O.write(x[:, :1], eta, delta, p.nu_log, p.write_log_gain, p.write_phase_response,
                     p.write_radial_response)
    assert torch.allclose(rr - er, wr[:, 0].bfloat16().double() - wr[:, 0], atol=1e-14)
    assert torch.allclose(ri - ei, wi[:, 0].bfloat16().double() - wi[:, 0], atol=1e-14)
    assert (rr - er).abs().max() > 0


def test_grouped_gates_expand_per_mode():
    g = torch.Generator().manual_seed(6)
    r = torch.rand(2, 5, 3, generator=g)
    phi = torch.rand(2, 5, 3, generator=g)
    ar, ai = O.polar_transition(r, phi, 12)
    assert ar.shape == (2, 5, 12)
    for m in range(12):
        assert torch.equal(ar[..., m], r[..., m // 4] * torch.cos(phi[..., m // 4]))


def test_polar_transition_is_r_exp_i_phi():
    """polar_transition(r, phi) = r e^{+i phi} in both parts: torch.polar, the
    quarter turns (phi = +-pi/2 puts r on the +-imaginary axis), and
    r e^{i phi} e^{-i phi} = r.  A conjugate-sign or swapped-part slip fails."""
    g = torch.Generator().manual_seed(61)
    r = torch.rand(2, 7, 5, generator=g, dtype=torch.float64) * 0.9 + 0.05
    phi = (torch.rand(2, 7, 5, generator=g, dtype=torch.float64) * 2 - 1) * math.pi
    ar, ai = O.polar_transition(r, phi, 5)
    ref = torch.polar(r, phi)
    assert torch.allclose(ar, ref.real, atol=1e-15) and torch.allclose(ai, ref.imag, atol=1e-15)
    quarter = torch.tensor([[[math.pi / 2, -math.pi / 2, 0.0, math.pi]]], dtype=torch.float64)
    rr = torch.full_like(quarter, 0.5)
    qr, qi = O.polar_transition(rr, quarter, 4)
    assert torch.allclose(qr, torch.tensor([[[0.0, 0.0, 0.5, -0.5]]], dtype=torch.float64), atol=1e-15)
    assert torch.allclose(qi, torch.tensor([[[0.5, -0.5, 0.0, 0.0]]], dtype=torch.float64), atol=1e-15)
    back = torch.complex(ar, ai) * torch.exp(-1j * phi)
    assert torch.allclose(back.real, r, atol=1e-15) and back.imag.abs().max() < 1e-15


def test_polar_transition_matches_p1_at_equal_radius_and_phase():
    """At eta = 0 the P1 radius is exp(-nu) and its phase theta + (1 - rho)
    delta: with nu = -log r and the phase phi = theta + (1 - r) delta, the
    P1 transition is the polar one of (r, phi), part for part."""
    g = torch.Generator().manual_seed(62)
    M, B, T = 6, 2, 9
    r = torch.rand(M, generator=g, dtype=torch.float64) * 0.5 + 0.45
    theta = torch.rand(M, generator=g, dtype=torch.float64) * 5.0 + 0.2
    delta = (torch.rand(B, T, 1, generator=g, dtype=torch.float64) * 2 - 1) * (math.pi / 2)
    eta = torch.zeros(B, T, 1, dtype=torch.float64)
    pr, pi = O.p1_transition(eta, delta, torch.log(-torch.log(r)), torch.log(theta))
    phi = theta + (1.0 - r) * delta                       # [B, T, M]
    ar, ai = O.polar_transition(r.expand(B, T, M), phi, M)
    assert torch.allclose(pr, ar, atol=1e-14) and torch.allclose(pi, ai, atol=1e-14)
    assert (ai * torch.sin(phi) >= 0).all()               # the imaginary part follows +sin(phi)


# --------------------------------------------------------------------------
# reset, initial-state and init semantics, pinned by properties a misread
# mask or state hand-off breaks (inverted, shifted or ignored resets; h0
# applied twice or not at all; segment_pos and reset_first in the wrong order)
# --------------------------------------------------------------------------
def _real_inputs(B=2, T=31, W=5, seed=11):
    g = torch.Generator().manual_seed(seed)
    return 0.5 + 0.49 * torch.rand(B, T, W, generator=g), torch.randn(B, T, W, generator=g)


@pytest.mark.parametrize("k", [1, 9, 36])
def test_split_invariance_complex_scan(k):
    """Scanning [0, T) equals scanning [0, k) and then [k, T) from the state
    at k - 1 (the h0 hand-off of sparc-kernal/forward/scan.py:821-826)."""
    ar, ai, wr, wi = _rand_complex_inputs(T=37, seed=21)
    (hr, hi), last = O.complex_scan(ar, ai, wr, wi)
    (pr, pi), plast = O.complex_scan(ar[:, :k], ai[:, :k], wr[:, :k], wi[:, :k])
    (sr, si), slast = O.complex_scan(ar[:, k:], ai[:, k:], wr[:, k:], wi[:, k:], h0=plast)
    assert torch.allclose(torch.cat((pr, sr), 1), hr, atol=1e-12)
    assert torch.allclose(torch.cat((pi, si), 1), hi, atol=1e-12)
    assert torch.allclose(slast[0], last[0], atol=1e-12) and torch.allclose(slast[1], last[1], atol=1e-12)


@pytest.mark.parametrize("k", [1, 13, 30])
def test_split_invariance_real_scan(k):
    a, b = _real_inputs()
    h, last = O.real_scan(a, b)
    hp, lp = O.real_scan(a[:, :k], b[:, :k])
    hs, ls = O.real_scan(a[:, k:], b[:, k:], h0=lp)
    assert torch.allclose(torch.cat((hp, hs), 1), h, atol=1e-12)
    assert torch.allclose(ls, last, atol=1e-12)


@pytest.mark.parametrize("transition", ["p1", "polar", "cartesian", "real"])
def test_split_invariance_grouped_scan(transition):
    B, T, M, G, k = 2, 29, 8, 4, 12
    g = torch.Generator().manual_seed(31)
    if transition == "p1":
        g0, g1 = 0.5 * torch.randn(B, T, G, generator=g), torch.randn(B, T, G, generator=g)
    elif transition == "polar":
        g0, g1 = 0.6 + 0.39 * torch.rand(B, T, G, generator=g), torch.randn(B, T, G, generator=g)
    else:
        g0, g1 = 0.6 * torch.rand(B, T, G, generator=g), 0.6 * torch.rand(B, T, G, generator=g)
    wr, wi = torch.randn(B, T, M, generator=g), torch.randn(B, T, M, generator=g)
    nu_log, theta_log = torch.randn(M, generator=g) - 2, torch.randn(M, generator=g)
    kw = dict(nu_log=nu_log, theta_log=theta_log)
    full, last = O.grouped_scan_forward(transition, g0, g1, wr, wi, **kw)
    pre, plast = O.grouped_scan_forward(transition, g0[:, :k], g1[:, :k], wr[:, :k], wi[:, :k], **kw)
    suf, slast = O.grouped_scan_forward(transition, g0[:, k:], g1[:, k:], wr[:, k:], wi[:, k:],
                                        h0=plast, **kw)
    if transition == "real":
        assert torch.allclose(torch.cat((pre, suf), 1), full, atol=1e-12)
        assert torch.allclose(slast, last, atol=1e-12)
    else:
        for p_, s_, f_ in zip(pre, suf, full):
            assert torch.allclose(torch.cat((p_, s_), 1), f_, atol=1e-12)
        assert torch.allclose(slast[0], last[0], atol=1e-12)


def test_segment_reset_equals_fresh_suffix_scan():
    """``segment_pos[b, t] == 0`` zeroes the transition at t
    (sparc-kernal/forward/scan.py:838-845): from t on, the outputs are a scan
    of the suffix from a zero state, and before t nothing changes.  A mask
    that is inverted, shifted by one step or ignored fails this."""
    ar, ai, wr, wi = _rand_complex_inputs(B=3, T=26, M=4, seed=41)
    B, T, M = wr.shape
    h0 = (torch.randn(B, M), torch.randn(B, M))
    seg = torch.arange(T).repeat(B, 1) + 5          # no segment starts ...
    seg[0, 10:] = torch.arange(T - 10)              # row 0: a segment starts at 10
    seg[2, 3:] = torch.arange(T - 3)                # row 2: at 3
    seg[2, 17:] = torch.arange(T - 17)              # ... and again at 17
    resets = O.reset_mask(B, T, seg)
    assert resets.sum() == 3 and resets[0, 10] and resets[2, 3] and resets[2, 17]
    (hr, hi), last = O.complex_scan(ar, ai, wr, wi, h0=h0, resets=resets)
    (nr, ni), _ = O.complex_scan(ar, ai, wr, wi, h0=h0)
    starts = {0: [10], 1: [], 2: [3, 17]}
    for b, ks in starts.items():
        bounds = [0] + ks + [T]
        for j, (s, e) in enumerate(zip(bounds[:-1], bounds[1:])):
            sl = slice(b, b + 1)
            if j == 0:   # before the first reset: the reset-free scan from h0
                assert torch.allclose(hr[b, s:e], nr[b, s:e], atol=1e-12)
                continue
            (fr, fi), _ = O.complex_scan(ar[sl, s:e], ai[sl, s:e], wr[sl, s:e], wi[sl, s:e])
            assert torch.allclose(hr[b, s:e], fr[0], atol=1e-12)
            assert torch.allclose(hi[b, s:e], fi[0], atol=1e-12)
    # row 1 has no reset: identical to the reset-free scan
    assert torch.equal(hr[1], nr[1])
    # the real scan and the module follow the same rule
    a, bb = _real_inputs(B=1, T=20, W=3)
    segr = torch.arange(20)[None] + 1
    segr[0, 8:] = torch.arange(12)
    h, _ = O.real_scan(a, bb, h0=torch.randn(1, 3), resets=O.reset_mask(1, 20, segr))
    fresh, _ = O.real_scan(a[:, 8:], bb[:, 8:])
    assert torch.allclose(h[:, 8:], fresh, atol=1e-12)


def test_module_segment_reset_equals_fresh_suffix_forward():
    """At module level (``mixer_forward(segment_pos=...)``) a segment start
    at k makes the outputs from k those of the module run on x[:, k:] alone."""
    g = torch.Generator().manual_seed(43)
    p = O.init_params(8, generator=g)
    p.phase_direction = 0.3 * torch.randn(9, generator=g)
    p.radial_direction = 0.3 * torch.randn(9, generator=g)
    x = torch.randn(1, 15, 8, generator=g)
    seg = torch.arange(15)[None] + 2
    seg[0, 6:] = torch.arange(9)
    h0 = (torch.randn(1, 4, generator=g), torch.randn(1, 4, generator=g))
    y, _ = O.mixer_forward(p, x, initial_state=h0, segment_pos=seg)
    y_suffix, _ = O.mixer_forward(p, x[:, 6:])
    y_prefix, _ = O.mixer_forward(p, x[:, :6], initial_state=h0)
    assert torch.allclose(y[:, 6:], y_suffix, atol=1e-12)
    assert torch.allclose(y[:, :6], y_prefix, atol=1e-12)


def test_reset_first_discards_h0():
    """``reset_first`` zeroes the first transition: with it, any h0 gives the
    zero-state scan (forward/scan.py:840-841)."""
    ar, ai, wr, wi = _rand_complex_inputs(T=12, seed=45)
    B, T, M = wr.shape
    h0 = (torch.randn(B, M), torch.randn(B, M))
    zero, _ = O.grouped_scan_forward("cartesian", ar, ai, wr, wi)
    with_h0, _ = O.grouped_scan_forward("cartesian", ar, ai, wr, wi, h0=h0, reset_first=True)
    without, _ = O.grouped_scan_forward("cartesian", ar, ai, wr, wi, h0=h0)
    assert torch.allclose(with_h0[0], zero[0], atol=1e-14) and torch.allclose(with_h0[1], zero[1], atol=1e-14)
    assert (without[0] - zero[0]).abs().max() > 1e-3      # h0 matters without the reset
    a, b = _real_inputs(T=9)
    hz, _ = O.grouped_scan_forward("real", a, None, b, None)
    hr, _ = O.grouped_scan_forward("real", a, None, b, None, h0=torch.randn(2, 5), reset_first=True)
    assert torch.allclose(hr, hz, atol=1e-14)


def test_segment_pos_wins_over_reset_first():
    """With ``segment_pos`` given, ``reset_first`` is ignored: the reference
    tests ``HAS_SEGMENTS`` before ``RESET_FIRST`` (forward/scan.py:838-843),
    so a row whose t = 0 is not a segment start keeps its h0."""
    ar, ai, wr, wi = _rand_complex_inputs(T=10, seed=47)
    B, T, M = wr.shape
    h0 = (torch.randn(B, M), torch.randn(B, M))
    seg = torch.arange(T).repeat(B, 1) + 3     # no zeros: no segment starts
    seg[1, 0] = 0                               # row 1 starts a segment at t = 0
    mask = O.reset_mask(B, T, seg, reset_first=True)
    assert not mask[0].any() and mask[1, 0] and mask[1].sum() == 1
    out, _ = O.grouped_scan_forward("cartesian", ar, ai, wr, wi, h0=h0, segment_pos=seg,
                                    reset_first=True)
    keep, _ = O.grouped_scan_forward("cartesian", ar, ai, wr, wi, h0=h0)
    zero, _ = O.grouped_scan_forward("cartesian", ar, ai, wr, wi)
    assert torch.allclose(out[0][0], keep[0][0], atol=1e-14)   # row 0 keeps h0
    assert torch.allclose(out[0][1], zero[0][1], atol=1e-14)   # row 1 was reset
    assert O.reset_mask(B, T, None, reset_first=True)[:, 0].all()


def test_adjoint_with_reset_splits_at_the_reset():
    """No gradient crosses a reset: the explicit adjoint of a scan reset at k
    equals, on [0, k), the adjoint of the prefix alone (no dlast) and, on
    [k, T), the adjoint of the suffix from a zero state; dh0 is the prefix's."""
    ar, ai, wr, wi = _rand_complex_inputs(B=1, T=19, M=3, seed=49)
    B, T, M = wr.shape
    k = 7
    h0 = (torch.randn(B, M), torch.randn(B, M))
    seg = torch.arange(T)[None] + 1
    seg[0, k:] = torch.arange(T - k)
    resets = O.reset_mask(B, T, seg)
    (hr, hi), _ = O.complex_scan(ar, ai, wr, wi, h0=h0, resets=resets)
    g = torch.Generator().manual_seed(50)
    dyr, dyi = torch.randn(B, T, M, generator=g), torch.randn(B, T, M, generator=g)
    dl = (torch.randn(B, M, generator=g), torch.randn(B, M, generator=g))
    full = O.complex_scan_adjoint(ar, ai, hr, hi, dyr, dyi, dlast=dl, h0=h0, resets=resets)
    pre = O.complex_scan_adjoint(ar[:, :k], ai[:, :k], hr[:, :k], hi[:, :k], dyr[:, :k],
                                 dyi[:, :k], h0=h0)
    suf = O.complex_scan_adjoint(ar[:, k:], ai[:, k:], hr[:, k:], hi[:, k:], dyr[:, k:],
                                 dyi[:, k:], dlast=dl)
    for j in range(4):
        assert torch.allclose(full[j][:, :k], pre[j], atol=1e-12)
        assert torch.allclose(full[j][:, k:], suf[j], atol=1e-12)
    assert torch.allclose(full[4][0], pre[4][0], atol=1e-12)
    assert full[0][:, k].abs().max() == 0 and full[1][:, k].abs().max() == 0


def test_init_matches_reference_golden_under_seed_0():
    """``torch.manual_seed(0); SPARCMixer(16)``: the golden fixture holds the
    reference module's nu_log and theta_log made exactly so
    (tests/golden/make_golden.py, sparc-kernal/sparc.py:65-73).  The oracle's
    init reproduces them bit for bit, and so does the product module."""
    import numpy as np
    import os
    import sparc_amd
    path = os.path.join(os.path.dirname(__file__), "golden", "p1_eager_golden.npz")
    with np.load(path, allow_pickle=False) as z:
        nu_ref, theta_ref = torch.from_numpy(z["nu_log"]), torch.from_numpy(z["theta_log"])
    torch.manual_seed(0)
    p = O.init_params(16)
    assert torch.equal(p.nu_log, nu_ref) and torch.equal(p.theta_log, theta_ref)
    torch.set_default_dtype(torch.float32)      # the reference module was built so
    torch.manual_seed(0)
    m = sparc_amd.SPARCMixer(16)
    assert m.nu_log.dtype == torch.float32
    assert torch.equal(m.nu_log.detach().double(), nu_ref)
    assert torch.equal(m.theta_log.detach().double(), theta_ref)
    assert torch.equal(m.write_log_gain.detach().double(), p.write_log_gain)
    # the spectrum's documented ranges: |a| = sqrt(U) in (0, 1), theta in (0, 2 pi)
    radius = torch.exp(-torch.exp(nu_ref))
    assert (radius > 0).all() and (radius < 1).all()
    theta = torch.exp(theta_ref)
    assert (theta > 0).all() and (theta < 2 * math.pi).all()


def test_init_gain_normalises_stationary_energy():
    """The initial write gain is the energy normaliser of the LTI system at
    init: a unit-variance i.i.d. write scaled by gamma has stationary state
    variance gamma^2 / (1 - |a|^2) = 1 (up to the 1e-8 guard), checked by
    summing the impulse response's energy, not by the gain formula."""
    torch.manual_seed(3)
    p = O.init_params(12)
    gamma = torch.exp(p.write_log_gain)
    a = torch.exp(-torch.exp(p.nu_log))            # |a| at eta = 0
    t = torch.arange(20000, dtype=torch.float64)[:, None]
    energy = (gamma[None] * a[None] ** t).square().sum(0)
    slow = a < 0.999                                 # series converged within 20000 terms
    assert torch.allclose(energy[slow], torch.ones_like(energy[slow]), atol=1e-6)
