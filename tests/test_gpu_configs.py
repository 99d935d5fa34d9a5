"""GPU parity at the shapes of the five benchmark configurations.

cfg1 runs whole against the float64 oracle.  cfg2-cfg4 run the HIP kernels at
their full size; every (batch row, mode) chain of the scan is independent, so
the float64 oracle then recomputes whole gate groups (all modes that share a
gate, so the gate gradients are complete sums) at the first, a middle and the
last group position, over every time step, and the HIP results of those
groups must match.  cfg3 also checks the drift of the last step (T-1) after
65536 steps of |a| up to 0.9999.

Tolerances (max |gpu - oracle| / max |oracle| per tensor): 1e-4 for fp32 I/O,
2e-2 for bf16 I/O with the fp32 state.
"""
import math

import pytest
import torch

import sparc_amd
from oracle import sparc_oracle as O
from sparc_amd import ops

pytestmark = pytest.mark.gpu


def rel_err(got, ref):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    return (got - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)


def group_modes(groups, gs):
    return torch.cat([torch.arange(g * gs, (g + 1) * gs) for g in groups])


# ---------------------------------------------------------------------------
# cfg1: one SPARC layer, B=2, T=256, d_model=64, N=16 (M=1024, width 2048), fp32
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("path", ["fused", "composed"])
@pytest.mark.parametrize("controller", [False, True], ids=["lti", "controller_on"])
def test_cfg1_layer_fwd_bwd(controller, path):
    """|a| = exp(-nu) in [0.9, 0.999] (nu = -log r, r ~ U[0.9, 0.999]), theta
    = 2 pi U (the module's init, == U(-pi, pi) mod 2 pi); eta = delta = 0 with
    the default zero directions, or random directions (controller on)."""
    print(f"[case] cfg1 controller={controller} path={path}", flush=True)
    sparc_amd.set_mixer_path(path)
    B, T, D, N = 2, 256, 64, 16
    M = D * N
    width = 2 * M
    torch.manual_seed(0)
    m = sparc_amd.SPARCMixer(width)
    g = torch.Generator().manual_seed(0)
    with torch.no_grad():
        r = 0.9 + 0.099 * torch.rand(M, generator=g, dtype=torch.float64)
        m.nu_log.copy_(torch.log(-torch.log(r)).float())
        if controller:
            m.phase_direction.copy_(torch.randn(width + 1, generator=g) / math.sqrt(width))
            m.radial_direction.copy_(torch.randn(width + 1, generator=g) / math.sqrt(width))
            m.write_phase_response.copy_(torch.randn(M, generator=g))
            m.write_radial_response.copy_(torch.randn(M, generator=g))
    names = ["nu_log", "theta_log", "phase_direction", "radial_direction", "write_log_gain",
             "write_phase_response", "write_radial_response"]
    p = O.MixerParams(**{n: getattr(m, n).detach().double().clone().requires_grad_() for n in names})
    x_cpu = torch.randn(B, T, width, generator=g)
    # output gradients only where the state is clearly away from 0 (the relu
    # mask is ambiguous within the fp32 rounding of 0)
    dy = torch.randn(B, T, width, generator=g, dtype=torch.float64)
    with torch.no_grad():
        eta, delta = O.controls(x_cpu.double(), p.phase_direction, p.radial_direction)
        wr, wi = O.write(x_cpu.double(), eta, delta, p.nu_log, p.write_log_gain,
                         p.write_phase_response, p.write_radial_response)
        ar, ai = O.p1_transition(eta[..., None], delta[..., None], p.nu_log, p.theta_log)
        (hr, hi), _ = O.complex_scan(ar, ai, wr, wi)
        h = torch.cat((hr, hi), -1)
        dy = dy * (h.abs() > 1e-3 * h.abs().max())
    mc = m.cuda()
    x = x_cpu.cuda().requires_grad_()
    y, cache = mc(x, return_cache=True)
    loss = (y * dy.cuda().float()).sum() + cache[0].sum() + cache[1].sum()
    grads = torch.autograd.grad(loss, [x] + [getattr(mc, n) for n in names])
    xo = x_cpu.double().requires_grad_()
    yo, lasto = O.mixer_forward(p, xo, return_cache=True)
    lo = (yo * dy).sum() + lasto[0].sum() + lasto[1].sum()
    grads_o = torch.autograd.grad(lo, [xo] + [getattr(p, n) for n in names])
    sparc_amd.set_mixer_path("auto")
    assert rel_err(y, yo) <= 1e-4
    assert rel_err(cache[0], lasto[0]) <= 1e-4 and rel_err(cache[1], lasto[1]) <= 1e-4
    for n, a, b in zip(["x"] + names, grads, grads_o):
        if not controller and n in ("phase_direction", "radial_direction", "write_phase_response",
                                    "write_radial_response") and b.abs().max() == 0:
            assert a.abs().max().item() == 0, n
            continue
        assert rel_err(a, b) <= 1e-4, f"grad {n}: {rel_err(a, b):.3g}"


# ---------------------------------------------------------------------------
# cfg2: complex chunked scan, B=8, T=4096, D=1024, N=16, bf16 I/O, fp32 state
# ---------------------------------------------------------------------------
def test_cfg2_full_size_sampled_groups():
    print("[case] cfg2 full size B=8 T=4096 M=16384 G=1024 bf16 polar", flush=True)
    B, T, D, N = 8, 4096, 1024, 16
    M, G = D * N, D
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    r = torch.sigmoid(torch.randn(B, T, G, device=dev, generator=g) + 2.0).to(torch.bfloat16)
    phi = ((torch.rand(B, T, G, device=dev, generator=g) * 2 - 1) * math.pi).to(torch.bfloat16)
    w_re = torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
    w_im = torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
    dy_re = torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
    dy_im = torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
    y_re, y_im, cs = ops.scan_forward_raw("polar", r, phi, w_re, w_im)
    gr = ops.scan_backward_raw("polar", r, phi, w_re, w_im, cs, dy_re, dy_im, y_re=y_re, y_im=y_im)
    torch.cuda.synchronize()
    rows, groups = [0, 5, 7], [0, 517, 1023]
    modes = group_modes(groups, N).to(dev)
    rr = torch.tensor(rows, device=dev)

    def pick(t, idx):
        return t[rr][:, :, idx].double().cpu()

    gsel = torch.tensor(groups, device=dev)
    leaves = [pick(r, gsel), pick(phi, gsel), pick(w_re, modes), pick(w_im, modes)]
    leaves = [v.clone().requires_grad_() for v in leaves]
    (hr, hi), last = O.grouped_scan_forward("polar", *leaves)
    loss = (hr * pick(dy_re, modes)).sum() + (hi * pick(dy_im, modes)).sum()
    d_r, d_phi, d_wr, d_wi = torch.autograd.grad(loss, leaves)
    tol = 2e-2
    assert rel_err(pick(y_re, modes), hr) <= tol
    assert rel_err(pick(y_im, modes), hi) <= tol
    assert rel_err(cs[rr][:, -1][:, modes, 0], last[0]) <= 1e-4  # fp32 state after T steps
    assert rel_err(pick(gr["dw_re"], modes), d_wr) <= tol
    assert rel_err(pick(gr["dw_im"], modes), d_wi) <= tol
    assert rel_err(pick(gr["dg0"], gsel), d_r) <= tol
    assert rel_err(pick(gr["dg1"], gsel), d_phi) <= tol


def test_few_chains_time_segments_full_size():
    """B=1, T=32768, D=128, N=16 polar bf16: 8 chains of 256 modes, which the
    serial kernels split into 128 time segments (two groups of 64 in the
    carry).  Outputs, final state and gradients against the look-back
    kernels everywhere, and against the float64 oracle on three whole gate
    groups over every step."""
    print("[case] few chains B=1 T=32768 M=2048 G=128 bf16 polar, segments vs look-back", flush=True)
    B, T, D, N = 1, 32768, 128, 16
    M, G = D * N, D
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(7)
    r = torch.sigmoid(torch.randn(B, T, G, device=dev, generator=g) + 2.0).to(torch.bfloat16)
    phi = ((torch.rand(B, T, G, device=dev, generator=g) * 2 - 1) * math.pi).to(torch.bfloat16)
    w_re, w_im, dy_re, dy_im = (torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
                                for _ in range(4))
    h0_re, h0_im, dl_re, dl_im = (torch.randn(B, M, device=dev, generator=g) for _ in range(4))

    def run(algorithm):
        ops.set_algorithm(algorithm)
        try:
            y_re, y_im, cs = ops.scan_forward_raw("polar", r, phi, w_re, w_im, h0_re=h0_re, h0_im=h0_im)
            gr = ops.scan_backward_raw("polar", r, phi, w_re, w_im, cs, dy_re, dy_im, h0_re=h0_re, h0_im=h0_im,
                                       dlast_re=dl_re, dlast_im=dl_im, want_dh0=True, y_re=y_re, y_im=y_im)
            torch.cuda.synchronize()
            return y_re, y_im, cs, gr
        finally:
            ops.set_algorithm("auto")

    y_re, y_im, cs, gr = run("auto")
    ly_re, ly_im, lcs, lgr = run("lookback")
    tol = 2e-2
    assert rel_err(y_re, ly_re) <= tol and rel_err(y_im, ly_im) <= tol
    assert rel_err(cs[:, -1], lcs[:, -1]) <= 1e-4
    for k in ("dw_re", "dw_im", "dg0", "dg1", "dh0_re", "dh0_im"):
        assert rel_err(gr[k], lgr[k]) <= tol, k
    del ly_re, ly_im, lcs, lgr
    groups = [0, 77, G - 1]
    modes = group_modes(groups, N).to(dev)
    gsel = torch.tensor(groups, device=dev)

    def pick(t, idx):
        return t[:, :, idx].double().cpu()

    leaves = [pick(r, gsel), pick(phi, gsel), pick(w_re, modes), pick(w_im, modes),
              h0_re[:, modes].double().cpu(), h0_im[:, modes].double().cpu()]
    leaves = [v.clone().requires_grad_() for v in leaves]
    (hr, hi), last = O.grouped_scan_forward("polar", *leaves[:4], h0=(leaves[4], leaves[5]))
    loss = (hr * pick(dy_re, modes)).sum() + (hi * pick(dy_im, modes)).sum() \
        + (last[0] * dl_re[:, modes].double().cpu()).sum() + (last[1] * dl_im[:, modes].double().cpu()).sum()
    d_r, d_phi, d_wr, d_wi, d_h0r, d_h0i = torch.autograd.grad(loss, leaves)
    assert rel_err(pick(y_re, modes), hr) <= tol
    assert rel_err(pick(y_im, modes), hi) <= tol
    assert rel_err(cs[:, -1][:, modes, 0], last[0]) <= 1e-4
    assert rel_err(cs[:, -1][:, modes, 1], last[1]) <= 1e-4
    assert rel_err(pick(gr["dw_re"], modes), d_wr) <= tol
    assert rel_err(pick(gr["dw_im"], modes), d_wi) <= tol
    assert rel_err(pick(gr["dg0"], gsel), d_r) <= tol
    assert rel_err(pick(gr["dg1"], gsel), d_phi) <= tol
    assert rel_err(gr["dh0_re"][:, modes], d_h0r) <= tol
    assert rel_err(gr["dh0_im"][:, modes], d_h0i) <= tol


def test_cfg2_shape_p1_operator_full_size():
    """The reference's own operator (P1, one (eta, delta) per token) at the
    cfg2 shape, bf16 writes: the fused route (the automatic choice) against
    the float64 oracle on three blocks of 16 modes over every row and step
    (outputs, final states, write gradients and the nu_log / theta_log
    gradients, which are complete sums per mode), and against the general
    chain kernels (ALGO_CHAIN) on the per-token eta / delta gradients, which
    sum over all 16384 modes."""
    print("[case] P1 operator full size B=8 T=4096 M=16384 G=1 bf16", flush=True)
    B, T, M = 8, 4096, 16384
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(3)
    eta = (O.LOG16 * torch.tanh(0.5 * torch.randn(B, T, 1, device=dev, generator=g))).float()
    delta = (O.HALF_PI * torch.tanh(torch.randn(B, T, 1, device=dev, generator=g))).float()
    p = O.init_params(2 * M, generator=torch.Generator().manual_seed(3))
    nu_log, theta_log = p.nu_log.float().to(dev), p.theta_log.float().to(dev)
    w_re, w_im, dy_re, dy_im = (torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
                                for _ in range(4))

    def run(algorithm):
        ops.set_algorithm(algorithm)
        try:
            y_re, y_im, cs = ops.scan_forward_raw("p1", eta, delta, w_re, w_im, nu_log, theta_log)
            gr = ops.scan_backward_raw("p1", eta, delta, w_re, w_im, cs, dy_re, dy_im, nu_log, theta_log,
                                       y_re=y_re, y_im=y_im)
            torch.cuda.synchronize()
            return y_re, y_im, cs, gr
        finally:
            ops.set_algorithm("auto")

    y_re, y_im, cs, gr = run("auto")
    gc = run("chain")[3]
    tol = 2e-2
    assert rel_err(gr["dg0"], gc["dg0"]) <= tol, "d eta against the chain kernels"
    assert rel_err(gr["dg1"], gc["dg1"]) <= tol, "d delta against the chain kernels"
    del gc
    modes = torch.cat([torch.arange(0, 16), torch.arange(8192, 8208), torch.arange(M - 16, M)]).to(dev)

    def pick(t):
        return t[:, :, modes].double().cpu()

    leaves = [eta.double().cpu(), delta.double().cpu(), pick(w_re), pick(w_im),
              nu_log[modes].double().cpu(), theta_log[modes].double().cpu()]
    leaves = [v.clone().requires_grad_() for v in leaves]
    (hr, hi), last = O.grouped_scan_forward("p1", leaves[0], leaves[1], leaves[2], leaves[3], leaves[4], leaves[5])
    loss = (hr * pick(dy_re)).sum() + (hi * pick(dy_im)).sum()
    _, _, d_wr, d_wi, d_nu, d_th = torch.autograd.grad(loss, leaves)
    assert rel_err(pick(y_re), hr) <= tol
    assert rel_err(pick(y_im), hi) <= tol
    assert rel_err(cs[:, -1][:, modes, 0], last[0]) <= 1e-4  # fp32 state after T steps
    assert rel_err(cs[:, -1][:, modes, 1], last[1]) <= 1e-4
    assert rel_err(pick(gr["dw_re"]), d_wr) <= tol
    assert rel_err(pick(gr["dw_im"]), d_wi) <= tol
    assert rel_err(gr["dnu"][modes], d_nu) <= tol
    assert rel_err(gr["dth"][modes], d_th) <= tol


# ---------------------------------------------------------------------------
# cfg3: real scan, B=4, T=65536, D=512, N=8, fp32, |a| in [0.95, 0.9999]
# ---------------------------------------------------------------------------
def test_cfg3_full_size_sampled_groups_and_drift():
    print("[case] cfg3 full size B=4 T=65536 M=4096 G=512 fp32 real", flush=True)
    B, T, D, N = 4, 65536, 512, 8
    M, G = D * N, D
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    a = 0.95 + 0.0499 * torch.rand(B, T, G, device=dev, generator=g)
    w = torch.randn(B, T, M, device=dev, generator=g)
    dy = torch.randn(B, T, M, device=dev, generator=g)
    y, _, cs = ops.scan_forward_raw("real", a, None, w, None)
    gr = ops.scan_backward_raw("real", a, None, w, None, cs, dy, None, y_re=y)
    torch.cuda.synchronize()
    groups = [0, 300, 511]
    modes = group_modes(groups, N).to(dev)
    gsel = torch.tensor(groups, device=dev)

    def pick(t, idx):
        return t[:, :, idx].double().cpu()

    # the oracle's explicit adjoint (autograd through 65536 per-step selects is
    # quadratic in T); the real scan is the complex one with zero imaginary parts
    a_g = pick(a, gsel)
    h, last = O.grouped_scan_forward("real", a_g, None, pick(w, modes), None)
    zero = torch.zeros_like(h)
    dar, _, d_w, _, _ = O.complex_scan_adjoint(O.expand_groups(a_g, 3 * N), zero, h, zero,
                                              pick(dy, modes), zero)
    d_a = dar.reshape(B, T, 3, N).sum(-1)
    tol = 1e-4
    yg = pick(y, modes)
    assert rel_err(yg, h) <= tol
    # drift at the last step, after 65536 steps and 1024 chunk carries
    assert rel_err(yg[:, -1], h[:, -1]) <= tol
    assert rel_err(cs[:, -1][:, modes], last) <= tol
    assert rel_err(pick(gr["dw_re"], modes), d_w) <= tol
    assert rel_err(pick(gr["dg0"], gsel), d_a) <= tol


# ---------------------------------------------------------------------------
# cfg4: decode, B=256, D=2048, N=16 (M=32768), state fp32 ~ N(0, 0.1)
# ---------------------------------------------------------------------------
def test_cfg4_full_size_decode_steps():
    """Eight in-place scan steps with fresh bf16 writes and polar gates, then
    the state and the last step's output of sampled rows and groups against
    the oracle's sequence scan from the same initial state."""
    print("[case] cfg4 full size B=256 M=32768 G=2048 bf16 polar, 8 steps", flush=True)
    B, D, N, steps = 256, 2048, 16, 8
    M, G = D * N, D
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(3)
    sr = 0.1 * torch.randn(B, M, device=dev, generator=g)
    si = 0.1 * torch.randn(B, M, device=dev, generator=g)
    h0 = (sr.clone(), si.clone())
    w_re = torch.randn(steps, B, M, device=dev, generator=g, dtype=torch.bfloat16)
    w_im = torch.randn(steps, B, M, device=dev, generator=g, dtype=torch.bfloat16)
    r = torch.sigmoid(torch.randn(steps, B, G, device=dev, generator=g) + 2.0).to(torch.bfloat16)
    phi = ((torch.rand(steps, B, G, device=dev, generator=g) * 2 - 1) * math.pi).to(torch.bfloat16)
    for t in range(steps):
        out = ops.scan_step("polar", r[t], phi[t], w_re[t], w_im[t], (sr, si), want_output=True)
    torch.cuda.synchronize()
    rows = torch.tensor([0, 100, 255], device=dev)
    groups = [0, 1000, 2047]
    modes = group_modes(groups, N).to(dev)
    gsel = torch.tensor(groups, device=dev)

    def seq(t, idx):  # [steps, B, K] -> [rows, steps, K]
        return t[:, rows][:, :, idx].permute(1, 0, 2).double().cpu()

    (hr, hi), last = O.grouped_scan_forward(
        "polar", seq(r, gsel), seq(phi, gsel), seq(w_re, modes), seq(w_im, modes),
        h0=(h0[0][rows][:, modes].double().cpu(), h0[1][rows][:, modes].double().cpu()))
    assert rel_err(sr[rows][:, modes], last[0]) <= 1e-4
    assert rel_err(si[rows][:, modes], last[1]) <= 1e-4
    assert rel_err(out[0][rows][:, modes], hr[:, -1]) <= 2e-2
    assert rel_err(out[1][rows][:, modes], hi[:, -1]) <= 2e-2
