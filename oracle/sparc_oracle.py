"""CPU oracle for the SPARC scan path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``sparc_amd``) imports this
module.  It may be imported by ``tests/``, by ``__graft_entry__.smoke()`` and by
``bench.py``'s ``cpu_baseline`` leg, and only as the checker / the timed CPU
baseline, never as a code path of the product.

It restates, in plain PyTorch on the CPU (float64 unless the caller passes
another dtype), the algorithm of the reference's SPARC layer:

* controls   -- ``make_controls``          sparc-kernal/forward/control.py:129-139
                 (JAX: ``control_signals``  sparc-impl/sparc/recurrence.py:20-25)
* write      -- ``make_scan_inputs`` (CPU)  sparc-kernal/forward/control.py:150-163
                 (JAX: recurrence.py:36-54)
* transition -- P1 ``radius``/``phase``     sparc-kernal/forward/scan.py:1584-1589
                 (JAX: recurrence.py:30-35)
* scan       -- ``_eager_complex_scan``     sparc-kernal/forward/scan.py:1355-1375
                 resets / h0 semantics of ``_sparc_tiled_serial_forward``
                 sparc-kernal/forward/scan.py:806-854
* associative scan -- ``_affine_scan_real2`` sparc-kernal/common.py:102-142, the
                 odd/even algorithm of ``jax.lax.associative_scan`` used by
                 ``associative_states`` sparc-impl/sparc/training/bptt.py:23-35
                 (composition rule ``affine_composition`` bptt.py:23-29)
* Hillis-Steele scan -- ``_associative_complex_scan`` forward/scan.py:1378-1395
* explicit adjoint -- ``_complex_backward`` sparc-kernal/backward/scan.py:130-161,
                 ``_real_backward`` backward/scan.py:34-52, reset/h0 handling of
                 ``_sparc_tiled_serial_backward`` backward/scan.py:227-314
* decode     -- eager ``run_decode_step``   sparc-kernal/forward/decode.py:296-306
* module init -- ``SPARCMixer.__init__``    sparc-kernal/sparc.py:59-88
* output     -- ``cat(out_r, out_i).relu()`` forward/scan.py:1598-1603

Gradients are taken with torch autograd through this restatement (float64),
and independently by the explicit adjoint ``complex_scan_adjoint``.

How each function is pinned (tests/test_oracle.py): closed forms of the linear
time-invariant case (geometric series, impulse response), odd/even and
Hillis-Steele associative scans against the sequential scan, real == complex
with zero phase, the explicit adjoint against autograd and against finite
differences (``torch.autograd.gradcheck``), decode-by-steps against the
sequence forward, and small golden vectors written from the reference's own
CPU-capable eager path (tests/golden/).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

LOG16 = math.log(16.0)
HALF_PI = math.pi / 2.0


# --------------------------------------------------------------------------
# parameters (sparc-kernal/sparc.py:59-88)
# --------------------------------------------------------------------------
@dataclass
class MixerParams:
    nu_log: torch.Tensor
    theta_log: torch.Tensor
    phase_direction: torch.Tensor
    radial_direction: torch.Tensor
    write_log_gain: torch.Tensor
    write_phase_response: torch.Tensor
    write_radial_response: torch.Tensor

    @property
    def modes(self) -> int:
        return self.nu_log.numel()

    def to(self, dtype=None, requires_grad=False) -> "MixerParams":
        out = {}
        for k, v in self.__dict__.items():
            t = v.detach().to(dtype=dtype or v.dtype).clone()
            t.requires_grad_(requires_grad)
            out[k] = t
        return MixerParams(**out)

    def tensors(self):
        return [self.nu_log, self.theta_log, self.phase_direction,
                self.radial_direction, self.write_log_gain,
                self.write_phase_response, self.write_radial_response]


def init_params(width: int, generator: torch.Generator | None = None,
                dtype=torch.float64) -> MixerParams:
    """Restates ``SPARCMixer.__init__`` (sparc-kernal/sparc.py:59-88)."""
    if width % 2:
        raise ValueError("SPARC rnn_width must be even")
    modes = width // 2
    tiny = torch.finfo(torch.float32).tiny
    radius_squared = torch.rand(modes, generator=generator, dtype=torch.float32).clamp_min(tiny)
    nu = -0.5 * torch.log(radius_squared)
    theta = (2.0 * math.pi * torch.rand(modes, generator=generator, dtype=torch.float32)).clamp_min(tiny)
    gain = torch.log(torch.sqrt(1.0 - torch.exp(-2.0 * nu)) + 1.0e-8)
    return MixerParams(
        nu_log=torch.log(nu).to(dtype),
        theta_log=torch.log(theta).to(dtype),
        phase_direction=torch.zeros(width + 1, dtype=dtype),
        radial_direction=torch.zeros(width + 1, dtype=dtype),
        write_log_gain=gain.to(dtype),
        write_phase_response=torch.zeros(modes, dtype=dtype),
        write_radial_response=torch.zeros(modes, dtype=dtype),
    )


# --------------------------------------------------------------------------
# P1 controls, write, transition
# --------------------------------------------------------------------------
def controls(x, phase_direction, radial_direction):
    """(eta, delta) per token.  sparc-kernal/forward/control.py:129-139:
    ``p = F.linear(x, dirs[:, :-1], dirs[:, -1])`` with row 0 the phase
    direction and row 1 the radial direction; eta = log16*tanh(p1),
    delta = (pi/2)*tanh(p0)."""
    width = x.shape[-1]
    phase_raw = x @ phase_direction[:width] + phase_direction[width]
    radial_raw = x @ radial_direction[:width] + radial_direction[width]
    return LOG16 * torch.tanh(radial_raw), HALF_PI * torch.tanh(phase_raw)


def write(x, eta, delta, nu_log, write_log_gain, write_phase_response,
          write_radial_response):
    """P1 write (w_r, w_i).  sparc-kernal/forward/control.py:150-163."""
    modes = nu_log.numel()
    nu = torch.exp(nu_log)
    effective_nu = nu * torch.exp(eta[..., None])
    ratio = torch.sqrt(torch.expm1(-2.0 * effective_nu) / torch.expm1(-2.0 * nu))
    phase, radial = delta / HALF_PI, eta / LOG16
    gate = 2.0 * torch.sigmoid(phase[..., None] * write_phase_response
                               + radial[..., None] * write_radial_response)
    gain = torch.exp(write_log_gain) * ratio * gate
    return torch.tanh(x[..., :modes]) * gain, torch.tanh(x[..., modes:]) * gain


def expand_groups(g: torch.Tensor, modes: int) -> torch.Tensor:
    """[..., G] gate groups -> [..., M] with mode m in group m // (M/G)."""
    groups = g.shape[-1]
    if modes % groups:
        raise ValueError("modes must be a multiple of the gate groups")
    return g.repeat_interleave(modes // groups, dim=-1)


def p1_transition(eta, delta, nu_log, theta_log):
    """a = rho*exp(i*(theta + (1-rho)*delta)), rho = exp(-nu*exp(eta)).
    eta/delta are [B,T,G]; sparc-kernal/forward/scan.py:1584-1589,
    sparc-impl/sparc/recurrence.py:30-35."""
    modes = nu_log.numel()
    eta_m, delta_m = expand_groups(eta, modes), expand_groups(delta, modes)
    nu, theta = torch.exp(nu_log), torch.exp(theta_log)
    radius = torch.exp(-nu * torch.exp(eta_m))
    phase = theta + (1.0 - radius) * delta_m
    return radius * torch.cos(phase), radius * torch.sin(phase)


def polar_transition(r, phi, modes):
    """a = r*exp(i*phi) with r, phi given per gate group [B,T,G]."""
    r_m, p_m = expand_groups(r, modes), expand_groups(phi, modes)
    return r_m * torch.cos(p_m), r_m * torch.sin(p_m)


def cartesian_transition(gr, gi, modes):
    """a = gr + i*gi given per gate group [B,T,G] (G = M is the reference's
    per-element ``complex_scan``, sparc-kernal/backward/scan.py:887-919)."""
    return expand_groups(gr, modes), expand_groups(gi, modes)


def reset_mask(batch, length, segment_pos=None, reset_first=False):
    """True where the transition is replaced by 0.  ``segment_pos == 0``
    wins over ``reset_first`` (forward/scan.py:838-843)."""
    if segment_pos is not None:
        return segment_pos == 0
    mask = torch.zeros(batch, length, dtype=torch.bool)
    if reset_first:
        mask[:, 0] = True
    return mask


# --------------------------------------------------------------------------
# scans
# --------------------------------------------------------------------------
def complex_scan(ar, ai, wr, wi, h0=None, resets=None):
    """Sequential h_t = a_t h_{t-1} + w_t over axis 1.

    Follows ``_eager_complex_scan`` (forward/scan.py:1355-1375) and, for
    ``h0``/``resets``, ``_sparc_tiled_serial_forward`` (forward/scan.py:806-854).
    Returns (h_r, h_i) [B,T,M] and the last state (last_r, last_i)."""
    batch, length, modes = wr.shape
    if h0 is None:
        xr = torch.zeros(batch, modes, dtype=wr.dtype)
        xi = torch.zeros(batch, modes, dtype=wr.dtype)
    else:
        xr, xi = h0[0].to(wr.dtype), h0[1].to(wr.dtype)
    outr, outi = [], []
    # unbind, not per-step indexing: its backward stacks the step gradients
    # once, where indexing would build a full-size gradient per step (O(T^2))
    steps = zip(ar.unbind(1), ai.unbind(1), wr.unbind(1), wi.unbind(1))
    for t, (a_r, a_i, w_r, w_i) in enumerate(steps):
        if resets is not None:
            keep = (~resets[:, t]).to(wr.dtype)[:, None]
            a_r, a_i = a_r * keep, a_i * keep
        xr, xi = a_r * xr - a_i * xi + w_r, a_i * xr + a_r * xi + w_i
        outr.append(xr)
        outi.append(xi)
    if length == 0:
        empty = wr.new_zeros(batch, 0, modes)
        return (empty, empty.clone()), (xr, xi)
    return (torch.stack(outr, 1), torch.stack(outi, 1)), (xr, xi)


def real_scan(a, b, h0=None, resets=None):
    """Sequential h_t = a_t h_{t-1} + b_t (forward/scan.py:621-635)."""
    batch, length, width = b.shape
    x = torch.zeros(batch, width, dtype=b.dtype) if h0 is None else h0.to(b.dtype)
    out = []
    for t, (at, bt) in enumerate(zip(a.unbind(1), b.unbind(1))):
        if resets is not None:
            at = at * (~resets[:, t]).to(b.dtype)[:, None]
        x = at * x + bt
        out.append(x)
    if length == 0:
        return b.new_zeros(batch, 0, width), x
    return torch.stack(out, 1), x


def _compose(left, right):
    """``affine_composition`` (sparc-impl/sparc/training/bptt.py:23-29):
    applying ``left`` then ``right``.  Each is (ar, ai, br, bi)."""
    lar, lai, lbr, lbi = left
    rar, rai, rbr, rbi = right
    return (rar * lar - rai * lai, rar * lai + rai * lar,
            rar * lbr - rai * lbi + rbr, rar * lbi + rai * lbr + rbi)


def associative_scan_oddeven(ar, ai, br, bi):
    """Odd/even recursive scan along axis -2: the algorithm of
    ``jax.lax.associative_scan`` (used by ``associative_states``,
    sparc-impl/sparc/training/bptt.py:32-35), as restated for PyTorch in
    ``_affine_scan_real2`` (sparc-kernal/common.py:102-142).

    One deliberate difference: for an odd length, ``_affine_scan_real2`` takes
    ``o[..., :-1]`` as the prior states of the even tail (common.py:124), which
    drops the state the last even element needs, while JAX combines every odd
    result with ``elems[2::2]``.  This follows JAX, the algorithm the
    reference layer runs.  Returns the states (h_r, h_i)."""
    def rec(a_r, a_i, b_r, b_i):
        length = a_r.shape[-2]
        if length < 2:
            return a_r, a_i, b_r, b_i
        ev = (a_r[..., 0::2, :], a_i[..., 0::2, :], b_r[..., 0::2, :], b_i[..., 0::2, :])
        od = (a_r[..., 1::2, :], a_i[..., 1::2, :], b_r[..., 1::2, :], b_i[..., 1::2, :])
        pairs = od[0].shape[-2]
        pair = _compose(tuple(e[..., :pairs, :] for e in ev), od)
        o = rec(*pair)
        n_even = ev[0].shape[-2]
        if n_even > 1:
            prior = tuple(v[..., :n_even - 1, :] for v in o)
            nxt = tuple(v[..., 2::2, :] for v in (a_r, a_i, b_r, b_i))
            tail = _compose(prior, nxt)
            e = tuple(torch.cat((v[..., :1, :], tl), dim=-2) for v, tl in zip(ev, tail))
        else:
            e = ev
        inter = tuple(torch.stack((ee[..., :pairs, :], oo), dim=-2).flatten(-3, -2)
                      for ee, oo in zip(e, o))
        if length % 2:
            inter = tuple(torch.cat((iv, ee[..., -1:, :]), dim=-2) for iv, ee in zip(inter, e))
        return inter

    out = rec(ar, ai, br, bi)
    return out[2], out[3]


def hillis_steele_scan(ar, ai, br, bi):
    """``_associative_complex_scan`` (forward/scan.py:1378-1395), axis 1."""
    par, pai, pbr, pbi = ar, ai, br, bi
    offset = 1
    while offset < ar.shape[1]:
        left = (par[:, :-offset], pai[:, :-offset], pbr[:, :-offset], pbi[:, :-offset])
        right = (par[:, offset:], pai[:, offset:], pbr[:, offset:], pbi[:, offset:])
        c = _compose(left, right)
        par = torch.cat((par[:, :offset], c[0]), 1)
        pai = torch.cat((pai[:, :offset], c[1]), 1)
        pbr = torch.cat((pbr[:, :offset], c[2]), 1)
        pbi = torch.cat((pbi[:, :offset], c[3]), 1)
        offset *= 2
    return pbr, pbi


def complex_scan_adjoint(ar, ai, hr, hi, dyr, dyi, dlast=None, h0=None, resets=None):
    """Explicit reverse-time adjoint of ``complex_scan``.

    Follows ``_complex_backward`` (sparc-kernal/backward/scan.py:130-161):
    lambda_t += dy_t; dA_t = lambda_t * conj(h_{t-1}); dw_t = lambda_t;
    lambda_{t-1} = conj(a_t) * lambda_t, with reset steps (a := 0) and h0 as
    in ``_sparc_tiled_serial_backward`` (backward/scan.py:227-314).
    Returns dar, dai, dwr, dwi, (dh0_r, dh0_i)."""
    batch, length, modes = dyr.shape
    lr = torch.zeros(batch, modes, dtype=dyr.dtype) if dlast is None else dlast[0].clone()
    li = torch.zeros(batch, modes, dtype=dyr.dtype) if dlast is None else dlast[1].clone()
    dar, dai = torch.zeros_like(dyr), torch.zeros_like(dyr)
    dwr, dwi = torch.zeros_like(dyr), torch.zeros_like(dyr)
    for t in range(length - 1, -1, -1):
        lr = lr + dyr[:, t]
        li = li + dyi[:, t]
        if t > 0:
            pr, pi = hr[:, t - 1], hi[:, t - 1]
        elif h0 is not None:
            pr, pi = h0[0], h0[1]
        else:
            pr, pi = torch.zeros_like(lr), torch.zeros_like(li)
        a_r, a_i = ar[:, t], ai[:, t]
        if resets is not None:
            keep = (~resets[:, t]).to(dyr.dtype)[:, None]
            a_r, a_i = a_r * keep, a_i * keep
        else:
            keep = None
        gr = lr * pr + li * pi
        gi = -lr * pi + li * pr
        if keep is not None:
            gr, gi = gr * keep, gi * keep
        dar[:, t], dai[:, t] = gr, gi
        dwr[:, t], dwi[:, t] = lr, li
        lr, li = a_r * lr + a_i * li, -a_i * lr + a_r * li
    return dar, dai, dwr, dwi, (lr, li)


# --------------------------------------------------------------------------
# module level
# --------------------------------------------------------------------------
def mixer_forward(p: MixerParams, x: torch.Tensor, return_cache=False,
                  initial_state=None, segment_pos=None, reset_first=False,
                  write_dtype=None):
    """``SPARCMixer.forward`` = ``run_sequence`` (forward/scan.py:1398-1603):
    controls, P1 write, P1 transition, scan, ``relu(cat(h_r, h_i))``.

    ``write_dtype`` (e.g. torch.bfloat16) models the reference's cast of the
    write to x's dtype (``write_r.to(x.dtype)``, forward/control.py:162-163):
    the write's value is rounded to it, and autograd rounds the write's
    gradient through the same cast.  The controls stay in the compute dtype
    (``x.float()``, control.py:129-137)."""
    eta, delta = controls(x, p.phase_direction, p.radial_direction)
    wr, wi = write(x, eta, delta, p.nu_log, p.write_log_gain,
                   p.write_phase_response, p.write_radial_response)
    if write_dtype is not None:
        wr, wi = wr.to(write_dtype).to(wr.dtype), wi.to(write_dtype).to(wi.dtype)
    ar, ai = p1_transition(eta[..., None], delta[..., None], p.nu_log, p.theta_log)
    resets = None
    if segment_pos is not None or reset_first:
        resets = reset_mask(x.shape[0], x.shape[1], segment_pos, reset_first)
    (hr, hi), last = complex_scan(ar, ai, wr, wi, h0=initial_state, resets=resets)
    y = torch.cat((hr, hi), dim=-1).relu()
    return y, (last if return_cache else None)


def decode_step(p: MixerParams, x: torch.Tensor, state, write_dtype=None):
    """Eager ``run_decode_step`` (forward/decode.py:296-306); x is [B, 2M].
    ``write_dtype`` models the cast of the write to x's dtype inside
    ``make_scan_inputs`` (forward/control.py:162-163), as in ``mixer_forward``."""
    eta, delta = controls(x, p.phase_direction, p.radial_direction)
    wr, wi = write(x[:, None], eta[:, None], delta[:, None], p.nu_log,
                   p.write_log_gain, p.write_phase_response,
                   p.write_radial_response)
    if write_dtype is not None:
        wr, wi = wr.to(write_dtype).to(wr.dtype), wi.to(write_dtype).to(wi.dtype)
    ar, ai = p1_transition(eta[:, None, None], delta[:, None, None], p.nu_log, p.theta_log)
    ar, ai, wr, wi = ar[:, 0], ai[:, 0], wr[:, 0], wi[:, 0]
    old_r, old_i = state
    new_r = ar * old_r - ai * old_i + wr
    new_i = ai * old_r + ar * old_i + wi
    return torch.cat((new_r, new_i), -1).relu(), (new_r, new_i)


def grouped_scan_forward(transition: str, g0, g1, w_re, w_im, nu_log=None,
                         theta_log=None, h0=None, segment_pos=None,
                         reset_first=False, relu_output=False):
    """Scan core with gates given per group: ``p1`` (eta, delta), ``polar``
    (r, phi), ``cartesian`` (ar, ai) or ``real`` (a).  Returns the output
    ((h_r, h_i) or visible relu(cat) [B,T,2M], or h for real) and the last
    state.  Everything in the dtype of the inputs."""
    if transition == "real":
        width = w_re.shape[-1]
        resets = None
        if segment_pos is not None or reset_first:
            resets = reset_mask(w_re.shape[0], w_re.shape[1], segment_pos, reset_first)
        return real_scan(expand_groups(g0, width), w_re, h0=h0, resets=resets)
    modes = w_re.shape[-1]
    if transition == "p1":
        ar, ai = p1_transition(g0, g1, nu_log, theta_log)
    elif transition == "polar":
        ar, ai = polar_transition(g0, g1, modes)
    elif transition == "cartesian":
        ar, ai = cartesian_transition(g0, g1, modes)
    else:
        raise ValueError(transition)
    resets = None
    if segment_pos is not None or reset_first:
        resets = reset_mask(w_re.shape[0], w_re.shape[1], segment_pos, reset_first)
    (hr, hi), last = complex_scan(ar, ai, w_re, w_im, h0=h0, resets=resets)
    if relu_output:
        return torch.cat((hr, hi), -1).relu(), last
    return (hr, hi), last
