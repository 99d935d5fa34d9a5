"""The module's fused sequence path: ``SPARCMixer.forward`` and its backward
as two C-ABI calls (sparc_mixer_forward / sparc_mixer_backward), reading x
directly instead of materialising the [B, L, M] write tensors.

Same values and gradients as the composed path (controls, write, scan and
epilogue as separate operators) up to float rounding; the write is kept in
fp32 inside the scan instead of being rounded to x's dtype first.  The
states h are saved in x's dtype for the backward, as the reference saves
out_r / out_i (sparc-kernal/backward/scan.py:1348-1356).
"""
from __future__ import annotations

import torch

from . import _lib
from .control import aligned16

_PATHS = ("auto", "fused", "composed")
_path = "auto"


def set_mixer_path(name: str) -> None:
    """Sequence path of ``SPARCMixer.forward``: "fused" (sparc_mixer_*),
    "composed" (controls, write, chunked scan as separate operators) or
    "auto" (the fused path whenever it supports the input)."""
    global _path
    if name not in _PATHS:
        raise ValueError(f"unknown mixer path {name!r}")
    _path = name


def get_mixer_path() -> str:
    return _path


_BWD_PLANS = ("auto", "pieces")


def set_backward_plan(name: str) -> str:
    """Form of the fused module backward (sparc_mixer_backward_plan):
    "auto" runs it in one launch wherever every chain fits on the GPU at once
    (the controls' backward inside), else in time pieces or as a scan launch
    followed by the controls' backward; "pieces" never takes the one-launch
    form.  Process-wide; returns the previous setting."""
    if name not in _BWD_PLANS:
        raise ValueError(f"unknown backward plan {name!r}")
    prev = _lib.load().sparc_mixer_backward_plan(_BWD_PLANS.index(name))
    return _BWD_PLANS[prev]


def backward_form(batch: int, length: int, modes: int, dtype: torch.dtype) -> str:
    """The form sparc_mixer_backward takes for this shape on the current GPU:
    "one_launch", "pieces" or "separate" (sparc_mixer_backward_form)."""
    f = _lib.load().sparc_mixer_backward_form(batch, length, modes, _lib.io_code(dtype))
    if f < 0:
        raise ValueError(_lib.load().sparc_last_error().decode(errors="replace"))
    return ("separate", "pieces", "one_launch")[f]


def fused_supported(x: torch.Tensor, modes: int) -> bool:
    return (x.is_cuda and x.dtype in (torch.float32, torch.bfloat16) and modes % 4 == 0
            and x.ndim == 3 and x.shape[0] > 0)


def use_fused(x: torch.Tensor, modes: int) -> bool:
    if _path == "composed":
        return False
    ok = fused_supported(x, modes)
    if _path == "fused":
        if not ok:
            raise ValueError("the fused mixer path needs GPU fp32/bf16 x [B, L, 2M] with M % 4 == 0")
        return True
    if not ok:
        return False
    return fused_preferred(x.shape[0], x.shape[1], modes)


def fused_preferred(batch: int, length: int, modes: int) -> bool:
    """The "auto" rule: the fused path at every shape.  Its kernels run one
    wave per chain (batch row x 64 modes); with fewer chains than SIMDs they
    split the sequence into segments (a summary pass, a carry across
    segments, then the replay), so they parallelise over time as the composed
    path's look-back scan does, with fewer passes.  Measured on MI355X (bf16,
    forward + backward, fused against composed): B=1 T=65536 width 2048
    1.12 against 1.96 ms; B=1 T=4096 width 4096 0.30 against 0.60 ms; B=4
    T=2048 width 8192 0.63 against 0.99 ms; B=8 T=4096 width 8192 1.94
    against 3.50 ms; widths down to 8 and sequences down to 300 steps about
    0.25 against 0.42 ms."""
    del batch, length, modes
    return True


_PARAMS = ("phase_direction", "radial_direction", "nu_log", "theta_log", "write_log_gain",
           "write_phase_response", "write_radial_response")


class _FusedMixer(torch.autograd.Function):
    """Outputs y = relu(cat(h_re, h_im)) [B, L, 2M] (x's dtype) and the last
    state (last_re, last_im) fp32 [B, M]."""

    @staticmethod
    def forward(ctx, x, phase_direction, radial_direction, nu_log, theta_log, write_log_gain,
                write_phase_response, write_radial_response, energy_response):
        lib = _lib.load()
        _lib.check_params(x.shape[-1], phase_direction=phase_direction, radial_direction=radial_direction,
                          nu_log=nu_log, theta_log=theta_log, write_log_gain=write_log_gain,
                          write_phase_response=write_phase_response, write_radial_response=write_radial_response)
        dev = _lib.require_gpu(x, phase_direction, nu_log)
        x = x.contiguous()
        params = [p.detach().float().contiguous() for p in (
            phase_direction, radial_direction, nu_log, theta_log, write_log_gain,
            write_phase_response, write_radial_response)]
        B, T, W = x.shape
        M = W // 2
        io = _lib.io_code(x.dtype)
        eta = torch.empty(B, T, dtype=torch.float32, device=dev)
        delta = torch.empty_like(eta)
        y = torch.empty_like(x)
        h_re = torch.empty(B, T, M, dtype=x.dtype, device=dev)
        h_im = torch.empty_like(h_re)
        last_re = torch.empty(B, M, dtype=torch.float32, device=dev)
        last_im = torch.empty_like(last_re)
        ws_bytes = lib.sparc_mixer_workspace_bytes(B, T, M, 0)
        if ws_bytes == 0:
            raise ValueError("invalid shape for the fused mixer")
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        P = _lib.ptr
        _lib.check(lib.sparc_mixer_forward(
            B, T, M, io, P(x), *[P(p) for p in params], P(eta), P(delta), P(y), P(h_re), P(h_im),
            P(last_re), P(last_im), P(ws), ws.numel(), _lib.stream_of(dev)), "sparc_mixer_forward")
        ctx.save_for_backward(x, *params, eta, delta, h_re, h_im)
        ctx.set_materialize_grads(False)  # unused last-state outputs: NULL, not zero tensors
        ctx.dtypes = [p.dtype for p in (phase_direction, radial_direction, nu_log, theta_log,
                                        write_log_gain, write_phase_response, write_radial_response)]
        ctx.energy = (energy_response.shape, energy_response.dtype)
        return y, last_re, last_im

    @staticmethod
    def backward(ctx, dy, dlast_re, dlast_im):
        x, pd, rd, nu, th, wlg, wpr, wrr, eta, delta, h_re, h_im = ctx.saved_tensors
        lib = _lib.load()
        dev = x.device
        B, T, W = x.shape
        M = W // 2
        if dy is None:
            dy = torch.zeros_like(x)
        dy = dy.to(x.dtype).contiguous()
        if dlast_re is not None or dlast_im is not None:
            z = torch.zeros(B, M, dtype=torch.float32, device=dev)
            dlast_re = z if dlast_re is None else dlast_re.float().contiguous()
            dlast_im = z.clone() if dlast_im is None else dlast_im.float().contiguous()
        dx = torch.empty_like(x)
        grads = [torch.empty(W + 1, dtype=torch.float32, device=dev) for _ in range(2)]
        grads += [torch.empty(M, dtype=torch.float32, device=dev) for _ in range(5)]
        ws = torch.empty(lib.sparc_mixer_workspace_bytes(B, T, M, 1), dtype=torch.uint8, device=dev)
        P = _lib.ptr
        _lib.check(lib.sparc_mixer_backward(
            B, T, M, _lib.io_code(x.dtype), P(x), P(pd), P(rd), P(nu), P(th), P(wlg), P(wpr), P(wrr),
            P(eta), P(delta), P(h_re), P(h_im), P(dy), P(dlast_re), P(dlast_im), P(dx),
            *[P(g) for g in grads], P(ws), ws.numel(), _lib.stream_of(dev)), "sparc_mixer_backward")
        grads = [g.to(dt) for g, dt in zip(grads, ctx.dtypes)]
        shape, dt = ctx.energy
        # energy_response is an inactive parameter (0 * sum in make_controls): gradient 0
        return (dx, *grads, torch.zeros(shape, dtype=dt, device=dev))


def fused_sequence(module, x: torch.Tensor):
    """(y, (last_re, last_im)) of the module on x through the fused path."""
    y, last_re, last_im = _FusedMixer.apply(
        x, *[getattr(module, n) for n in _PARAMS], module.energy_response)
    return y, (last_re, last_im)


# ---------------------------------------------------------------------------
# the mixer behind its input projection, with the controls folded into it
# ---------------------------------------------------------------------------
_FOLD_MAX_DIM = 4096  # sparc_controls_fold's widest model dimension


class _ProjectedMixer(torch.autograd.Function):
    """y = SPARCMixer(xn @ W^T) for xn [B, L, D] and the projection W [2M, D].

    The controls are p = x.u + b with x = xn W^T, i.e. p = xn (W^T u) + b: a
    [B*L, D] x [D, 2] product instead of two dot products over the 2M-wide x.
    Backward, the controls' input gradient dp0 u_phase + dp1 u_radial is a
    rank-2 term that the projection's own gradients absorb as
    d xn += dp (u W) and dW += u^T (dp^T xn); the direction gradient is
    (dp^T xn) W^T.  The scan, the write and the epilogue run as
    sparc_mixer_scan_forward / _backward."""

    @staticmethod
    def forward(ctx, xn, weight, phase_direction, radial_direction, nu_log, theta_log, write_log_gain,
                write_phase_response, write_radial_response, energy_response):
        lib = _lib.load()
        B, T, D = xn.shape
        W = weight.shape[0]
        if weight.shape != (W, D):
            raise ValueError(f"the projection must be [2M, {D}], got {list(weight.shape)}")
        _lib.check_params(W, phase_direction=phase_direction, radial_direction=radial_direction,
                          nu_log=nu_log, theta_log=theta_log, write_log_gain=write_log_gain,
                          write_phase_response=write_phase_response, write_radial_response=write_radial_response)
        dev = _lib.require_gpu(xn, weight, phase_direction)
        M = W // 2
        x = torch.nn.functional.linear(xn, weight).contiguous()  # [B, T, 2M] in the activation dtype
        # the directions and the per-mode parameters in one fp32 buffer (one
        # copy and at most one cast, not one per tensor): dirs [2, 2M + 1]
        # (phase, radial), then five [M] views
        ps = (phase_direction, radial_direction, nu_log, theta_log, write_log_gain, write_phase_response,
              write_radial_response)
        if all(p.dtype == ps[0].dtype for p in ps):
            flat = torch.cat([p.detach().reshape(-1) for p in ps]).float()
        else:
            flat = torch.cat([p.detach().reshape(-1).float() for p in ps])
        dirs = flat[:2 * (W + 1)].view(2, W + 1)
        params = list(flat[2 * (W + 1):].split(M))
        # the folded directions [W^T u_phase, b_phase], [W^T u_radial, b_radial]
        # in rows of a 16-byte multiple (each row a 16-byte aligned vector);
        # entries 0..D are written below and the kernels read no others
        v = torch.empty(2, (D + 4) // 4 * 4, dtype=torch.float32, device=dev)
        wc = aligned16(weight.detach())
        if D <= _FOLD_MAX_DIM:  # sparc_controls_fold: one pass over W, no fp32 copy of it
            fws = torch.empty(lib.sparc_controls_fold_workspace_bytes(W, D), dtype=torch.uint8, device=dev)
            _lib.check(lib.sparc_controls_fold(W, D, _lib.io_code(wc.dtype), _lib.ptr(wc), _lib.ptr(dirs[0]),
                                               _lib.ptr(dirs[1]), _lib.ptr(v[0]), _lib.ptr(v[1]), _lib.ptr(fws),
                                               fws.numel(), _lib.stream_of(dev)), "sparc_controls_fold")
        else:
            torch.mm(dirs[:, :W], wc.float(), out=v[:, :D])
            v[:, D] = dirs[:, W]
        xn2 = aligned16(xn.detach().reshape(-1, D))
        eta = torch.empty(B * T, dtype=torch.float32, device=dev)
        delta = torch.empty_like(eta)
        P = _lib.ptr
        _lib.check(lib.sparc_controls_forward(B * T, D, _lib.io_code(xn.dtype), P(xn2), P(v[0]), P(v[1]), P(eta),
                                              P(delta), _lib.stream_of(dev)), "sparc_controls_forward")
        io = _lib.io_code(x.dtype)
        y = torch.empty_like(x)
        h_re = torch.empty(B, T, M, dtype=x.dtype, device=dev)
        h_im = torch.empty_like(h_re)
        last_re = torch.empty(B, M, dtype=torch.float32, device=dev)
        last_im = torch.empty_like(last_re)
        ws_bytes = lib.sparc_mixer_workspace_bytes(B, T, M, 0)
        if ws_bytes == 0:
            raise ValueError("invalid shape for the fused mixer")
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.sparc_mixer_scan_forward(
            B, T, M, io, P(x), P(eta), P(delta), *[P(t) for t in params], P(y), P(h_re), P(h_im),
            P(last_re), P(last_im), P(ws), ws.numel(), _lib.stream_of(dev)), "sparc_mixer_scan_forward")
        ctx.save_for_backward(xn2, weight, dirs, v, x, eta, delta, h_re, h_im, *params)
        ctx.dtypes = [t.dtype for t in (phase_direction, radial_direction, nu_log, theta_log,
                                        write_log_gain, write_phase_response, write_radial_response)]
        ctx.energy = (energy_response.shape, energy_response.dtype)
        return y, last_re, last_im

    @staticmethod
    def backward(ctx, dy, dlast_re, dlast_im):
        xn2, weight, dirs, v, x, eta, delta, h_re, h_im, *params = ctx.saved_tensors
        lib = _lib.load()
        dev = x.device
        B, T, W = x.shape
        D = xn2.shape[-1]
        M = W // 2
        if dy is None:
            dy = torch.zeros_like(x)
        dy = dy.to(x.dtype).contiguous()
        if dlast_re is not None or dlast_im is not None:
            z = torch.zeros(B, M, dtype=torch.float32, device=dev)
            dlast_re = z if dlast_re is None else dlast_re.float().contiguous()
            dlast_im = z.clone() if dlast_im is None else dlast_im.float().contiguous()
        dx = torch.empty_like(x)
        deta = torch.empty(B * T, dtype=torch.float32, device=dev)
        ddelta = torch.empty_like(deta)
        # every parameter gradient in one fp32 buffer, laid out as in forward
        # (cast back in one kernel below)
        gflat = torch.empty(2 * (W + 1) + 5 * M, dtype=torch.float32, device=dev)
        g_dirs = gflat[:2 * (W + 1)].view(2, W + 1)
        grads = list(gflat[2 * (W + 1):].split(M))
        ws = torch.empty(lib.sparc_mixer_workspace_bytes(B, T, M, 1), dtype=torch.uint8, device=dev)
        P = _lib.ptr
        _lib.check(lib.sparc_mixer_scan_backward(
            B, T, M, _lib.io_code(x.dtype), P(x), P(eta), P(delta), *[P(t) for t in params],
            P(h_re), P(h_im), P(dy), P(dlast_re), P(dlast_im), P(dx), P(deta), P(ddelta),
            *[P(g) for g in grads], P(ws), ws.numel(), _lib.stream_of(dev)), "sparc_mixer_scan_backward")
        # the controls over xn: g_xn += dp (W^T u) in place and the folded
        # directions' gradients dv = [dp^T xn, sum dp] (dp: the gradients of
        # the two dot products per token)
        dx2 = dx.reshape(-1, W)
        g_xn = aligned16(dx2 @ weight)                                                 # [B*T, D]
        dv = torch.empty(2, v.shape[1], dtype=torch.float32, device=dev)
        cws = torch.empty(lib.sparc_controls_workspace_bytes(B * T, D), dtype=torch.uint8, device=dev)
        _lib.check(lib.sparc_controls_backward(
            B * T, D, _lib.io_code(x.dtype), P(xn2), P(v[0]), P(v[1]), P(eta), P(delta), P(deta), P(ddelta),
            P(g_xn), P(dv[0]), P(dv[1]), P(cws), cws.numel(), _lib.stream_of(dev)), "sparc_controls_backward")
        dpx = dv[:, :D]                                                                # [2, D]
        if D <= _FOLD_MAX_DIM:
            # the folded directions' gradients back through W, and their rank-2
            # share u^T dpx of dW added in place
            g_w = aligned16(dx2.t() @ xn2)
            wc = aligned16(weight)
            _lib.check(lib.sparc_controls_fold_backward(W, D, _lib.io_code(wc.dtype), P(wc), P(dirs[0]), P(dirs[1]),
                                                        P(dv[0]), P(dv[1]), P(g_dirs[0]), P(g_dirs[1]), P(g_w),
                                                        _lib.stream_of(dev)), "sparc_controls_fold_backward")
        else:
            g_w = dx2.t() @ xn2 + (dirs[:, :W].t() @ dpx).to(weight.dtype)
            g_dirs[:, :W] = dpx @ weight.float().t()                                    # [2, 2M + 1]
            g_dirs[:, W] = dv[:, D]
        g_xn = g_xn.reshape(B, T, D)
        if all(dt == ctx.dtypes[0] for dt in ctx.dtypes):
            gc = gflat.to(ctx.dtypes[0])
            out = [gc[:W + 1], gc[W + 1:2 * (W + 1)], *gc[2 * (W + 1):].split(M)]
        else:
            out = [g.to(dt) for g, dt in zip([g_dirs[0], g_dirs[1], *grads], ctx.dtypes)]
        shape, dt = ctx.energy
        return (g_xn, g_w.to(weight.dtype), *out, torch.zeros(shape, dtype=dt, device=dev))


def projected_fused_supported(xn: torch.Tensor, weight: torch.Tensor) -> bool:
    return (xn.is_cuda and xn.dtype in (torch.float32, torch.bfloat16) and weight.dtype == xn.dtype
            and weight.shape[0] % 8 == 0 and xn.ndim == 3 and xn.shape[0] > 0 and xn.shape[-1] % 8 == 0
            and xn.shape[1] > 0)


def projected_sequence(module, xn: torch.Tensor, weight: torch.Tensor):
    """(y, (last_re, last_im)) of ``module`` on ``xn @ weight^T`` with the
    controls folded into the projection."""
    y, last_re, last_im = _ProjectedMixer.apply(
        xn, weight, *[getattr(module, n) for n in _PARAMS], module.energy_response)
    return y, (last_re, last_im)
