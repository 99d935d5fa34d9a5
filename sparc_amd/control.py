"""P1 controls and write prologue.

``make_controls`` (sparc-kernal/forward/control.py:129-139) runs as HIP
kernels (sparc_controls_forward / sparc_controls_backward) for inputs whose
width is a multiple of 8, and in the reference's torch formulation
otherwise; the write ``gain * tanh(x)`` and its backward run as HIP kernels
(sparc_write_forward / sparc_write_backward) in place of
``_latest_write_forward`` / ``_latest_write_backward``
(sparc-kernal/forward/control.py:166-195, backward/control.py:10-89).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import _lib

LOG16 = math.log(16.0)
HALF_PI = math.pi / 2.0


def aligned16(t: torch.Tensor) -> torch.Tensor:
    """``t`` contiguous with a 16-byte aligned start (a copy if needed)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _Controls(torch.autograd.Function):
    """eta, delta of rows x [..., W] against two directions [W + 1] (bias
    last) through sparc_controls_forward / sparc_controls_backward."""

    @staticmethod
    def forward(ctx, x, phase_direction, radial_direction):
        lib = _lib.load()
        W = x.shape[-1]
        _lib.check_params(W, phase_direction=phase_direction, radial_direction=radial_direction)
        dev = _lib.require_gpu(x, phase_direction, radial_direction)
        rows = x.numel() // W
        x2 = aligned16(x)
        pd = aligned16(phase_direction.detach().float())
        rd = aligned16(radial_direction.detach().float())
        eta = torch.empty(x.shape[:-1], dtype=torch.float32, device=dev)
        delta = torch.empty_like(eta)
        P = _lib.ptr
        _lib.check(lib.sparc_controls_forward(rows, W, _lib.io_code(x.dtype), P(x2), P(pd), P(rd), P(eta), P(delta),
                                              _lib.stream_of(dev)), "sparc_controls_forward")
        ctx.save_for_backward(x2, pd, rd, eta, delta)
        ctx.dtypes = (phase_direction.dtype, radial_direction.dtype)
        return eta, delta

    @staticmethod
    def backward(ctx, deta, ddelta):
        x2, pd, rd, eta, delta = ctx.saved_tensors
        lib = _lib.load()
        dev = x2.device
        W = x2.shape[-1]
        rows = x2.numel() // W
        deta = torch.zeros_like(eta) if deta is None else deta.float().contiguous()
        ddelta = torch.zeros_like(delta) if ddelta is None else ddelta.float().contiguous()
        dx = torch.zeros_like(x2)  # the kernel adds the controls' term in place
        dpd = torch.empty(W + 1, dtype=torch.float32, device=dev)
        drd = torch.empty_like(dpd)
        ws = torch.empty(lib.sparc_controls_workspace_bytes(rows, W), dtype=torch.uint8, device=dev)
        P = _lib.ptr
        _lib.check(lib.sparc_controls_backward(
            rows, W, _lib.io_code(x2.dtype), P(x2), P(pd), P(rd), P(eta), P(delta), P(deta), P(ddelta), P(dx),
            P(dpd), P(drd), P(ws), ws.numel(), _lib.stream_of(dev)), "sparc_controls_backward")
        return dx, dpd.to(ctx.dtypes[0]), drd.to(ctx.dtypes[1])


def controls_supported(x: torch.Tensor) -> bool:
    return x.is_cuda and x.dtype in (torch.float32, torch.bfloat16) and x.shape[-1] % 8 == 0 and x.numel() > 0


def make_controls(module, x: torch.Tensor):
    """(eta, delta) fp32 [B, L]: eta = log16*tanh(x.u_r + b_r),
    delta = (pi/2)*tanh(x.u_p + b_p).  sparc-kernal/forward/control.py:129-139."""
    inactive_energy_slot = 0.0 * module.energy_response.sum()
    if controls_supported(x):
        eta, delta = _Controls.apply(x, module.phase_direction, module.radial_direction)
        return eta + inactive_energy_slot, delta
    directions = torch.stack((module.phase_direction, module.radial_direction))
    with torch.autocast(device_type=x.device.type, enabled=False):
        projected = F.linear(x.float(), directions[:, :-1].float(), directions[:, -1].float())
        return (
            LOG16 * torch.tanh(projected[..., 1]) + inactive_energy_slot,
            HALF_PI * torch.tanh(projected[..., 0]),
        )


class _LatestSPARCWrite(torch.autograd.Function):
    """``_LatestSPARCWrite`` (sparc-kernal/backward/control.py:92-129)."""

    @staticmethod
    def forward(ctx, raw_x, eta, delta, nu_log, write_log_gain, phase_response, radial_response):
        lib = _lib.load()
        if raw_x.ndim != 3 or eta.shape != raw_x.shape[:2] or delta.shape != eta.shape:
            raise ValueError("the write needs x [B, L, 2M] and eta, delta [B, L]")
        _lib.check_params(raw_x.shape[-1], nu_log=nu_log, write_log_gain=write_log_gain,
                          write_phase_response=phase_response, write_radial_response=radial_response)
        dev = _lib.require_gpu(raw_x, eta, delta, nu_log)
        raw_x = raw_x.contiguous()
        eta, delta = eta.float().contiguous(), delta.float().contiguous()
        params = [p.float().contiguous() for p in (nu_log, write_log_gain, phase_response, radial_response)]
        B, L, W = raw_x.shape
        M, rows = W // 2, B * L
        w_r = torch.empty(B, L, M, dtype=raw_x.dtype, device=dev)
        w_i = torch.empty_like(w_r)
        P = _lib.ptr
        _lib.check(lib.sparc_write_forward(
            rows, M, _lib.io_code(raw_x.dtype), P(raw_x), P(eta), P(delta),
            *[P(p) for p in params], P(w_r), P(w_i), _lib.stream_of(dev)), "sparc_write_forward")
        ctx.save_for_backward(raw_x, eta, delta, *params)
        ctx.param_dtypes = (nu_log.dtype, write_log_gain.dtype, phase_response.dtype, radial_response.dtype)
        return w_r, w_i

    @staticmethod
    def backward(ctx, grad_r, grad_i):
        raw_x, eta, delta, nu_log, wlg, wpr, wrr = ctx.saved_tensors
        lib = _lib.load()
        dev = raw_x.device
        B, L, W = raw_x.shape
        M, rows = W // 2, B * L
        if grad_r is None:
            grad_r = torch.zeros(B, L, M, dtype=raw_x.dtype, device=dev)
        if grad_i is None:
            grad_i = torch.zeros(B, L, M, dtype=raw_x.dtype, device=dev)
        grad_r = grad_r.to(raw_x.dtype).contiguous()
        grad_i = grad_i.to(raw_x.dtype).contiguous()
        dx = torch.empty_like(raw_x)
        deta = torch.empty(B, L, dtype=torch.float32, device=dev)
        ddelta = torch.empty_like(deta)
        grads = [torch.empty(M, dtype=torch.float32, device=dev) for _ in range(4)]
        ws_bytes = lib.sparc_write_workspace_bytes(rows, M)
        ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
        P = _lib.ptr
        _lib.check(lib.sparc_write_backward(
            rows, M, _lib.io_code(raw_x.dtype), P(raw_x), P(eta), P(delta), P(nu_log), P(wlg),
            P(wpr), P(wrr), P(grad_r), P(grad_i), P(dx), P(deta), P(ddelta),
            *[P(g) for g in grads], P(ws), ws.numel(), _lib.stream_of(dev)), "sparc_write_backward")
        grads = [g.to(dt) for g, dt in zip(grads, ctx.param_dtypes)]
        return (dx, deta, ddelta, *grads)


def latest_sparc_write(raw_x, eta, delta, nu_log, write_log_gain, phase_response, radial_response):
    """``latest_sparc_write`` (sparc-kernal/backward/control.py:132-137)."""
    return _LatestSPARCWrite.apply(raw_x, eta, delta, nu_log, write_log_gain,
                                   phase_response, radial_response)


def make_scan_inputs(module, x: torch.Tensor):
    """``make_scan_inputs`` (sparc-kernal/forward/control.py:141-149):
    (eta, delta, write_r, write_i)."""
    eta, delta = make_controls(module, x)
    write_r, write_i = latest_sparc_write(
        x, eta, delta, module.nu_log, module.write_log_gain,
        module.write_phase_response, module.write_radial_response)
    return eta, delta, write_r, write_i
