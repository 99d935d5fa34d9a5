"""Single-step decode: ``prepare_decode`` / ``run_decode_step``
(sparc-kernal/forward/decode.py:252-306) over the fused HIP decode kernel
(``sparc_decode_step``, replacing ``_latest_sparc_decode``, decode.py:10-75).
"""
from __future__ import annotations

import torch

from . import _lib


def prepare_decode(module) -> None:
    """``prepare_decode`` (forward/decode.py:252-255)."""
    module._inference_fused = True
    module._inference_pack = None


@torch.no_grad()
def latest_sparc_decode(module, x: torch.Tensor, state, out_state=None):
    """One fused P1 step.  ``out_state`` = (re, im) fp32 [B, M] receives the
    new state (it may be ``state`` itself for an in-place update); by default
    fresh tensors are returned, as in the reference (decode.py:58-75)."""
    lib = _lib.load()
    if x.ndim != 2 or x.shape[-1] % 2:
        raise ValueError("SPARC decode expects [B, 2M]")
    x = x.contiguous()
    batch, width = x.shape
    modes = width // 2
    state_r, state_i = state
    if state_r.shape != (batch, modes) or state_i.shape != state_r.shape:
        raise ValueError("SPARC decode state shape mismatch")
    dev = _lib.require_gpu(x, state_r, state_i)
    state_r = state_r.float().contiguous()
    state_i = state_i.float().contiguous()
    if out_state is None:
        new_r = torch.empty_like(state_r)
        new_i = torch.empty_like(state_i)
    else:
        new_r, new_i = out_state
        if (new_r.dtype != torch.float32 or new_i.dtype != torch.float32 or not new_r.is_contiguous()
                or not new_i.is_contiguous() or new_r.shape != (batch, modes) or new_i.shape != (batch, modes)):
            raise ValueError("out_state must be contiguous fp32 [B, M] tensors")
    y = torch.empty_like(x)
    params = [p.detach().float().contiguous() for p in (
        module.phase_direction, module.radial_direction, module.nu_log, module.theta_log,
        module.write_log_gain, module.write_phase_response, module.write_radial_response)]
    P = _lib.ptr
    _lib.check(lib.sparc_decode_step(
        batch, modes, _lib.io_code(x.dtype), P(x), *[P(p) for p in params],
        P(state_r), P(state_i), P(new_r), P(new_i), P(y), _lib.stream_of(dev)), "sparc_decode_step")
    return y, (new_r, new_i)


def run_decode_step(module, x: torch.Tensor, state, segment_pos):
    """``run_decode_step`` (forward/decode.py:273-306); ``segment_pos`` is
    ignored as in the reference.  With ``module.decode_in_place`` the new state
    overwrites ``state`` (same tensors returned)."""
    del segment_pos
    out = state if getattr(module, "decode_in_place", False) else None
    return latest_sparc_decode(module, x, state, out_state=out)


__all__ = ["prepare_decode", "run_decode_step", "latest_sparc_decode"]
