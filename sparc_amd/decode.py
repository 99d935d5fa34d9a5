"""Single-step decode: ``prepare_decode`` / ``run_decode_step``
(sparc-kernal/forward/decode.py:252-306) over the HIP decode step, replacing
``_latest_sparc_decode`` (decode.py:10-75): ``sparc_decode_step_prepared``
(per-mode constants cached on the module, controls split over workgroups)
when the mode count is a multiple of 4, else the single-kernel
``sparc_decode_step``.  Before ``prepare_inference`` a step follows the
reference's eager branch (decode.py:296-306) instead: the write is stored in
x's dtype, then one ``sparc_scan_step``.
"""
from __future__ import annotations

import torch

from . import _lib


_CONST_PARAMS = ("nu_log", "theta_log", "write_log_gain", "write_phase_response",
                 "write_radial_response")


def _param_key(module):
    """Identity of the parameters the per-mode constants derive from: their
    storage and in-place version counters (optimizer steps and ``copy_`` bump
    the counters)."""
    return tuple((getattr(module, n).data_ptr(), getattr(module, n)._version, getattr(module, n).device)
                 for n in _CONST_PARAMS)


def _decode_constants(module):
    """The per-mode constants table [M, 8] of the prepared decode step, built
    by ``sparc_decode_prepare`` and rebuilt when a parameter changes."""
    key = _param_key(module)
    cache = getattr(module, "_decode_consts", None)
    if cache is not None and cache[0] == key:
        return cache[1]
    lib = _lib.load()
    modes = module.nu_log.numel()
    _lib.check_params(2 * modes, **{n: getattr(module, n) for n in _CONST_PARAMS})
    params = [getattr(module, n).detach().float().contiguous() for n in _CONST_PARAMS]
    dev = _lib.require_gpu(*params)
    consts = torch.empty(modes, 8, dtype=torch.float32, device=dev)
    P = _lib.ptr
    _lib.check(lib.sparc_decode_prepare(modes, *[P(t) for t in params], P(consts), _lib.stream_of(dev)),
               "sparc_decode_prepare")
    module._decode_consts = (key, consts)
    return consts


def _decode_workspace(module, batch, modes, dev):
    lib = _lib.load()
    need = lib.sparc_decode_workspace_bytes(batch, modes)
    ws = getattr(module, "_decode_ws", None)
    if ws is None or ws.numel() < need or ws.device != dev:
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        module._decode_ws = ws
    return ws


def prepare_decode(module) -> None:
    """``prepare_decode`` (forward/decode.py:252-255).  Also (re)builds the
    per-mode constants of the prepared decode step when the module is on the
    GPU; later steps rebuild them by themselves if a parameter changes in
    place."""
    module._inference_fused = True
    module._inference_pack = None
    module._decode_consts = None
    if module.nu_log.is_cuda and module.nu_log.numel() % 4 == 0:
        _decode_constants(module)


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
    _lib.check_params(width, phase_direction=module.phase_direction, radial_direction=module.radial_direction,
                      **{n: getattr(module, n) for n in _CONST_PARAMS})
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
    P = _lib.ptr
    if modes % 4 == 0:
        dirs = [p.detach().float().contiguous() for p in (module.phase_direction, module.radial_direction)]
        consts = _decode_constants(module)
        ws = _decode_workspace(module, batch, modes, dev)
        _lib.check(lib.sparc_decode_step_prepared(
            batch, modes, _lib.io_code(x.dtype), P(x), P(dirs[0]), P(dirs[1]), P(consts),
            P(state_r), P(state_i), P(new_r), P(new_i), P(y), P(ws), ws.numel(), _lib.stream_of(dev)),
            "sparc_decode_step_prepared")
        return y, (new_r, new_i)
    params = [p.detach().float().contiguous() for p in (
        module.phase_direction, module.radial_direction, module.nu_log, module.theta_log,
        module.write_log_gain, module.write_phase_response, module.write_radial_response)]
    _lib.check(lib.sparc_decode_step(
        batch, modes, _lib.io_code(x.dtype), P(x), *[P(p) for p in params],
        P(state_r), P(state_i), P(new_r), P(new_i), P(y), _lib.stream_of(dev)), "sparc_decode_step")
    return y, (new_r, new_i)


@torch.no_grad()
def eager_decode_step(module, x: torch.Tensor, state, out_state=None):
    """The step before ``prepare_inference``: the reference's eager branch of
    ``run_decode_step`` (forward/decode.py:296-306).  ``make_scan_inputs`` on
    the single token stores the write in x's dtype (``write_r.to(x.dtype)``,
    forward/control.py:162-163; bf16 x rounds it), then h' = a h + w in fp32
    and y = relu(cat(h'_r, h'_i)) in x's dtype.  HIP throughout: the controls
    and write kernels of the composed sequence path, then
    ``sparc_scan_step``.  ``out_state`` as in ``latest_sparc_decode``."""
    from .control import make_scan_inputs
    from .ops import scan_step
    if x.ndim != 2 or x.shape[-1] % 2:
        raise ValueError("SPARC decode expects [B, 2M]")
    batch, width = x.shape
    modes = width // 2
    state_r, state_i = state
    if state_r.shape != (batch, modes) or state_i.shape != state_r.shape:
        raise ValueError("SPARC decode state shape mismatch")
    _lib.require_gpu(x, state_r, state_i)
    eta, delta, write_r, write_i = make_scan_inputs(module, x[:, None])
    if out_state is None:
        new_r = state_r.float().clone(memory_format=torch.contiguous_format)
        new_i = state_i.float().clone(memory_format=torch.contiguous_format)
    else:
        new_r, new_i = out_state
        if (new_r.dtype != torch.float32 or new_i.dtype != torch.float32 or not new_r.is_contiguous()
                or not new_i.is_contiguous() or new_r.shape != (batch, modes) or new_i.shape != (batch, modes)):
            raise ValueError("out_state must be contiguous fp32 [B, M] tensors")
        if new_r.data_ptr() != state_r.data_ptr():
            new_r.copy_(state_r)
        if new_i.data_ptr() != state_i.data_ptr():
            new_i.copy_(state_i)
    y = scan_step("p1", eta, delta, write_r[:, 0], write_i[:, 0], (new_r, new_i),
                  nu_log=module.nu_log.detach().float().contiguous(),
                  theta_log=module.theta_log.detach().float().contiguous(),
                  relu_output=True, want_output=True)
    return y, (new_r, new_i)


def run_decode_step(module, x: torch.Tensor, state, segment_pos):
    """``run_decode_step`` (forward/decode.py:273-306); ``segment_pos`` is
    ignored as in the reference.  After ``prepare_inference`` the fused step
    (``latest_sparc_decode``, the write kept in fp32); before it the
    reference's eager step (``eager_decode_step``, the write stored in x's
    dtype).  With ``module.decode_in_place`` the new state overwrites
    ``state`` (same tensors returned)."""
    del segment_pos
    out = state if getattr(module, "decode_in_place", False) else None
    if not getattr(module, "_inference_fused", False):
        return eager_decode_step(module, x, state, out_state=out)
    return latest_sparc_decode(module, x, state, out_state=out)


__all__ = ["prepare_decode", "run_decode_step", "latest_sparc_decode", "eager_decode_step"]
