"""SPARC scan operators: autograd Functions over the HIP C ABI.

Public names, argument meaning and ``ValueError`` behaviour follow the
reference operators re-exported by ``sparc-kernal/sparc.py:18-55`` and defined
in ``sparc-kernal/backward/scan.py:1643-1877``.  Every operator runs the same
single-pass chunked HIP scan (include/sparc_hip.h); the reference's
implementation knobs (chunk sizes, mode blocks, carry strategies) are
validated exactly as the reference validates them and otherwise do not change
the computation.

Grouped-gate extensions (not in the reference): ``chunk_scan`` with
``transition`` in {"p1", "polar", "cartesian", "real"} and gates [B, T, G]
shared by groups of M/G modes.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import ALGO_FLAGS, FLAG_RELU_OUTPUT, FLAG_RESET_FIRST, TRANSITIONS

_algorithm = "auto"


def set_algorithm(name: str) -> None:
    """Scan algorithm for every later call: "auto" (by shape), "lookback"
    (one workgroup per (chain, chunk) tile, carries between workgroups),
    "chain" (one workgroup per (batch row, mode block) chain) or "serial"
    (one wave per chain, step by step; lane-shared gates only, else "chain")."""
    global _algorithm
    if name not in ALGO_FLAGS:
        raise ValueError(f"unknown scan algorithm {name!r}")
    _algorithm = name


def get_algorithm() -> str:
    return _algorithm


def _flags(relu_output, reset_first):
    return ((FLAG_RELU_OUTPUT if relu_output else 0) | (FLAG_RESET_FIRST if reset_first else 0)
            | ALGO_FLAGS[_algorithm])


# ---------------------------------------------------------------------------
# raw calls
# ---------------------------------------------------------------------------
def _desc(transition, B, T, M, G, io, gate_io, flags):
    return _lib.ScanDesc(B, T, M, G, TRANSITIONS[transition], io, gate_io, flags)


def _workspace(n_bytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(n_bytes), 256), dtype=torch.uint8, device=device)


def _check_scan_inputs(transition, g0, g1, w_re, w_im, nu_log, theta_log, h0_re, h0_im,
                       segment_pos, step=False):
    """Shapes and dtypes of a raw launch's inputs against its descriptor
    (B, T, M from w_re, G from g0); ValueError on any mismatch.  ``step``:
    the single-step layout (w [B, M], gates [B, G], no T axis)."""
    if transition not in TRANSITIONS:
        raise ValueError(f"unknown transition {transition!r}")
    cplx, p1 = transition != "real", transition == "p1"
    lead = tuple(w_re.shape[:-1])
    if w_re.ndim != (2 if step else 3) or g0.ndim != w_re.ndim or tuple(g0.shape[:-1]) != lead:
        raise ValueError("writes must be [B, T, M] and gates [B, T, G] ([B, M], [B, G] for a step)")
    M, G, io = w_re.shape[-1], g0.shape[-1], w_re.dtype
    if G <= 0 or M % G:
        raise ValueError("the gate group count G must divide M")
    gate_dtype = torch.float32 if p1 else g0.dtype
    if not p1 and gate_dtype != io and not (gate_dtype == torch.float32 and io == torch.bfloat16):
        raise ValueError("gates must be in the writes' dtype, or fp32 beside bf16 writes")
    _lib.expect(g0, lead + (G,), gate_dtype, "g0")
    if cplx:
        _lib.expect(g1, lead + (G,), gate_dtype, "g1")
        _lib.expect(w_im, lead + (M,), io, "w_im")
    if p1:
        _lib.expect(nu_log, (M,), torch.float32, "nu_log")
        _lib.expect(theta_log, (M,), torch.float32, "theta_log")
    B = lead[0]
    if h0_re is not None:
        _lib.expect(h0_re, (B, M), torch.float32, "h0_re")
    if h0_im is not None or (h0_re is not None and cplx):
        _lib.expect(h0_im, (B, M), torch.float32, "h0_im")
    if segment_pos is not None:
        _lib.expect(segment_pos, lead, torch.int32, "segment_pos")


def scan_forward_raw(transition, g0, g1, w_re, w_im, nu_log=None, theta_log=None,
                     h0_re=None, h0_im=None, segment_pos=None, reset_first=False,
                     relu_output=False):
    """One forward launch.  Inputs must be contiguous GPU tensors of the
    dtypes the C ABI expects (ValueError otherwise).  Returns (y_re, y_im,
    chunk_state)."""
    lib = _lib.load()
    _check_scan_inputs(transition, g0, g1, w_re, w_im, nu_log, theta_log, h0_re, h0_im, segment_pos)
    dev = _lib.require_gpu(g0, g1, w_re, w_im, nu_log, theta_log, h0_re, h0_im, segment_pos)
    B, T, M = w_re.shape
    G = g0.shape[-1]
    io = _lib.io_code(w_re.dtype)
    gate_io = _lib.io_code(g0.dtype)
    d = _desc(transition, B, T, M, G, io, gate_io, _flags(relu_output, reset_first))
    n_chunks = lib.sparc_scan_chunk_count(ctypes.byref(d))
    cplx = transition != "real"
    if relu_output:
        y_re, y_im = torch.empty(B, T, 2 * M, dtype=w_re.dtype, device=dev), None
    else:
        y_re = torch.empty(B, T, M, dtype=w_re.dtype, device=dev)
        y_im = torch.empty(B, T, M, dtype=w_re.dtype, device=dev) if cplx else None
    cs_shape = (B, n_chunks, M, 2) if cplx else (B, n_chunks, M)
    chunk_state = torch.empty(cs_shape, dtype=torch.float32, device=dev)
    ws_bytes = lib.sparc_scan_workspace_bytes(ctypes.byref(d), 0)
    if ws_bytes == 0:
        raise ValueError("invalid SPARC scan shapes/dtypes (sparc_scan_workspace_bytes == 0)")
    ws = _workspace(ws_bytes, dev)
    P = _lib.ptr
    _lib.check(lib.sparc_scan_forward(
        ctypes.byref(d), P(g0), P(g1), P(nu_log), P(theta_log), P(w_re), P(w_im),
        P(h0_re), P(h0_im), P(segment_pos), P(y_re), P(y_im), P(chunk_state),
        P(ws), ws.numel(), _lib.stream_of(dev)), "sparc_scan_forward")
    return y_re, y_im, chunk_state


def scan_backward_raw(transition, g0, g1, w_re, w_im, chunk_state, dy_re, dy_im,
                      nu_log=None, theta_log=None, h0_re=None, h0_im=None,
                      segment_pos=None, reset_first=False, relu_output=False,
                      dlast_re=None, dlast_im=None, want_dh0=False, y_re=None, y_im=None):
    """One backward launch.  ``y_re``/``y_im``: the forward's outputs (no relu
    epilogue), from which plans with lane-shared gates read the states instead
    of recomputing them.  Returns dict of gradients."""
    lib = _lib.load()
    _check_scan_inputs(transition, g0, g1, w_re, w_im, nu_log, theta_log, h0_re, h0_im, segment_pos)
    B, T, M = w_re.shape
    G = g0.shape[-1]
    io = _lib.io_code(w_re.dtype)
    gate_io = _lib.io_code(g0.dtype)
    d = _desc(transition, B, T, M, G, io, gate_io, _flags(relu_output, reset_first))
    cplx = transition != "real"
    n_chunks = lib.sparc_scan_chunk_count(ctypes.byref(d))
    _lib.expect(chunk_state, (B, n_chunks, M, 2) if cplx else (B, n_chunks, M), torch.float32, "chunk_state")
    _lib.expect(dy_re, (B, T, 2 * M if relu_output else M), w_re.dtype, "dy_re")
    if cplx and not relu_output:
        _lib.expect(dy_im, (B, T, M), w_re.dtype, "dy_im")
    for name, t in (("y_re", y_re), ("y_im", y_im)):
        if t is not None:
            _lib.expect(t, (B, T, M), w_re.dtype, name)
    for name, t in (("dlast_re", dlast_re), ("dlast_im", dlast_im)):
        if t is not None:
            _lib.expect(t, (B, M), torch.float32, name)
    dev = _lib.require_gpu(g0, w_re, chunk_state, dy_re)
    dw_re = torch.empty_like(w_re)
    dw_im = torch.empty_like(w_im) if cplx else None
    dg0 = torch.empty_like(g0)
    dg1 = torch.empty_like(g1) if cplx else None
    p1 = transition == "p1"
    dnu = torch.empty(M, dtype=torch.float32, device=dev) if p1 else None
    dth = torch.empty(M, dtype=torch.float32, device=dev) if p1 else None
    dh0_re = torch.empty(B, M, dtype=torch.float32, device=dev) if want_dh0 else None
    dh0_im = torch.empty(B, M, dtype=torch.float32, device=dev) if (want_dh0 and cplx) else None
    ws_bytes = lib.sparc_scan_workspace_bytes(ctypes.byref(d), 1)
    if ws_bytes == 0:
        raise ValueError("invalid SPARC scan shapes/dtypes (sparc_scan_workspace_bytes == 0)")
    ws = _workspace(ws_bytes, dev)
    P = _lib.ptr
    _lib.check(lib.sparc_scan_backward(
        ctypes.byref(d), P(g0), P(g1), P(nu_log), P(theta_log), P(w_re), P(w_im),
        P(y_re), P(y_im), P(h0_re), P(h0_im), P(segment_pos), P(chunk_state), P(dy_re), P(dy_im),
        P(dlast_re), P(dlast_im), P(dw_re), P(dw_im), P(dg0), P(dg1), P(dnu), P(dth),
        P(dh0_re), P(dh0_im), P(ws), ws.numel(), _lib.stream_of(dev)), "sparc_scan_backward")
    return dict(dw_re=dw_re, dw_im=dw_im, dg0=dg0, dg1=dg1, dnu=dnu, dth=dth,
                dh0_re=dh0_re, dh0_im=dh0_im)


@torch.no_grad()
def scan_step(transition, g0, g1, w_re, w_im, state, nu_log=None, theta_log=None,
              relu_output=False, want_output=False, reset_first=False):
    """One scan step for B independent rows with the state updated in place
    (the scan-core decode step): h <- a h + w, the same as ``chunk_scan`` with
    T = 1 and the state as initial state.

    g0, g1: gates [B, G] (fp32 eta, delta for "p1"; otherwise bf16 beside bf16
    w, else passed as fp32);
    w_re, w_im: [B, M]; state: (state_re, state_im) fp32 [B, M] contiguous
    (a single tensor for "real"), modified in place.  Returns the new state in
    w's dtype (``relu(cat)`` [B, 2M] with ``relu_output``) when
    ``want_output``, else None."""
    if transition not in TRANSITIONS:
        raise ValueError(f"unknown transition {transition!r}")
    cplx = transition != "real"
    st_re, st_im = (state if cplx else (state, None))
    if w_re.ndim != 2 or st_re.shape != w_re.shape or st_re.dtype != torch.float32:
        raise ValueError("scan_step expects w [B, M] and an fp32 state [B, M]")
    if not st_re.is_contiguous() or (st_im is not None and not st_im.is_contiguous()):
        raise ValueError("scan_step updates the state in place: it must be contiguous")
    if cplx and (st_im is None or st_im.shape != st_re.shape or st_im.dtype != torch.float32 or w_im is None):
        raise ValueError("complex scan steps need fp32 (state_re, state_im) and w_im")
    B, M = w_re.shape
    G = g0.shape[-1]
    if g0.shape != (B, G) or M % G or (cplx and (g1 is None or g1.shape != g0.shape)):
        raise ValueError("gates must be [B, G] with G dividing M")
    p1 = transition == "p1"
    io = _lib.io_code(w_re.dtype)
    if not p1:
        g0, g1 = _gate_dtype(g0, g1, w_re.dtype)
    else:
        g0, g1 = g0.float(), g1.float()
    gate_io = _lib.io_code(g0.dtype)
    lib = _lib.load()
    _check_scan_inputs(transition, g0, g1, w_re, w_im, nu_log, theta_log, None, None, None, step=True)
    dev = _lib.require_gpu(g0, w_re, st_re)
    y_re = y_im = None
    if want_output:
        if relu_output:
            y_re = torch.empty(B, 2 * M, dtype=w_re.dtype, device=dev)
        else:
            y_re = torch.empty_like(w_re)
            y_im = torch.empty_like(w_re) if cplx else None
    d = _desc(transition, B, 1, M, G, io, gate_io, _flags(relu_output, reset_first) & 3)
    P = _lib.ptr
    _lib.check(lib.sparc_scan_step(
        ctypes.byref(d), P(_c(g0)), P(_c(g1)), P(nu_log), P(theta_log), P(_c(w_re)), P(_c(w_im)),
        P(st_re), P(st_im), P(y_re), P(y_im), _lib.stream_of(dev)), "sparc_scan_step")
    if not want_output:
        return None
    return y_re if (relu_output or not cplx) else (y_re, y_im)


# ---------------------------------------------------------------------------
# autograd
# ---------------------------------------------------------------------------
def _c(t):
    return None if t is None else t.contiguous()


def _gate_dtype(g0, g1, io_dtype):
    """Gates of the polar, cartesian and real transitions keep bf16 only
    beside bf16 writes; otherwise they go to the library as fp32 (exact for
    bf16 gates).  The reference loads ``a`` in its own dtype and computes in
    fp32 whatever the writes' dtype (forward/scan.py:629-630, 707-710)."""
    both_bf16 = g0.dtype == torch.bfloat16 and (g1 is None or g1.dtype == torch.bfloat16)
    dt = torch.bfloat16 if (both_bf16 and io_dtype == torch.bfloat16) else torch.float32
    return g0.to(dt), (None if g1 is None else g1.to(dt))


class _ChunkScan(torch.autograd.Function):
    """Differentiable chunked scan for every transition.

    Outputs (y_re, y_im, last_re, last_im); y_re is the visible relu(cat)
    output with ``relu_output``; unused outputs are empty tensors."""

    @staticmethod
    def forward(ctx, transition, relu_output, reset_first, g0, g1, nu_log, theta_log,
                w_re, w_im, h0_re, h0_im, segment_pos):
        y_re, y_im, cs = scan_forward_raw(
            transition, g0, g1, w_re, w_im, nu_log, theta_log, h0_re, h0_im,
            segment_pos, reset_first, relu_output)
        cplx = transition != "real"
        B, T, M = w_re.shape
        if T > 0:
            last_re = cs[:, -1, :, 0].contiguous() if cplx else cs[:, -1].contiguous()
            last_im = cs[:, -1, :, 1].contiguous() if cplx else w_re.new_empty(0, dtype=torch.float32)
        else:
            zero = torch.zeros(B, M, dtype=torch.float32, device=w_re.device)
            last_re = h0_re.clone() if h0_re is not None else zero
            last_im = (h0_im.clone() if h0_im is not None else zero.clone()) if cplx \
                else w_re.new_empty(0, dtype=torch.float32)
        # without the relu epilogue y is the state (rounded to the I/O dtype),
        # which the backward reads instead of recomputing it
        saved_y = (None, None) if relu_output else (y_re, y_im)
        ctx.save_for_backward(g0, g1, nu_log, theta_log, w_re, w_im, h0_re, h0_im, segment_pos, cs,
                              *saved_y)
        ctx.cfg = (transition, relu_output, reset_first)
        if y_im is None:
            y_im = w_re.new_empty(0)
        ctx.mark_non_differentiable(y_im) if y_im.numel() == 0 else None
        return y_re, y_im, last_re, last_im

    @staticmethod
    def backward(ctx, dy_re, dy_im, dlast_re, dlast_im):
        g0, g1, nu_log, theta_log, w_re, w_im, h0_re, h0_im, segment_pos, cs, ys_re, ys_im = \
            ctx.saved_tensors
        transition, relu_output, reset_first = ctx.cfg
        cplx = transition != "real"
        if dy_re is None:
            shape = (*w_re.shape[:2], 2 * w_re.shape[2]) if relu_output else w_re.shape
            dy_re = torch.zeros(shape, dtype=w_re.dtype, device=w_re.device)
        if cplx and not relu_output and dy_im is None:
            dy_im = torch.zeros_like(w_re)
        if not cplx or relu_output:
            dy_im = None
        if dlast_re is not None or dlast_im is not None:
            B, M = w_re.shape[0], w_re.shape[2]
            z = torch.zeros(B, M, dtype=torch.float32, device=w_re.device)
            dlast_re = z if dlast_re is None else dlast_re.float().contiguous()
            if cplx:
                dlast_im = z.clone() if dlast_im is None else dlast_im.float().contiguous()
            else:
                dlast_im = None
        g = scan_backward_raw(
            transition, g0, g1, w_re, w_im, cs, _c(dy_re).to(w_re.dtype), _c(dy_im).to(w_re.dtype) if dy_im is not None else None,
            nu_log, theta_log, h0_re, h0_im, segment_pos, reset_first, relu_output,
            dlast_re, dlast_im, want_dh0=h0_re is not None, y_re=ys_re, y_im=ys_im)
        return (None, None, None, g["dg0"], g["dg1"], g["dnu"], g["dth"],
                g["dw_re"], g["dw_im"], g["dh0_re"], g["dh0_im"], None)


def chunk_scan(transition: str, g0, g1, w_re, w_im=None, nu_log=None, theta_log=None,
               initial_state=None, segment_pos=None, reset_first=False,
               relu_output=False):
    """Differentiable scan h_t = a_t h_{t-1} + w_t with gates per group.

    transition: "p1" (g0 = eta, g1 = delta, fp32 [B,T,G]; nu_log/theta_log [M]),
    "polar" (g0 = r, g1 = phi), "cartesian" (g0 + i g1), "real" (g0 = a).
    Gates of non-P1 transitions keep their dtype: bf16 gates with bf16 w run
    in bf16 I/O, anything else passes fp32 gates (bf16 gates beside fp32 w are
    widened exactly); their gradients come back in the gates' dtype.
    Returns (y, last): y = (h_re, h_im) [B,T,M] each, or relu(cat) [B,T,2M]
    with relu_output, or h [B,T,M] for "real"; last = (last_re, last_im) fp32
    [B,M] (a single tensor for "real")."""
    if transition not in TRANSITIONS:
        raise ValueError(f"unknown transition {transition!r}")
    cplx = transition != "real"
    if w_re.ndim != 3:
        raise ValueError("writes must be [B, T, M]")
    B, T, M = w_re.shape
    if cplx and (w_im is None or w_im.shape != w_re.shape):
        raise ValueError("complex scans need matching w_re, w_im [B, T, M]")
    if g0.ndim == 2:
        g0 = g0[..., None]
        g1 = None if g1 is None else g1[..., None]
    if g0.shape[:2] != (B, T) or g0.ndim != 3 or M % g0.shape[-1]:
        raise ValueError("gates must be [B, T, G] with G dividing M")
    if cplx and (g1 is None or g1.shape != g0.shape):
        raise ValueError("complex scans need two gate tensors of the same shape")
    if transition == "p1":
        if nu_log is None or theta_log is None or nu_log.shape != (M,) or theta_log.shape != (M,):
            raise ValueError("P1 scans need nu_log and theta_log of shape [M]")
        g0, g1 = g0.float(), g1.float()
        nu_log, theta_log = nu_log.float(), theta_log.float()
    else:
        g0, g1 = _gate_dtype(g0, g1, w_re.dtype)
        nu_log = theta_log = None
    h0_re = h0_im = None
    if initial_state is not None:
        if cplx:
            h0_re, h0_im = initial_state
            if h0_re.shape != (B, M) or h0_im.shape != (B, M):
                raise ValueError("initial SPARC states must have shape [B,M]")
            h0_re, h0_im = h0_re.float(), h0_im.float()
        else:
            h0_re = initial_state.float()
            if h0_re.shape != (B, M):
                raise ValueError("initial state must have shape [B,M]")
    if segment_pos is not None:
        if segment_pos.shape != (B, T):
            raise ValueError("segment_pos must have shape [B,L]")
        segment_pos = segment_pos.to(torch.int32)
    y_re, y_im, last_re, last_im = _ChunkScan.apply(
        transition, bool(relu_output), bool(reset_first), _c(g0), _c(g1), _c(nu_log), _c(theta_log),
        _c(w_re), _c(w_im), _c(h0_re), _c(h0_im), _c(segment_pos))
    if not cplx:
        return y_re, last_re
    if relu_output:
        return y_re, (last_re, last_im)
    return (y_re, y_im), (last_re, last_im)


# ---------------------------------------------------------------------------
# reference-named operators (sparc-kernal/backward/scan.py:1643-1877)
# ---------------------------------------------------------------------------
def _check_sparc_shapes(eta, delta, br, bi):
    if eta.shape != delta.shape or eta.ndim != 2:
        raise ValueError("SPARC controls must be matching [B, L] tensors")
    if br.shape != bi.shape or br.ndim != 3:
        raise ValueError("SPARC writes must be matching [B, L, M] tensors")
    if eta.shape != br.shape[:2]:
        raise ValueError("SPARC control, spectrum and write shapes disagree")


def sparc_scan(eta, delta, nu_log, theta_log, br, bi):
    """``sparc_scan`` (backward/scan.py:1658-1661, _SPARCScan :922-968)."""
    _check_sparc_shapes(eta, delta, br, bi)
    if nu_log.shape != (br.shape[2],) or theta_log.shape != (br.shape[2],):
        raise ValueError("SPARC control, spectrum and write shapes disagree")
    (out_r, out_i), _ = chunk_scan("p1", eta, delta, br, bi, nu_log, theta_log)
    return out_r, out_i


@torch.no_grad()
def sparc_scan_with_last(eta, delta, nu_log, theta_log, br, bi):
    """``sparc_scan_with_last`` (backward/scan.py:1857-1877), no gradient like
    the reference."""
    if eta.shape != delta.shape or br.shape != bi.shape:
        raise ValueError("SPARC control or write shapes disagree")
    (out_r, out_i), (last_r, last_i) = chunk_scan("p1", eta, delta, br, bi, nu_log, theta_log)
    return out_r, out_i, last_r, last_i


def sparc_tiled_serial_scan(eta, delta, nu_log, theta_log, br, bi, *, segment_pos=None,
                            initial_state=None, block_size: int = 128, reset_first: bool = False):
    """``sparc_tiled_serial_scan`` (backward/scan.py:1664-1687,
    _SPARCTiledSerialScan :971-1070): h0, segment resets, reset_first,
    gradients of the last state and of h0."""
    if eta.shape != delta.shape or eta.ndim != 2:
        raise ValueError("SPARC controls must be matching [B,L] tensors")
    if br.shape != bi.shape or br.ndim != 3:
        raise ValueError("SPARC writes must be matching [B,L,M] tensors")
    if eta.shape != br.shape[:2]:
        raise ValueError("SPARC controls and writes disagree")
    if nu_log.shape != (br.shape[2],) or theta_log.shape != (br.shape[2],):
        raise ValueError("SPARC static spectrum has the wrong shape")
    if block_size not in (32, 64, 128, 256):
        raise ValueError("block_size must be 32, 64, 128 or 256")
    (out_r, out_i), (last_r, last_i) = chunk_scan(
        "p1", eta, delta, br, bi, nu_log, theta_log, initial_state=initial_state,
        segment_pos=segment_pos, reset_first=reset_first)
    return out_r, out_i, last_r, last_i


def sparc_chunk_scan(eta, delta, nu_log, theta_log, br, bi, chunk_size: int = 32,
                     hierarchical_prefix: bool = False, precompute_shared: bool = False,
                     compressed_transition: bool = False, atomic_shared: bool = False,
                     two_stage_spectral: bool = False, compact_control_cache: bool = False,
                     precompute_spectral: bool = False, mode_block_size: int = 128,
                     raw_x=None, fused_write: bool = False, backward_chunk_group: int = 1,
                     fused_output_relu: bool = False, prefix_group_size: int = 0,
                     controller_backward_cache=None):
    """``sparc_chunk_scan`` (backward/scan.py:1703-1751, _SPARCChunkScan
    :1124-1640).  Returns (out_r, out_i), or relu(cat) [B,L,2M] with
    ``fused_output_relu``."""
    if fused_write or controller_backward_cache is not None:
        raise NotImplementedError(
            "the P2 fused write / fused controller paths (unreachable from SPARCMixer) "
            "are not part of this build")
    if eta.shape != delta.shape:
        raise ValueError("SPARC control or write shapes disagree")
    batch, length = eta.shape
    modes = nu_log.numel()
    if br.shape != (batch, length, modes) or bi.shape != br.shape:
        raise ValueError("SPARC control or write shapes disagree")
    if chunk_size not in (16, 32, 64) or length % chunk_size:
        raise ValueError("chunk size must be 16, 32 or 64 and divide length")
    chunks = length // chunk_size
    if mode_block_size not in (32, 64, 128, 256):
        raise ValueError("mode block size must be 32, 64, 128 or 256")
    if backward_chunk_group not in (1, 2):
        raise ValueError("backward chunk group must be 1 or 2")
    if chunks % backward_chunk_group:
        raise ValueError("backward chunk group must divide the chunk count")
    if backward_chunk_group > 1 and two_stage_spectral:
        raise ValueError("grouped replay and two-stage spectral are exclusive")
    if backward_chunk_group > 1 and fused_output_relu:
        raise ValueError("grouped replay and fused output are exclusive")
    if abs(prefix_group_size) not in (0, 32, 64, 128):
        raise ValueError("prefix group size must be 0, 32, 64 or 128")
    if prefix_group_size and not hierarchical_prefix:
        raise ValueError("a grouped prefix requires hierarchical_prefix")
    y, _ = chunk_scan("p1", eta, delta, br, bi, nu_log, theta_log,
                      relu_output=fused_output_relu)
    return y


def sparc_training_scan_dispatch(eta, delta, nu_log, theta_log, br, bi, *, chunk_size: int = 16,
                                 hierarchical_prefix: bool = False, precompute_shared: bool = False,
                                 compressed_transition: bool = False, atomic_shared: bool = False,
                                 two_stage_spectral: bool = False, compact_control_cache: bool = False,
                                 precompute_spectral: bool = False, raw_x=None, fused_write: bool = False,
                                 backward_chunk_group: int = 1, fused_output_relu: bool = False,
                                 prefix_group_size: int = 0, controller_backward_cache=None,
                                 segment_pos=None, initial_state=None, reset_first: bool = False,
                                 block_size: int = 128):
    """``sparc_training_scan_dispatch`` (backward/scan.py:1754-1818): resets,
    h0 or a partial last chunk take the tiled-serial semantics, otherwise the
    chunk scan; both are the same HIP scan here."""
    if fused_write and raw_x is None:
        raise ValueError("raw_x is required by the fused-write SPARC path")
    fallback = segment_pos is not None or initial_state is not None or eta.shape[1] % chunk_size != 0
    if fallback:
        if controller_backward_cache is not None:
            raise ValueError("fused controller backward does not support fallback semantics")
        if fused_write:
            raise NotImplementedError("the P2 fused write is not part of this build")
        out_r, out_i, _, _ = sparc_tiled_serial_scan(
            eta, delta, nu_log, theta_log, br, bi, segment_pos=segment_pos,
            initial_state=initial_state, block_size=block_size, reset_first=reset_first)
        if fused_output_relu:
            return torch.cat((out_r, out_i), dim=-1).relu()
        return out_r, out_i
    return sparc_chunk_scan(
        eta, delta, nu_log, theta_log, br, bi, chunk_size, hierarchical_prefix,
        precompute_shared, compressed_transition, atomic_shared, two_stage_spectral,
        compact_control_cache, precompute_spectral, mode_block_size=block_size,
        raw_x=raw_x, fused_write=fused_write, backward_chunk_group=backward_chunk_group,
        fused_output_relu=fused_output_relu, prefix_group_size=prefix_group_size,
        controller_backward_cache=controller_backward_cache)


def complex_scan(ar, ai, br, bi):
    """``complex_scan`` (backward/scan.py:1653-1655, _ComplexScan :887-919):
    per-element complex transition."""
    shape = ar.shape
    if any(t.shape != shape for t in (ai, br, bi)) or ar.ndim != 3:
        raise ValueError("complex scan expects matching [B, L, M] tensors")
    (out_r, out_i), _ = chunk_scan("cartesian", ar, ai, br, bi)
    return out_r, out_i


@torch.no_grad()
def complex_scan_with_last(ar, ai, br, bi):
    """``complex_scan_with_last`` (backward/scan.py:1839-1854), no gradient."""
    shape = ar.shape
    if any(t.shape != shape for t in (ai, br, bi)) or ar.ndim != 3:
        raise ValueError("complex scan expects matching [B, L, M] tensors")
    (out_r, out_i), (last_r, last_i) = chunk_scan("cartesian", ar, ai, br, bi)
    return out_r, out_i, last_r, last_i


def real_scan(a, b):
    """``real_scan`` (backward/scan.py:1643-1644, _RealScan :793-822)."""
    if a.shape != b.shape or a.ndim != 3:
        raise ValueError("real scan expects matching [B, L, D] tensors")
    out, _ = chunk_scan("real", a, None, b)
    return out


def real_chunk_scan(a, b, chunk_size: int = 16):
    """``real_chunk_scan`` (backward/scan.py:1647-1650, _RealChunkScan :825-884)."""
    if a.shape != b.shape or a.ndim != 3:
        raise ValueError("real chunk scan expects matching [B, L, D] tensors")
    if chunk_size not in (16, 32, 64) or a.shape[1] % chunk_size:
        raise ValueError("chunk size must be 16, 32 or 64 and divide length")
    out, _ = chunk_scan("real", a, None, b)
    return out


@torch.no_grad()
def real_scan_with_last(a, b):
    """``real_scan_with_last`` (backward/scan.py:1821-1836), no gradient."""
    if a.shape != b.shape or a.ndim != 3:
        raise ValueError("real scan expects matching [B, L, D] tensors")
    return chunk_scan("real", a, None, b)


# grouped forms used by the benchmark shapes -------------------------------
def polar_chunk_scan(r, phi, w_re, w_im, initial_state=None):
    """Complex scan with a = r*exp(i*phi), gates [B,T,G] shared by M/G modes."""
    return chunk_scan("polar", r, phi, w_re, w_im, initial_state=initial_state)


def grouped_real_scan(a, b, initial_state=None):
    """Real scan h = a*h + b with a [B,T,G] shared by W/G channels."""
    return chunk_scan("real", a, None, b, initial_state=initial_state)
