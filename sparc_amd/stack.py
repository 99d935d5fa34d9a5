"""A stack of SPARC blocks: the model of the 12-layer training configuration.

Each block is pre-norm and residual:

    x <- x + out_proj(SPARCMixer(in_proj(rms_norm(x))))

with ``in_proj`` d_model -> 2M and ``out_proj`` 2M -> d_model (M = d_model *
N complex modes, so the mixer's width is 2M), and a final RMSNorm.  The
projections are plain GEMMs (torch -> hipBLASLt on MI355X); the mixer is the
fused HIP sequence path, with its two control dot products folded into the
input projection (``fuse_projection``).  The reference ships the layer, not a network
(sparc-kernal/sparc.py:58-128); this stack is the configuration the layer is
benchmarked in.
"""
from __future__ import annotations

import os

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib
from . import mixer as _mixer
from .control import aligned16
from .sparc import SPARCMixer

# Fold the controls into the input projection (see mixer._ProjectedMixer);
# False runs the projection and the module separately.
fuse_projection = True
# RMSNorm through sparc_rms_norm_forward / _backward where the shape allows
# (rms_norm below); False keeps torch's RMSNorm.
fused_norm = True


class _RMSNorm(torch.autograd.Function):
    """y = x / sqrt(mean(x^2) + eps) * weight over the last dimension
    (torch.nn.RMSNorm's formula) through the library's RMSNorm kernels; the
    backward's weight gradient is a fixed-order sum over rows."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        lib = _lib.load()
        dev = _lib.require_gpu(x, weight)
        D = x.shape[-1]
        x2 = aligned16(x.detach().reshape(-1, D))
        w = aligned16(weight.detach())
        y = torch.empty_like(x2)
        rstd = torch.empty(x2.shape[0], dtype=torch.float32, device=dev)
        P = _lib.ptr
        _lib.check(lib.sparc_rms_norm_forward(x2.shape[0], D, _lib.io_code(x.dtype), P(x2), P(w), float(eps), P(y),
                                              P(rstd), _lib.stream_of(dev)), "sparc_rms_norm_forward")
        ctx.save_for_backward(x2, w, rstd)
        ctx.wdtype = weight.dtype
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, w, rstd = ctx.saved_tensors
        lib = _lib.load()
        dev = x2.device
        rows, D = x2.shape
        dy2 = aligned16(dy.to(x2.dtype).reshape(rows, D))
        dx = torch.empty_like(x2)
        dw = torch.empty(D, dtype=torch.float32, device=dev)
        ws = torch.empty(lib.sparc_rms_norm_workspace_bytes(rows, D), dtype=torch.uint8, device=dev)
        P = _lib.ptr
        _lib.check(lib.sparc_rms_norm_backward(rows, D, _lib.io_code(x2.dtype), P(x2), P(w), P(rstd), P(dy2), P(dx),
                                               P(dw), P(ws), ws.numel(), _lib.stream_of(dev)),
                   "sparc_rms_norm_backward")
        return dx.view(dy.shape), dw.to(ctx.wdtype), None


def rms_norm(norm: nn.RMSNorm, x: torch.Tensor) -> torch.Tensor:
    """``norm(x)`` through the library's RMSNorm kernels when ``fused_norm``
    is set and the shape allows (GPU tensors, float32 or bfloat16 with the
    weight in the same dtype, a last dimension that is a multiple of 8 up to
    4096), else torch's."""
    D = x.shape[-1]
    w = norm.weight
    if (fused_norm and x.is_cuda and x.dtype in (torch.float32, torch.bfloat16) and w is not None
            and w.dtype == x.dtype and D % 8 == 0 and D <= 4096 and x.numel() > 0):
        eps = norm.eps if norm.eps is not None else torch.finfo(x.dtype).eps
        return _RMSNorm.apply(x, w, eps)
    return norm(x)


class SPARCBlock(nn.Module):
    def __init__(self, d_model: int, n_states: int, eps: float = 1e-6):
        super().__init__()
        modes = d_model * n_states
        self.norm = nn.RMSNorm(d_model, eps=eps)
        self.in_proj = nn.Linear(d_model, 2 * modes, bias=False)
        self.mixer = SPARCMixer(2 * modes)
        self.out_proj = nn.Linear(2 * modes, d_model, bias=False)
        with torch.no_grad():  # keep the residual stream's scale at init
            self.out_proj.weight.mul_(1.0 / (2 * modes) ** 0.5)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xn = rms_norm(self.norm, x)
        if fuse_projection and _mixer.get_mixer_path() != "composed" and \
                _mixer.projected_fused_supported(xn, self.in_proj.weight):
            y, _ = _mixer.projected_sequence(self.mixer, xn, self.in_proj.weight)
        else:
            y, _ = self.mixer(self.in_proj(xn))
        return x + self.out_proj(y)


class SPARCStack(nn.Module):
    """``n_layers`` SPARC blocks on a [B, T, d_model] stream."""

    def __init__(self, n_layers: int, d_model: int, n_states: int, eps: float = 1e-6):
        super().__init__()
        self.blocks = nn.ModuleList(SPARCBlock(d_model, n_states, eps) for _ in range(n_layers))
        self.norm = nn.RMSNorm(d_model, eps=eps)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for blk in self.blocks:
            x = blk(x)
        return rms_norm(self.norm, x)


GEMM_TUNING_FILE = os.path.join(os.path.dirname(__file__), "tuning", "gemm_stack_gfx950.csv")


def use_tuned_gemms(path: str = GEMM_TUNING_FILE) -> bool:
    """Route torch's GEMMs through TunableOp with the solutions recorded in
    ``path`` (by default the stack's shapes measured on MI355X, written by
    ``python -m sparc_amd.tuning.tune_stack_gemms``).  Tuning stays off:
    shapes missing from the file keep torch's default solution, and nothing
    is written back.  Returns whether the file was accepted (its validator
    lines must match this torch, HIP, hipBLASLt, rocBLAS and GPU).  The
    setting is process-wide; ``use_default_gemms()`` undoes it."""
    import torch.cuda.tunable as tn
    tn.enable(True)
    tn.tuning_enable(False)
    tn.set_filename(path)
    return bool(tn.read_file(path))


def use_default_gemms() -> None:
    """Switch TunableOp off again (torch's default GEMM solutions)."""
    import torch.cuda.tunable as tn
    tn.enable(False)


def rms_norm_reference(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm as torch.nn.RMSNorm computes it (for references in other dtypes)."""
    return F.rms_norm(x, (x.shape[-1],), weight, eps)


__all__ = ["SPARCBlock", "SPARCStack", "rms_norm", "rms_norm_reference", "use_tuned_gemms", "use_default_gemms",
           "GEMM_TUNING_FILE"]
