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

from . import mixer as _mixer
from .sparc import SPARCMixer

# Fold the controls into the input projection (see mixer._ProjectedMixer);
# False runs the projection and the module separately.
fuse_projection = True


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
        xn = self.norm(x)
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
        return self.norm(x)


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


__all__ = ["SPARCBlock", "SPARCStack", "rms_norm_reference", "use_tuned_gemms", "use_default_gemms",
           "GEMM_TUNING_FILE"]
