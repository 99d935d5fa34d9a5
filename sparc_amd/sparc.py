"""Drop-in ``SPARCMixer`` (sparc-kernal/sparc.py:58-128) over the HIP kernels.

Constructor, parameters and buffers, ``forward(x, return_cache=False)``,
``step(x, state, segment_pos)``, ``prepare_inference()`` and the knob setters
keep the reference's signatures, defaults and ``ValueError``s.  The sequence
forward is ``run_sequence`` below (reference: sparc-kernal/forward/scan.py:
1398-1603): by default the fused HIP path (controls, write, P1 scan and
``relu(cat(h_re, h_im))`` epilogue in two C-ABI calls forward and backward,
``sparc_amd.mixer``; few chains over long sequences split time into
segments there).  ``set_mixer_path("composed")`` selects the composed path
instead (controls, HIP write prologue and HIP chunked P1 scan with the
epilogue fused into its store, as separate operators).
"""
from __future__ import annotations

import math

import torch
from torch import nn

from .control import latest_sparc_write, make_controls, make_scan_inputs
from .decode import prepare_decode, run_decode_step
from .mixer import fused_sequence, use_fused
from .ops import chunk_scan

_NAMED_BACKENDS = ("tiled_serial", "triton", "precomputed_decay", "framework_eager",
                   "associative_bf16", "associative_fp32")


def _validate_backend(backend: str) -> None:
    """Accepts every backend string the reference's ``run_sequence`` accepts
    (forward/scan.py:1407-1597) and raises its ``ValueError`` otherwise.  All
    of them compute the same P1 scan; here they select the same HIP kernels."""
    if backend == "auto" or backend in _NAMED_BACKENDS:
        return
    b = backend.replace("_fused_write", "").replace("compressed_", "")
    if b.startswith("affine_tile_s"):
        return
    if "chunk" in b and b.rsplit("chunk", 1)[1].isdigit():
        return
    raise ValueError(f"unknown scan backend: {backend}")


def run_sequence(module, x: torch.Tensor, return_cache: bool = False):
    """Sequence forward.  Returns (y, cache): y = relu(cat(h_re, h_im))
    [B, L, 2M] in x's dtype, cache = (last_re, last_im) fp32 [B, M] or None.

    Unlike the reference, the cache path keeps gradients through the scan
    (the reference computes it under ``torch.no_grad`` when M <= 512,
    backward/scan.py:1857)."""
    _validate_backend(module.scan_backend)
    if x.ndim != 3 or x.shape[-1] != module.width:
        raise ValueError(f"SPARCMixer expects [B, L, {module.width}] inputs")
    if use_fused(x, module.modes):
        y, last = fused_sequence(module, x)
        return y, (last if return_cache else None)
    eta, delta, write_r, write_i = make_scan_inputs(module, x)
    y, last = chunk_scan("p1", eta, delta, write_r, write_i, module.nu_log, module.theta_log,
                         relu_output=True)
    y = y.to(x.dtype)
    return y, (last if return_cache else None)


class SPARCMixer(nn.Module):
    def __init__(self, width: int):
        super().__init__()
        if width % 2:
            raise ValueError("SPARC rnn_width must be even")
        self.width = width
        self.modes = width // 2
        radius_squared = torch.rand(self.modes).clamp_min(torch.finfo(torch.float32).tiny)
        nu = -0.5 * torch.log(radius_squared)
        theta = (2.0 * math.pi * torch.rand(self.modes)).clamp_min(torch.finfo(torch.float32).tiny)
        self.nu_log = nn.Parameter(torch.log(nu))
        self.theta_log = nn.Parameter(torch.log(theta))
        self.phase_direction = nn.Parameter(torch.zeros(width + 1))
        self.radial_direction = nn.Parameter(torch.zeros(width + 1))
        self.register_buffer("phase_amplitude", torch.zeros(()))
        self.register_buffer("radial_amplitude", torch.zeros(()))
        initial_gain = torch.log(torch.sqrt(1.0 - torch.exp(-2.0 * nu)) + 1.0e-8)
        self.write_log_gain = nn.Parameter(initial_gain)
        self.energy_response = nn.Parameter(torch.full((self.modes,), 0.5493061443340548))
        self.write_phase_response = nn.Parameter(torch.zeros(self.modes))
        self.write_radial_response = nn.Parameter(torch.zeros(self.modes))
        self._inference_fused = False
        self._decode_backend = "auto"
        self._inference_pack = None
        self._tiled_training_block_size = 128
        self._controller_projection_dtype = "fp32_fused_coords"
        self.scan_backend = "auto"
        # not in the reference: write the decode state in place (step returns
        # the same state tensors it was given)
        self.decode_in_place = False

    def forward(self, x: torch.Tensor, return_cache: bool = False):
        return run_sequence(self, x, return_cache)

    def set_scan_backend(self, backend: str) -> None:
        self.scan_backend = backend

    def set_tiled_training_block_size(self, block_size: int) -> None:
        if block_size not in (32, 64, 128, 256):
            raise ValueError(block_size)
        self._tiled_training_block_size = block_size

    def set_controller_projection_dtype(self, dtype: str) -> None:
        if dtype not in (
            "fp32", "bf16", "triton_fp32",
            "fp32_rounded", "triton_fp32_rounded", "fp32_recompute",
            "fp32_triton_backward", "fp32_cache_save",
            "fp32_cache_recompute", "fp32_fused_coords",
        ):
            raise ValueError(dtype)
        self._controller_projection_dtype = dtype

    def prepare_inference(self) -> None:
        prepare_decode(self)

    def set_decode_backend(self, backend: str) -> None:
        if backend not in ("auto", "fused", "packed", "blocked16", "blocked32", "blocked64"):
            raise ValueError(backend)
        self._decode_backend = backend

    def step(self, x: torch.Tensor, state, segment_pos):
        return run_decode_step(self, x, state, segment_pos)


__all__ = ["SPARCMixer", "run_sequence", "make_controls", "make_scan_inputs",
           "latest_sparc_write"]
