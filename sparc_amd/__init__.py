"""sparc_amd: MI355X-native (gfx950) SPARC chunked diagonal linear scan.

Drop-in for the reference's ``sparc`` module surface on the scan path
(sparc-kernal/sparc.py): ``SPARCMixer`` and the scan operators, dispatching
to hand-written HIP kernels through the C ABI in include/sparc_hip.h.
"""
from .control import latest_sparc_write, make_controls, make_scan_inputs
from .decode import latest_sparc_decode, prepare_decode, run_decode_step
from .ops import (
    chunk_scan,
    complex_scan,
    complex_scan_with_last,
    grouped_real_scan,
    polar_chunk_scan,
    real_chunk_scan,
    real_scan,
    real_scan_with_last,
    scan_step,
    sparc_chunk_scan,
    sparc_scan,
    sparc_scan_with_last,
    sparc_tiled_serial_scan,
    sparc_training_scan_dispatch,
)
from .mixer import backward_form, get_mixer_path, set_backward_plan, set_mixer_path
from .sparc import SPARCMixer, run_sequence

__all__ = [
    "SPARCMixer", "run_sequence", "make_controls", "make_scan_inputs", "latest_sparc_write",
    "prepare_decode", "run_decode_step", "latest_sparc_decode", "chunk_scan", "complex_scan",
    "complex_scan_with_last", "real_scan", "real_chunk_scan", "real_scan_with_last",
    "sparc_scan", "sparc_scan_with_last", "sparc_chunk_scan", "sparc_tiled_serial_scan",
    "sparc_training_scan_dispatch", "polar_chunk_scan", "grouped_real_scan", "scan_step",
    "set_mixer_path", "get_mixer_path", "set_backward_plan", "backward_form",
]
