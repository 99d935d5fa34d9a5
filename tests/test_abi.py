"""CPU checks of the C ABI and the host logic: the library loads, exports
every symbol include/sparc_hip.h declares, validates descriptors on the host
(no GPU call is made for an invalid request), and the Python operators raise
the reference's ValueErrors.  No compute call is made here."""
import ctypes
import os
import re

import pytest
import torch

import sparc_amd
from sparc_amd import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "sparc_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sparc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = header_symbols()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(_lib.EXPORTED_SYMBOLS) == declared
    assert lib.sparc_version().startswith(b"sparc_hip")


def _desc(**kw):
    base = dict(batch=2, length=100, modes=256, groups=16, transition=1, io_dtype=1,
                gate_dtype=1, flags=0)
    base.update(kw)
    return _lib.ScanDesc(**base)


def test_workspace_and_chunk_queries():
    lib = _lib.load()
    d = _desc()
    assert lib.sparc_scan_chunk_length(ctypes.byref(d)) == 64
    assert lib.sparc_scan_chunk_count(ctypes.byref(d)) == 2
    assert lib.sparc_scan_workspace_bytes(ctypes.byref(d), 0) > 0
    assert lib.sparc_scan_workspace_bytes(ctypes.byref(d), 1) >= lib.sparc_scan_workspace_bytes(ctypes.byref(d), 0)
    # cfg2 shape: 8 x 4096 x 16384 modes, 1024 gate groups
    big = _desc(batch=8, length=4096, modes=16384, groups=1024)
    assert lib.sparc_scan_chunk_count(ctypes.byref(big)) == 64
    assert 0 < lib.sparc_scan_workspace_bytes(ctypes.byref(big), 1) < 1 << 30


@pytest.mark.parametrize("kw,msg", [
    (dict(groups=3), b"groups must divide"),
    (dict(transition=7), b"unknown transition"),
    (dict(io_dtype=5), b"io_dtype"),
    (dict(transition=0, gate_dtype=1), b"P1 gates"),
    (dict(io_dtype=0, gate_dtype=1), b"bf16 gates need bf16 I/O"),
    (dict(gate_dtype=3), b"unknown gate_dtype"),
    (dict(transition=3, flags=1), b"RELU_OUTPUT"),
    (dict(batch=0), b"must be > 0"),
    (dict(groups=256 // 3 * 0 + 64, modes=192), b"unsupported gate group"),
])
def test_invalid_descriptors_rejected_on_host(kw, msg):
    lib = _lib.load()
    d = _desc(**kw)
    assert lib.sparc_scan_workspace_bytes(ctypes.byref(d), 0) == 0
    st = lib.sparc_scan_forward(ctypes.byref(d), *([None] * 13), 0, None)
    assert st == 1
    assert msg in lib.sparc_last_error()


@pytest.mark.parametrize("transition,groups", [(1, 16), (2, 256), (3, 256), (3, 16)])
def test_fp32_gates_with_bf16_io_plan(transition, groups):
    """fp32 gates beside bf16 writes (the reference's generic scans upcast
    `a` from its own dtype) are a valid plan for the polar, cartesian and real
    transitions, per-element or grouped."""
    lib = _lib.load()
    d = _desc(transition=transition, groups=groups, io_dtype=1, gate_dtype=0)
    assert lib.sparc_scan_workspace_bytes(ctypes.byref(d), 0) > 0
    assert lib.sparc_scan_workspace_bytes(ctypes.byref(d), 1) > 0


def test_forward_requires_workspace():
    lib = _lib.load()
    d = _desc()
    st = lib.sparc_scan_forward(ctypes.byref(d), *([None] * 12), None, 0, None)
    assert st == 4 and b"workspace" in lib.sparc_last_error()


def test_reference_value_errors():
    eta = torch.zeros(2, 48)
    nu = torch.zeros(8)
    br = torch.zeros(2, 48, 8)
    with pytest.raises(ValueError, match="chunk size must be 16, 32 or 64"):
        ops.sparc_chunk_scan(eta, eta, nu, nu, br, br, chunk_size=40)
    with pytest.raises(ValueError, match="chunk size must be 16, 32 or 64"):
        ops.sparc_chunk_scan(eta, eta, nu, nu, br, br, chunk_size=32)  # 48 % 32
    with pytest.raises(ValueError, match="mode block size"):
        ops.sparc_chunk_scan(eta, eta, nu, nu, br, br, chunk_size=16, mode_block_size=100)
    with pytest.raises(ValueError, match="backward chunk group must divide"):
        ops.sparc_chunk_scan(eta, eta, nu, nu, br, br, chunk_size=16, backward_chunk_group=2)
    eta64, br64 = torch.zeros(2, 64), torch.zeros(2, 64, 8)
    with pytest.raises(ValueError, match="grouped replay and fused output"):
        ops.sparc_chunk_scan(eta64, eta64, nu, nu, br64, br64, chunk_size=16,
                             backward_chunk_group=2, fused_output_relu=True)
    with pytest.raises(ValueError, match="real chunk scan expects"):
        ops.real_chunk_scan(torch.zeros(2, 4, 3), torch.zeros(2, 4, 2))
    with pytest.raises(ValueError, match="complex scan expects"):
        ops.complex_scan(br, br, br, torch.zeros(2, 48, 4))
    with pytest.raises(ValueError, match="block_size must be"):
        ops.sparc_tiled_serial_scan(eta, eta, nu, nu, br, br, block_size=48)
    with pytest.raises(ValueError, match="SPARC controls must be matching"):
        ops.sparc_scan(eta, torch.zeros(2, 47), nu, nu, br, br)


def test_module_surface_and_knobs():
    m = sparc_amd.SPARCMixer(16)
    names = {n for n, _ in m.named_parameters()}
    assert names == {"nu_log", "theta_log", "phase_direction", "radial_direction",
                     "write_log_gain", "energy_response", "write_phase_response",
                     "write_radial_response"}
    assert {n for n, _ in m.named_buffers()} == {"phase_amplitude", "radial_amplitude"}
    with pytest.raises(ValueError):
        sparc_amd.SPARCMixer(15)
    with pytest.raises(ValueError):
        m.set_tiled_training_block_size(100)
    with pytest.raises(ValueError):
        m.set_decode_backend("nope")
    with pytest.raises(ValueError):
        m.set_controller_projection_dtype("fp64")
    m.set_scan_backend("bogus")
    with pytest.raises(ValueError, match="unknown scan backend"):
        m(torch.zeros(1, 4, 16))
    for ok in ("auto", "chunk16", "fused_output_shared_sfu_chunk32", "framework_eager",
               "associative_fp32", "tiled_serial", "affine_tile_s16_m64_w4"):
        sparc_amd.sparc._validate_backend(ok)


def test_cpu_tensors_fail_loudly():
    """No CPU fallback: the HIP operators refuse host tensors."""
    eta = torch.zeros(1, 16)
    nu = torch.zeros(4)
    br = torch.zeros(1, 16, 4)
    with pytest.raises(RuntimeError, match="need GPU tensors"):
        ops.sparc_scan(eta, eta, nu, nu, br, br)


def test_controls_entry_points_validate_on_host():
    """sparc_controls_*: width must be a positive multiple of 8, pointers
    non-NULL, the workspace large enough; the workspace holds one row of
    partial direction gradients per row block (at most 65535 row blocks)."""
    lib = _lib.load()
    assert lib.sparc_controls_workspace_bytes(10, 12) == 0
    assert lib.sparc_controls_workspace_bytes(-1, 8) == 0
    up = lambda n: (n + 255) // 256 * 256
    # 1000 rows of width 8: 16-row blocks -> 63 blocks
    assert lib.sparc_controls_workspace_bytes(1000, 8) == up(2 * 63 * 8 * 4) + up(2 * 63 * 4)
    # 10M rows: 128-row blocks, capped at 65535 (the workgroups loop over the rest)
    assert lib.sparc_controls_workspace_bytes(10_000_000, 8) == up(2 * 65535 * 8 * 4) + up(2 * 65535 * 4)
    assert lib.sparc_controls_forward(4, 12, 0, *([None] * 5), None) == 1
    assert b"multiple of 8" in lib.sparc_last_error()
    assert lib.sparc_controls_forward(4, 16, 0, *([None] * 5), None) == 1
    assert b"NULL" in lib.sparc_last_error()
    assert lib.sparc_controls_forward(4, 16, 7, *([None] * 5), None) == 1
    assert b"io_dtype" in lib.sparc_last_error()
    fake = ctypes.c_void_p(256)  # never dereferenced: the size check fails first
    st = lib.sparc_controls_backward(4, 16, 0, *([fake] * 10), fake, 0, None)
    assert st == 4 and b"workspace" in lib.sparc_last_error()


def test_rms_norm_entry_points_validate_on_host():
    """sparc_rms_norm_*: cols a positive multiple of 8 up to 4096, a known
    I/O type, non-NULL pointers, a large enough workspace (one fp32 partial
    row of dweight per 128 rows at these widths)."""
    lib = _lib.load()
    assert lib.sparc_rms_norm_workspace_bytes(-1, 768) == 0
    assert lib.sparc_rms_norm_workspace_bytes(10, 12) == 0
    assert lib.sparc_rms_norm_workspace_bytes(1000, 768) == 8 * 768 * 4 + 256
    eps = ctypes.c_float(1e-6)
    assert lib.sparc_rms_norm_forward(4, 12, 0, None, None, eps, None, None, None) == 1
    assert b"multiple of 8" in lib.sparc_last_error()
    assert lib.sparc_rms_norm_forward(4, 8192, 0, None, None, eps, None, None, None) == 1
    assert lib.sparc_rms_norm_forward(4, 16, 7, None, None, eps, None, None, None) == 1
    assert b"io_dtype" in lib.sparc_last_error()
    assert lib.sparc_rms_norm_forward(4, 16, 0, None, None, eps, None, None, None) == 1
    assert b"NULL" in lib.sparc_last_error()
    fake = ctypes.c_void_p(256)  # never dereferenced: the size check fails first
    st = lib.sparc_rms_norm_backward(4, 16, 0, *([fake] * 7), 0, None)
    assert st == 4 and b"workspace" in lib.sparc_last_error()


def test_controls_fold_entry_points_validate_on_host():
    """sparc_controls_fold*: width > 0, dim a positive multiple of 8 up to
    4096, a known I/O type, non-NULL pointers, a large enough workspace (two
    fp32 partial rows per 64 rows of W)."""
    lib = _lib.load()
    assert lib.sparc_controls_fold_workspace_bytes(0, 768) == 0
    assert lib.sparc_controls_fold_workspace_bytes(64, 12) == 0
    assert lib.sparc_controls_fold_workspace_bytes(64, 8192) == 0
    assert lib.sparc_controls_fold_workspace_bytes(24576, 768) == 2 * 384 * 768 * 4 + 256
    assert lib.sparc_controls_fold_workspace_bytes(65, 8) == 2 * 2 * 8 * 4 + 256
    assert lib.sparc_controls_fold(64, 12, 0, *([None] * 6), 0, None) == 1
    assert b"multiple of 8" in lib.sparc_last_error()
    assert lib.sparc_controls_fold(64, 16, 7, *([None] * 6), 0, None) == 1
    assert b"io_dtype" in lib.sparc_last_error()
    assert lib.sparc_controls_fold(64, 16, 0, *([None] * 6), 0, None) == 1
    assert b"NULL" in lib.sparc_last_error()
    fake = ctypes.c_void_p(256)  # never dereferenced: the size check fails first
    assert lib.sparc_controls_fold(64, 16, 0, *([fake] * 6), 16, None) == 4
    assert b"workspace" in lib.sparc_last_error()
    assert lib.sparc_controls_fold_backward(0, 16, 0, *([fake] * 8), None) == 1
    assert lib.sparc_controls_fold_backward(64, 16, 0, None, *([fake] * 7), None) == 1
    assert b"NULL" in lib.sparc_last_error()
    # dweight needs the directions
    assert lib.sparc_controls_fold_backward(64, 16, 0, fake, None, None, *([fake] * 5), None) == 1
    assert b"NULL" in lib.sparc_last_error()
    assert lib.sparc_controls_fold_backward(64, 16, 0, ctypes.c_void_p(258), *([fake] * 7), None) == 1
    assert b"aligned" in lib.sparc_last_error()
    assert lib.sparc_controls_fold_backward(64, 16, 0, fake, *([fake] * 6), ctypes.c_void_p(264), None) == 1
    assert b"aligned" in lib.sparc_last_error()


def _raw_inputs(transition="p1", B=2, T=5, M=8, G=2, io=torch.float32):
    g = torch.float32 if transition == "p1" else io
    d = dict(g0=torch.zeros(B, T, G, dtype=g), g1=torch.zeros(B, T, G, dtype=g),
             w_re=torch.zeros(B, T, M, dtype=io), w_im=torch.zeros(B, T, M, dtype=io),
             nu_log=torch.zeros(M), theta_log=torch.zeros(M))
    if transition == "real":
        d.update(g1=None, w_im=None, nu_log=None, theta_log=None)
    elif transition != "p1":
        d.update(nu_log=None, theta_log=None)
    return d


@pytest.mark.parametrize("change,msg", [
    (dict(nu_log=torch.zeros(7)), "nu_log"),                          # shorter than M
    (dict(theta_log=torch.zeros(8, dtype=torch.float64)), "theta_log"),
    (dict(w_im=torch.zeros(2, 5, 4)), "w_im"),
    (dict(g1=torch.zeros(2, 4, 2)), "g1"),
    (dict(g0=torch.zeros(2, 5, 3)), "divide"),
    (dict(h0_re=torch.zeros(2, 8)), "h0_im"),                         # complex h0 needs both halves
    (dict(segment_pos=torch.ones(2, 5, dtype=torch.int64)), "segment_pos"),
])
def test_raw_scan_rejects_mismatched_tensors(change, msg):
    """The raw launch wrappers check every tensor against the descriptor
    before any pointer reaches the C ABI (on any device)."""
    kw = _raw_inputs()
    kw.update(change)
    with pytest.raises(ValueError, match=msg):
        ops.scan_forward_raw("p1", **kw)


def test_raw_backward_and_step_reject_mismatched_tensors():
    kw = _raw_inputs("polar", io=torch.bfloat16)
    cs = torch.zeros(2, 1, 8, 2)
    dy = torch.zeros(2, 5, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="chunk_state"):
        ops.scan_backward_raw("polar", kw["g0"], kw["g1"], kw["w_re"], kw["w_im"], cs[:, :, :4], dy, dy)
    with pytest.raises(ValueError, match="dy_re"):
        ops.scan_backward_raw("polar", kw["g0"], kw["g1"], kw["w_re"], kw["w_im"], cs, dy, dy, relu_output=True)
    with pytest.raises(ValueError, match="g1"):   # the two gates in one dtype
        ops.scan_forward_raw("polar", **{**kw, "g0": kw["g0"].float()})
    kw32 = _raw_inputs("polar", io=torch.float32)
    with pytest.raises(ValueError, match="writes' dtype"):   # bf16 gates need bf16 writes
        ops.scan_forward_raw("polar", **{**kw32, "g0": kw32["g0"].bfloat16(), "g1": kw32["g1"].bfloat16()})
    state = (torch.zeros(2, 8), torch.zeros(2, 8))
    with pytest.raises(ValueError, match="nu_log"):
        ops.scan_step("p1", torch.zeros(2, 1), torch.zeros(2, 1), torch.zeros(2, 8), torch.zeros(2, 8),
                      state, torch.zeros(4), torch.zeros(8))
    with pytest.raises(ValueError, match="w_im"):
        ops.scan_step("polar", torch.zeros(2, 1), torch.zeros(2, 1), torch.zeros(2, 8), torch.zeros(2, 6),
                      state)


def test_pointer_helper_refuses_non_contiguous():
    t = torch.zeros(4, 6)
    assert _lib.ptr(t) == t.data_ptr() and _lib.ptr(None) is None
    with pytest.raises(ValueError, match="contiguous"):
        _lib.ptr(t.t())


def test_module_paths_reject_wrong_parameter_shapes():
    """Controls, write, fused and projected mixer and decode check every
    parameter's length against the input width before any launch."""
    from sparc_amd import control, mixer
    from sparc_amd.decode import latest_sparc_decode
    m = sparc_amd.SPARCMixer(16)  # M = 8
    x = torch.zeros(2, 3, 16)
    good = [getattr(m, n).detach() for n in ("phase_direction", "radial_direction", "nu_log", "theta_log",
                                             "write_log_gain", "write_phase_response",
                                             "write_radial_response")]
    with pytest.raises(ValueError, match="phase_direction"):
        control._Controls.apply(x, torch.zeros(16), good[1])
    with pytest.raises(ValueError, match="nu_log"):
        control._LatestSPARCWrite.apply(x, torch.zeros(2, 3), torch.zeros(2, 3), torch.zeros(7), *good[4:])
    with pytest.raises(ValueError, match="theta_log"):
        mixer._FusedMixer.apply(x, good[0], good[1], good[2], torch.zeros(9), *good[4:], m.energy_response)
    with pytest.raises(ValueError, match="radial_direction"):
        mixer._ProjectedMixer.apply(torch.zeros(2, 3, 4), torch.zeros(16, 4), good[0], torch.zeros(4),
                                    *good[2:], m.energy_response)
    with pytest.raises(ValueError, match="projection"):
        mixer._ProjectedMixer.apply(torch.zeros(2, 3, 4), torch.zeros(16, 5), *good, m.energy_response)
    with torch.no_grad():
        m.write_log_gain = torch.nn.Parameter(torch.zeros(6))
    with pytest.raises(ValueError, match="write_log_gain"):
        latest_sparc_decode(m, torch.zeros(2, 16), (torch.zeros(2, 8), torch.zeros(2, 8)))
