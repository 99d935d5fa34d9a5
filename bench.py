#!/usr/bin/env python3
"""Benchmark of the SPARC chunked complex scan on one MI355X.

Metric: fwd+bwd tokens/s and fraction of the HBM roofline at
B=8, T=4096, D=1024, N=16 (M = D*N = 16384 complex modes, G = D = 1024 gate
groups of N modes), bf16 inputs/gates/gradients, fp32 state; plus the
single-step decode latency at B=256 (D=2048, N=16, width 2M = 65536).

One step = the forward scan and the backward scan of one batch, inputs
resident in HBM: the two C-ABI calls sparc_scan_forward / sparc_scan_backward
(one kernel each at this shape: the serial one-chain-per-workgroup kernels
with 4 modes per lane; the backward reads the states from the forward's saved
output).

Algorithmic bytes per step, B*T*(M*10*s + G*6*s_g) with s = s_g = 2:
  forward : read w (re, im), write y (re, im)      -> 8 B per mode-step
            read r, phi                            -> 4 B per group-step
  backward: read dy, read w, write dw (re, im)     -> 12 B per mode-step
            read r, phi, write dr, dphi            -> 8 B per group-step
The roofline object reports the dominant (backward) kernel: its algorithmic
bytes per launch over its average launch time, timed with HIP events on the
launch stream inside the timed region.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
# untimed passes before each secondary report's timed region (the headline
# takes --warmup): each allocates fresh buffers, and its first passes over
# them run a few percent slower than the ones after
SUB_WARMUP = 10
ROOT = os.path.dirname(os.path.abspath(__file__))
TRAFFIC_FILE = os.path.join("profiles", "scan_cfg2_hbm_traffic.md")
TRAFFIC_FILE_CFG3 = os.path.join("profiles", "scan_cfg3_hbm_traffic.md")
COUNTERS_FILE = os.path.join("profiles", "counters_bench_kernels.md")
# kernels each algorithm runs at this shape (backward, forward)
ALGO_KERNELS = {"auto": ("chain_bwd_serial_kernel", "chain_fwd_serial_kernel"),
                "serial": ("chain_bwd_serial_kernel", "chain_fwd_serial_kernel"),
                "chain": ("chain_bwd_saved_kernel", "chain_fwd_fast_kernel"),
                "lookback": ("scan_bwd_kernel", "scan_fwd_kernel")}


def measured_traffic(path: str = TRAFFIC_FILE) -> dict:
    """HBM bytes per launch by kernel name, from a committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (calibrated against a 1 GiB copy); empty
    if the file is absent."""
    out = {}
    try:
        with open(os.path.join(ROOT, path)) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic":
                    out[parts[1]] = int(parts[2])
    except OSError:
        pass
    return out


def measured_valu_busy(path: str = COUNTERS_FILE) -> dict:
    """VALU-busy percentage by kernel name from the committed counter summary
    (rocprofv3 VALUBusy); empty if the file is absent."""
    out = {}
    try:
        with open(os.path.join(ROOT, path)) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "valu_busy":
                    out[parts[1]] = float(parts[2])
    except OSError:
        pass
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def scan_case(B, T, M, G, dev, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    r = torch.sigmoid(torch.randn(B, T, G, device=dev, generator=g) + 2.0).to(torch.bfloat16)
    phi = ((torch.rand(B, T, G, device=dev, generator=g) * 2 - 1) * math.pi).to(torch.bfloat16)
    w_re = torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
    w_im = torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
    dy_re = torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
    dy_im = torch.randn(B, T, M, device=dev, generator=g, dtype=torch.bfloat16)
    return r, phi, w_re, w_im, dy_re, dy_im


def bench_scan(args, dev, B=8, T=4096, D=1024, N=16, steps=None):
    """Polar scan fwd+bwd (bf16 I/O, gates shared per channel) at one shape:
    the headline cfg2 shape by default."""
    from sparc_amd import _lib
    lib = _lib.load()
    M, G = D * N, D
    n_steps = steps or args.steps
    r, phi, w_re, w_im, dy_re, dy_im = scan_case(B, T, M, G, dev)
    d = _lib.ScanDesc(B, T, M, G, _lib.TRANSITIONS["polar"], _lib.SPARC_BF16, _lib.SPARC_BF16,
                      _lib.ALGO_FLAGS[args.algo])
    n_chunks = lib.sparc_scan_chunk_count(ctypes.byref(d))
    y_re, y_im = torch.empty_like(w_re), torch.empty_like(w_im)
    cs = torch.empty(B, n_chunks, M, 2, device=dev, dtype=torch.float32)
    dw_re, dw_im = torch.empty_like(w_re), torch.empty_like(w_im)
    dr, dphi = torch.empty_like(r), torch.empty_like(phi)
    ws_f = torch.empty(lib.sparc_scan_workspace_bytes(ctypes.byref(d), 0), dtype=torch.uint8, device=dev)
    ws_b = torch.empty(lib.sparc_scan_workspace_bytes(ctypes.byref(d), 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream
    P = _lib.ptr

    def fwd():
        _lib.check(lib.sparc_scan_forward(
            ctypes.byref(d), P(r), P(phi), None, None, P(w_re), P(w_im), None, None, None,
            P(y_re), P(y_im), P(cs), P(ws_f), ws_f.numel(), st), "forward")

    def bwd():
        _lib.check(lib.sparc_scan_backward(
            ctypes.byref(d), P(r), P(phi), None, None, P(w_re), P(w_im), P(y_re), P(y_im),
            None, None, None, P(cs), P(dy_re), P(dy_im), None, None, P(dw_re), P(dw_im), P(dr), P(dphi),
            None, None, None, None, P(ws_b), ws_b.numel(), st), "backward")

    for _ in range(args.warmup):
        fwd()
        bwd()
    torch.cuda.synchronize(dev)
    if lib.sparc_scan_workspace_error(P(ws_f), st) or lib.sparc_scan_workspace_error(P(ws_b), st):
        raise RuntimeError("a look-back wait hit its bound during warmup")

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(n_steps)]
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for e0, e1, e2 in ev:
        e0.record(stream)
        fwd()
        e1.record(stream)
        bwd()
        e2.record(stream)
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    fwd_ms = sum(e0.elapsed_time(e1) for e0, e1, _ in ev) / n_steps
    bwd_ms = sum(e1.elapsed_time(e2) for _, e1, e2 in ev) / n_steps
    if lib.sparc_scan_workspace_error(P(ws_f), st) or lib.sparc_scan_workspace_error(P(ws_b), st):
        raise RuntimeError("a look-back wait hit its bound during the timed region")

    tokens = B * T
    mode_steps, group_steps = B * T * M, B * T * G
    bytes_fwd = mode_steps * 8 + group_steps * 4
    bytes_bwd = mode_steps * 12 + group_steps * 8
    ms_step = elapsed * 1e3 / n_steps
    return dict(
        B=B, T=T, D=D, N=N, M=M, G=G, ms_step=ms_step,
        tokens_per_s=tokens * n_steps / elapsed,
        fwd_ms=fwd_ms, bwd_ms=bwd_ms,
        bytes_fwd=bytes_fwd, bytes_bwd=bytes_bwd,
        fwd_gbs=bytes_fwd / fwd_ms / 1e6, bwd_gbs=bytes_bwd / bwd_ms / 1e6,
        step_gbs=(bytes_fwd + bytes_bwd) / ms_step / 1e6,
    )


def bench_cfg3(args, dev):
    """cfg3, reported beside the headline: the real scan, B=4, T=65536,
    D=512, N=8 (M = 4096 modes, G = 512 gate groups of 8), fp32 throughout,
    a ~ U[0.95, 0.9999] per (b, t, d), w and dy ~ N(0, 1).  64 chains of 256
    modes: the decoupled look-back kernels, one workgroup per (chain, 64-step
    chunk); the backward reads the states from the saved output.

    Algorithmic bytes: forward B*T*(8*M + 4*G) (read w, write y; read a),
    backward B*T*(12*M + 8*G) (read dy and y, write dw; read a, write da)."""
    from sparc_amd import _lib
    lib = _lib.load()
    B, T, D, N = 4, 65536, 512, 8
    M, G = D * N, D
    g = torch.Generator(device=dev).manual_seed(0)
    a = 0.95 + 0.0499 * torch.rand(B, T, G, device=dev, generator=g)
    w = torch.randn(B, T, M, device=dev, generator=g)
    dy = torch.randn(B, T, M, device=dev, generator=g)
    y, dw, da = torch.empty_like(w), torch.empty_like(w), torch.empty_like(a)
    d = _lib.ScanDesc(B, T, M, G, _lib.TRANSITIONS["real"], _lib.SPARC_F32, _lib.SPARC_F32, 0)
    cs = torch.empty(B, lib.sparc_scan_chunk_count(ctypes.byref(d)), M, device=dev)
    ws_f = torch.empty(lib.sparc_scan_workspace_bytes(ctypes.byref(d), 0), dtype=torch.uint8, device=dev)
    ws_b = torch.empty(lib.sparc_scan_workspace_bytes(ctypes.byref(d), 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream
    P = _lib.ptr

    def fwd():
        _lib.check(lib.sparc_scan_forward(ctypes.byref(d), P(a), None, None, None, P(w), None, None, None,
                                          None, P(y), None, P(cs), P(ws_f), ws_f.numel(), st), "forward")

    def bwd():
        _lib.check(lib.sparc_scan_backward(
            ctypes.byref(d), P(a), None, None, None, P(w), None, P(y), None, None, None, None, P(cs),
            P(dy), None, None, None, P(dw), None, P(da), None, None, None, None, None,
            P(ws_b), ws_b.numel(), st), "backward")

    for _ in range(SUB_WARMUP):
        fwd()
        bwd()
    steps = max(3, args.steps // 4)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for e0, e1, e2 in ev:
        e0.record(stream)
        fwd()
        e1.record(stream)
        bwd()
        e2.record(stream)
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    if lib.sparc_scan_workspace_error(P(ws_f), st) or lib.sparc_scan_workspace_error(P(ws_b), st):
        raise RuntimeError("a look-back wait hit its bound in the cfg3 run")
    fwd_ms = sum(e0.elapsed_time(e1) for e0, e1, _ in ev) / steps
    bwd_ms = sum(e1.elapsed_time(e2) for _, e1, e2 in ev) / steps
    bytes_fwd = B * T * (8 * M + 4 * G)
    bytes_bwd = B * T * (12 * M + 8 * G)
    ms_step = elapsed * 1e3 / steps
    del a, w, dy, y, dw, da, cs
    traffic = measured_traffic(TRAFFIC_FILE_CFG3)
    return {
        "workload": "real scan fwd+bwd, fp32, gates shared by the N=8 states of a channel",
        "B": B, "T": T, "D": D, "N": N, "M": M, "G": G, "steps": steps,
        "tokens_per_s": round(B * T * steps / elapsed, 1), "ms_per_step": round(ms_step, 4),
        "step_frac": round((bytes_fwd + bytes_bwd) / ms_step / 1e6 / HBM_PEAK_GBS, 4),
        "forward": {"kernel": "scan_fwd_kernel (look-back)", "avg_launch_ms": round(fwd_ms, 4),
                    "bytes_per_launch": bytes_fwd, "traffic": traffic.get("scan_fwd_kernel"),
                    "frac": round(bytes_fwd / fwd_ms / 1e6 / HBM_PEAK_GBS, 4)},
        "backward": {"kernel": "scan_bwd_kernel (look-back, saved output)", "avg_launch_ms": round(bwd_ms, 4),
                     "bytes_per_launch": bytes_bwd, "traffic": traffic.get("scan_bwd_kernel"),
                     "frac": round(bytes_bwd / bwd_ms / 1e6 / HBM_PEAK_GBS, 4)},
        "traffic_source": TRAFFIC_FILE_CFG3 if traffic else None,
    }


def _p1_timed(dev, B, T, M, steps, warmup=SUB_WARMUP):
    """Forward and backward of the P1 scan through the C ABI (bf16 writes, fp32
    eta/delta, G = 1) over `steps` timed pairs after `warmup` untimed ones:
    (fwd ms, bwd ms, wall s)."""
    from sparc_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device=dev).manual_seed(0)
    eta = 2.772588722239781 * torch.tanh(0.5 * torch.randn(B, T, 1, device=dev, generator=g))
    delta = 1.5707963267948966 * torch.tanh(torch.randn(B, T, 1, device=dev, generator=g))
    nu_log = torch.log(-0.5 * torch.log(torch.rand(M, device=dev, generator=g).clamp_min(1e-30)))
    theta_log = torch.log((2 * math.pi * torch.rand(M, device=dev, generator=g)).clamp_min(1e-30))
    w_re, w_im, dy_re, dy_im = (torch.randn(B, T, M, device=dev, generator=g).bfloat16() for _ in range(4))
    y_re, y_im, dw_re, dw_im = (torch.empty_like(w_re) for _ in range(4))
    deta, ddelta = torch.empty_like(eta), torch.empty_like(delta)
    dnu, dth = torch.empty_like(nu_log), torch.empty_like(theta_log)
    d = _lib.ScanDesc(B, T, M, 1, _lib.TRANSITIONS["p1"], _lib.SPARC_BF16, _lib.SPARC_F32, 0)
    cs = torch.empty(B, lib.sparc_scan_chunk_count(ctypes.byref(d)), M, 2, device=dev)
    ws_f = torch.empty(lib.sparc_scan_workspace_bytes(ctypes.byref(d), 0), dtype=torch.uint8, device=dev)
    ws_b = torch.empty(lib.sparc_scan_workspace_bytes(ctypes.byref(d), 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream
    P = _lib.ptr

    def fwd():
        _lib.check(lib.sparc_scan_forward(ctypes.byref(d), P(eta), P(delta), P(nu_log), P(theta_log), P(w_re),
                                          P(w_im), None, None, None, P(y_re), P(y_im), P(cs), P(ws_f),
                                          ws_f.numel(), st), "forward")

    def bwd():
        _lib.check(lib.sparc_scan_backward(
            ctypes.byref(d), P(eta), P(delta), P(nu_log), P(theta_log), P(w_re), P(w_im), P(y_re), P(y_im),
            None, None, None, P(cs), P(dy_re), P(dy_im), None, None, P(dw_re), P(dw_im), P(deta), P(ddelta),
            P(dnu), P(dth), None, None, P(ws_b), ws_b.numel(), st), "backward")

    for _ in range(warmup):
        fwd()
        bwd()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for e0, e1, e2 in ev:
        e0.record(stream)
        fwd()
        e1.record(stream)
        bwd()
        e2.record(stream)
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    fwd_ms = sum(e0.elapsed_time(e1) for e0, e1, _ in ev) / steps
    bwd_ms = sum(e1.elapsed_time(e2) for _, e1, e2 in ev) / steps
    del w_re, w_im, dy_re, dy_im, y_re, y_im, dw_re, dw_im, cs
    torch.cuda.empty_cache()
    return fwd_ms, bwd_ms, elapsed


def _p1_bytes(B, T, M):
    """Algorithmic bytes of the P1 scan: forward B*T*(8*M + 8) (read w, write
    y; read eta, delta), backward B*T*(12*M + 16) (read dy and y, write dw;
    read eta, delta, write their gradients)."""
    return B * T * (8 * M + 8), B * T * (12 * M + 16)


def bench_p1(args, dev):
    """The reference's own scan operator (sparc_chunk_scan: the P1 transition
    from per-token eta, delta and per-mode nu_log, theta_log; writes given) at
    the headline shape: B=8, T=4096, M=16384, one gate pair per token (G = 1),
    bf16 writes, fp32 eta/delta, fp32 state.  Forward and backward through the
    C ABI; at G = 1 they run the fused kernels with the writes given (the
    forward on chains of 256 modes with helper waves, mixer_fwd_wide_kernel;
    the backward one wave per chain of 64 modes, mixer_bwd_kernel), the
    backward reading the states from the forward's output.  Beside it the few-chain
    form, B=1, T=65536, M=2048 (32 chains of 64 modes, split into time
    segments: a summary pass, the carry, a replay)."""
    B, T, M = 8, 4096, 16384
    steps = max(3, args.steps // 2)
    fwd_ms, bwd_ms, elapsed = _p1_timed(dev, B, T, M, steps)
    bytes_fwd, bytes_bwd = _p1_bytes(B, T, M)
    ms_step = elapsed * 1e3 / steps
    traffic = measured_traffic(COUNTERS_FILE)
    valu = measured_valu_busy()
    kf, kb = "mixer_fwd_wide_kernel (writes given)", "mixer_bwd_kernel (writes given)"
    Bf, Tf, Mf, sf = 1, 65536, 2048, 10
    ff_ms, fb_ms, fel = _p1_timed(dev, Bf, Tf, Mf, sf)
    fbf, fbb = _p1_bytes(Bf, Tf, Mf)
    fms = fel * 1e3 / sf
    return {
        "workload": "P1 chunk scan fwd+bwd (the reference's sparc_chunk_scan), one (eta, delta) per token",
        "B": B, "T": T, "M": M, "G": 1, "io_dtype": "bf16", "steps": steps,
        "tokens_per_s": round(B * T * steps / elapsed, 1), "ms_per_step": round(ms_step, 4),
        "step_frac": round((bytes_fwd + bytes_bwd) / ms_step / 1e6 / HBM_PEAK_GBS, 4),
        "forward": {"kernel": kf, "avg_launch_ms": round(fwd_ms, 4), "bytes_per_launch": bytes_fwd,
                    "traffic": traffic.get("mixer_fwd_wide_kernel_p1"), "valu_busy_pct": valu.get("mixer_fwd_wide_kernel_p1"),
                    "frac": round(bytes_fwd / fwd_ms / 1e6 / HBM_PEAK_GBS, 4)},
        "backward": {"kernel": kb, "avg_launch_ms": round(bwd_ms, 4), "bytes_per_launch": bytes_bwd,
                     "traffic": traffic.get("mixer_bwd_kernel_p1"), "valu_busy_pct": valu.get("mixer_bwd_kernel_p1"),
                     "frac": round(bytes_bwd / bwd_ms / 1e6 / HBM_PEAK_GBS, 4)},
        "counters_source": COUNTERS_FILE if "mixer_fwd_wide_kernel_p1" in traffic else None,
        "few_chains": {
            "workload": "P1 chunk scan fwd+bwd, few long chains (time segments)",
            "B": Bf, "T": Tf, "M": Mf, "G": 1, "steps": sf, "ms_per_step": round(fms, 4),
            "tokens_per_s": round(Bf * Tf * sf / fel, 1), "bytes_per_step": fbf + fbb,
            "step_frac": round((fbf + fbb) / fms / 1e6 / HBM_PEAK_GBS, 4),
            "forward": {"avg_launch_ms": round(ff_ms, 4), "bytes_per_launch": fbf,
                        "frac": round(fbf / ff_ms / 1e6 / HBM_PEAK_GBS, 4)},
            "backward": {"avg_launch_ms": round(fb_ms, 4), "bytes_per_launch": fbb,
                         "frac": round(fbb / fb_ms / 1e6 / HBM_PEAK_GBS, 4)},
        },
    }


def bench_cfg5(args, dev):
    """cfg5: a 12-layer stack of SPARC blocks (RMSNorm -> Linear(768 -> 2M) ->
    SPARCMixer -> Linear(2M -> 768), residual; M = 768*16 = 12288), bf16
    weights and activations, B=16, T=2048, token embeddings ~ N(0, 1).  One
    step = forward, backward (loss: mean square of the output) and an AdamW
    update (torch's fused AdamW kernel).  The projections are 6 * tokens * 12
    * 2 * 768 * 24576 = 89.1 TFLOP per step (hipBLASLt / rocBLAS GEMMs through
    torch, with the solutions of the stack's TunableOp file when its library
    versions match); the mixers run the fused HIP sequence path."""
    from sparc_amd.stack import SPARCStack, use_default_gemms, use_tuned_gemms
    L, d_model, N, B, T = 12, 768, 16, 16, 2048
    torch.manual_seed(0)
    model = SPARCStack(L, d_model, N).to(dev).to(torch.bfloat16)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)
    tuned = use_tuned_gemms()
    x = torch.randn(B, T, d_model, device=dev, dtype=torch.bfloat16)

    def step():
        opt.zero_grad(set_to_none=True)
        loss = model(x).float().square().mean()
        loss.backward()
        opt.step()
        return loss

    for _ in range(2):
        step()
    torch.cuda.synchronize(dev)
    steps = 3
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    if not math.isfinite(loss.item()):
        raise RuntimeError("cfg5: non-finite loss")
    ms = elapsed * 1e3 / steps
    flop = 6.0 * B * T * L * 2 * d_model * 2 * d_model * N
    use_default_gemms()
    del model, opt, x
    torch.cuda.empty_cache()
    return {"workload": "12 SPARC blocks (RMSNorm, Linear 768->24576, SPARCMixer, Linear 24576->768), "
                        "fwd + bwd + AdamW", "layers": L, "d_model": d_model, "N": N, "B": B, "T": T,
            "dtype": "bf16", "optimizer": "AdamW (fused)",
            "gemm_solutions": "sparc_amd/tuning/gemm_stack_gfx950.csv" if tuned else "torch default",
            "steps": steps, "ms_per_step": round(ms, 2),
            "tokens_per_s": round(B * T / (ms * 1e-3), 1), "gemm_tflop_per_step": round(flop / 1e12, 1),
            "model_tflops": round(flop / (ms * 1e-3) / 1e12, 1)}


def bench_module(args, dev):
    """The drop-in module at the headline shape: SPARCMixer(2 * D * N) forward
    + backward on x [8, 4096, 32768] bf16 (fp32 parameters, initialised as the
    reference does, controllers and write responses set to small random
    values so that every term is active).  On this shape the module runs the
    fused sequence path (controls, write, P1 scan, relu(cat) epilogue and their
    backward; the backward in one launch with the controls' backward inside,
    `backward_form`).  Its kernels are VALU-bound (the counter summary's VALU
    busy), so its roofline object reports the HBM rate of its algorithmic
    bytes beside the measured traffic and VALU-busy figures."""
    import sparc_amd
    from sparc_amd.mixer import use_fused
    B, T, W = 8, 4096, 2 * 1024 * 16
    torch.manual_seed(0)
    m = sparc_amd.SPARCMixer(W).to(dev)
    with torch.no_grad():
        m.phase_direction.normal_(0, 1 / math.sqrt(W))
        m.radial_direction.normal_(0, 1 / math.sqrt(W))
        m.write_phase_response.normal_()
        m.write_radial_response.normal_()
    x = torch.randn(B, T, W, device=dev, dtype=torch.bfloat16).requires_grad_()
    dy = torch.randn(B, T, W, device=dev, dtype=torch.bfloat16)
    path = "fused" if use_fused(x, W // 2) else "composed"

    def step():
        x.grad = None
        for p in m.parameters():
            p.grad = None
        y, _ = m(x)
        y.backward(dy)

    for _ in range(SUB_WARMUP):
        step()
    torch.cuda.synchronize(dev)
    steps = 5
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / steps
    del m, x, dy
    torch.cuda.empty_cache()
    # algorithmic bytes of the drop-in (G = 1) form: per token 10 bf16 planes
    # of M (x in, y out; dy in, x in, dx out) and 6 fp32 control values
    M = W // 2
    algo_bytes = B * T * (M * 10 * 2 + 6 * 4)
    form = sparc_amd.backward_form(B, T, M, torch.bfloat16)
    kernels = ("ctrl_fwd_kernel", "mixer_fwd_wide_kernel", "mixer_bwd_kernel")
    if form != "one_launch":
        kernels += ("ctrl_bwd_kernel",)
    traffic = measured_traffic(COUNTERS_FILE)
    valu = measured_valu_busy()
    measured = sum(traffic[k] for k in kernels) if path == "fused" and all(k in traffic for k in kernels) else None
    gbs = algo_bytes / (ms * 1e-3) / 1e9
    roof = {"bound": "valu", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_step": algo_bytes,
            "traffic": measured, "traffic_source": COUNTERS_FILE if measured else None,
            "valu_busy_pct": {k: valu[k] for k in kernels if k in valu} or None}
    out = {"workload": "SPARCMixer forward + backward (the drop-in module), bf16 x, fp32 parameters",
           "B": B, "T": T, "width": W, "path": path, "backward_form": form, "steps": steps,
           "ms_per_step": round(ms, 3),
           "tokens_per_s": round(B * T / (ms * 1e-3), 1), "roofline": roof}
    out["few_chains"] = bench_module_few_chains(dev)
    return out


def bench_module_few_chains(dev):
    """The module on few long chains: B=1, T=65536, width 2048 (16 chains of
    64 modes).  The fused kernels split the sequence into time segments
    (summary pass, carry across segments, replay).  Algorithmic bytes of the
    drop-in form as for the headline module report."""
    import sparc_amd
    B, T, W = 1, 65536, 2048
    torch.manual_seed(0)
    m = sparc_amd.SPARCMixer(W).to(dev)
    with torch.no_grad():
        m.phase_direction.normal_(0, 1 / math.sqrt(W))
        m.radial_direction.normal_(0, 1 / math.sqrt(W))
        m.write_phase_response.normal_()
        m.write_radial_response.normal_()
    x = torch.randn(B, T, W, device=dev, dtype=torch.bfloat16).requires_grad_()
    dy = torch.randn(B, T, W, device=dev, dtype=torch.bfloat16)

    def step():
        x.grad = None
        for p in m.parameters():
            p.grad = None
        y, _ = m(x)
        y.backward(dy)

    for _ in range(SUB_WARMUP):
        step()
    torch.cuda.synchronize(dev)
    steps = 10
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / steps
    M = W // 2
    algo_bytes = B * T * (M * 10 * 2 + 6 * 4)
    gbs = algo_bytes / (ms * 1e-3) / 1e9
    del m, x, dy
    return {"workload": "SPARCMixer forward + backward, few long chains (time segments)", "B": B, "T": T,
            "width": W, "steps": steps, "ms_per_step": round(ms, 3), "tokens_per_s": round(B * T / (ms * 1e-3), 1),
            "bytes_per_step": algo_bytes, "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


def _graph_time_us(dev, n_graph, reps, step_fn):
    """Captures reps HIP graphs of n_graph calls step_fn(i) (i = global step)
    after one eager call, replays them all once untimed and once timed;
    returns microseconds per step."""
    step_fn(0)
    torch.cuda.synchronize(dev)
    graphs = []
    cap_stream = torch.cuda.Stream(dev)
    cap_stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(cap_stream):
        for rep in range(reps):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=cap_stream):
                for i in range(n_graph):
                    step_fn(rep * n_graph + i)
            graphs.append(gr)
    torch.cuda.current_stream(dev).wait_stream(cap_stream)
    torch.cuda.synchronize(dev)
    for gr in graphs[:1]:
        gr.replay()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s = torch.cuda.current_stream(dev)
    e0.record(s)
    for gr in graphs:
        gr.replay()
    e1.record(s)
    torch.cuda.synchronize(dev)
    return e0.elapsed_time(e1) * 1e3 / (n_graph * reps)


def bench_decode_core(args, dev):
    """cfg4, scan-core form: B=256 rows, M = 32768 modes (D=2048, N=16), fresh
    bf16 writes and fresh polar gates per (row, channel) every step (the cfg2
    distributions), fp32 state N(0, 0.1) updated in place by sparc_scan_step;
    steps replayed from captured HIP graphs of 100 steps."""
    from sparc_amd import ops
    B, D, N = 256, 2048, 16
    M, G = D * N, D
    n_graph = 100
    reps = max(1, args.decode_steps // n_graph)
    n = n_graph * reps
    g = torch.Generator(device=dev).manual_seed(2)
    w_re = torch.randn(n, B, M, device=dev, generator=g, dtype=torch.bfloat16)
    w_im = torch.randn(n, B, M, device=dev, generator=g, dtype=torch.bfloat16)
    r = torch.sigmoid(torch.randn(n, B, G, device=dev, generator=g) + 2.0).to(torch.bfloat16)
    phi = ((torch.rand(n, B, G, device=dev, generator=g) * 2 - 1) * math.pi).to(torch.bfloat16)
    sr = 0.1 * torch.randn(B, M, device=dev, generator=g)
    si = 0.1 * torch.randn(B, M, device=dev, generator=g)

    def step(i):
        ops.scan_step("polar", r[i], phi[i], w_re[i], w_im[i], (sr, si))

    us = _graph_time_us(dev, n_graph, reps, step)
    bytes_step = B * (M * 20 + G * 4)  # state read + written (16 B), w (4 B), gates (4 B per group)
    del w_re, w_im, r, phi
    return dict(B=B, M=M, G=G, steps=n, us_per_step=us, tokens_per_s=B / (us * 1e-6),
                bytes_per_step=bytes_step, gbs=bytes_step / (us * 1e-6) / 1e9)


def bench_decode(args, dev):
    """cfg4: B=256 rows, width 65536 (M = 32768 = D*N, D=2048, N=16), fresh
    bf16 x every step, fp32 state N(0, 0.1) updated in place; steps replayed
    from a captured HIP graph of 100 steps."""
    import sparc_amd
    from sparc_amd.decode import latest_sparc_decode
    B, D, N = 256, 2048, 16
    M = D * N
    width = 2 * M
    torch.manual_seed(0)
    m = sparc_amd.SPARCMixer(width).to(dev)
    with torch.no_grad():
        m.phase_direction.normal_(0, 1.0 / math.sqrt(width))
        m.radial_direction.normal_(0, 1.0 / math.sqrt(width))
        m.write_phase_response.normal_()
        m.write_radial_response.normal_()
    m.prepare_inference()
    n_graph = 100
    reps = max(1, args.decode_steps // n_graph)
    g = torch.Generator(device=dev).manual_seed(1)
    xs = torch.randn(n_graph * reps, B, width, device=dev, generator=g, dtype=torch.bfloat16)
    sr = 0.1 * torch.randn(B, M, device=dev, generator=g)
    si = 0.1 * torch.randn(B, M, device=dev, generator=g)

    def step(i):
        latest_sparc_decode(m, xs[i], (sr, si), out_state=(sr, si))

    us = _graph_time_us(dev, n_graph, reps, step)
    bytes_step = B * M * 24
    del xs
    return dict(B=B, D=D, N=N, M=M, steps=n_graph * reps, us_per_step=us,
                tokens_per_s=B / (us * 1e-6), bytes_per_step=bytes_step,
                gbs=bytes_step / (us * 1e-6) / 1e9)


def cpu_baseline(args):
    """The oracle's restatement of the reference's eager CPU path on the cfg2
    shape at reduced T: materialised transitions, a Python time loop over
    [B, M] tensors (forward/scan.py:1355-1375), torch autograd backward, fp32,
    all host threads torch is allowed to use."""
    from oracle import sparc_oracle as O
    threads = torch.get_num_threads()
    B, D, N, Ts = 8, 1024, 16, args.cpu_T
    M, G = D * N, D
    g = torch.Generator().manual_seed(0)
    r = torch.sigmoid(torch.randn(B, Ts, G, generator=g) + 2.0).to(torch.bfloat16).float()
    phi = ((torch.rand(B, Ts, G, generator=g) * 2 - 1) * math.pi).to(torch.bfloat16).float()
    w_re = torch.randn(B, Ts, M, generator=g).to(torch.bfloat16).float()
    w_im = torch.randn(B, Ts, M, generator=g).to(torch.bfloat16).float()
    dy_re = torch.randn(B, Ts, M, generator=g).to(torch.bfloat16).float()
    dy_im = torch.randn(B, Ts, M, generator=g).to(torch.bfloat16).float()
    reps, total = 0, 0.0
    while total < args.cpu_seconds or reps == 0:
        leaves = [t.clone().requires_grad_() for t in (r, phi, w_re, w_im)]
        t0 = time.perf_counter()
        (hr, hi), _ = O.grouped_scan_forward("polar", *leaves)
        loss = (hr * dy_re).sum() + (hi * dy_im).sum()
        loss.backward()
        total += time.perf_counter() - t0
        reps += 1
    return dict(value=B * Ts * reps / total, unit="tokens/s", cores=threads, kind="port",
                sample=f"oracle eager polar scan fwd+bwd (autograd), fp32, B={B} T={Ts} "
                       f"M={M} G={G}, {reps} reps in {total:.1f}s on {threads} threads "
                       f"({cpu_model()}, os.cpu_count()={os.cpu_count()})")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--decode-steps", type=int, default=1000)
    ap.add_argument("--cpu-T", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cfg3", action="store_true", help="skip the cfg3 (real, T=65536) report")
    ap.add_argument("--no-cfg5", action="store_true", help="skip the cfg5 (12-layer stack) report")
    ap.add_argument("--no-module", action="store_true", help="skip the module (SPARCMixer) report")
    ap.add_argument("--no-p1", action="store_true", help="skip the P1 operator (sparc_chunk_scan) report")
    ap.add_argument("--algo", default="auto", choices=["auto", "serial", "chain", "lookback"],
                    help="scan algorithm (auto picks the serial kernels at this shape)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="first copy, sum and fill 1 GiB (kernels of known traffic, "
                         "to calibrate the FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's scan runs on a single MI355X "
              "(multi-GPU sharding is a design note, not implemented); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda", 0)
    if args.copy_probe:
        # kernels of known traffic for the FETCH_SIZE / WRITE_SIZE factors:
        # a 1 GiB copy (1 GiB read, 1 GiB written), a 1 GiB sum (read only)
        # and a 1 GiB fill (written only)
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize(dev)
        total = src.sum(dtype=torch.float32)
        dst.fill_(2.0)
        torch.cuda.synchronize(dev)
        del src, dst, total
    res = bench_scan(args, dev)
    # few long chains: 8 chains of 256 modes, which the serial kernels split
    # into time segments (the reference's long-context regime)
    few = bench_scan(argparse.Namespace(**{**vars(args), "warmup": max(args.warmup, SUB_WARMUP)}), dev,
                     B=1, T=65536, D=128, N=16, steps=10)
    p1 = None if args.no_p1 else bench_p1(args, dev)
    cfg3 = None if args.no_cfg3 else bench_cfg3(args, dev)
    cfg5 = None if args.no_cfg5 else bench_cfg5(args, dev)
    module = None if args.no_module else bench_module(args, dev)
    core = None if args.no_decode else bench_decode_core(args, dev)
    dec = None if args.no_decode else bench_decode(args, dev)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args)
    k_bwd, k_fwd = ALGO_KERNELS[args.algo]
    traffic = measured_traffic()
    roof = {
        "bound": "hbm",
        "kernel": f"{k_bwd} (backward scan, polar, bf16 I/O, fp32 state, 4 modes per lane)",
        "achieved": round(res["bwd_gbs"], 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(res["bwd_gbs"] / HBM_PEAK_GBS, 4),
        "traffic": traffic.get(k_bwd),
        "traffic_source": TRAFFIC_FILE if k_bwd in traffic else None,
        "bytes_per_launch": res["bytes_bwd"],
        "avg_launch_ms": round(res["bwd_ms"], 4),
        "forward": {"kernel": k_fwd, "achieved": round(res["fwd_gbs"], 1),
                    "frac": round(res["fwd_gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic.get(k_fwd),
                    "bytes_per_launch": res["bytes_fwd"], "avg_launch_ms": round(res["fwd_ms"], 4)},
        "step_frac": round(res["step_gbs"] / HBM_PEAK_GBS, 4),
    }
    line = {
        "metric": "fwd+bwd tokens/s & %HBM roofline @B8 T4096 D1024 N16; decode step us @B256",
        "value": round(res["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "secondary_warmup": SUB_WARMUP,
        "ms_per_step": round(res["ms_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: w, dy ~ N(0,1); r = sigmoid(N(2,1)); phi ~ U(-pi,pi)",
        "config": {"workload": "complex chunked scan fwd+bwd (polar gates shared per channel)",
                   "B": res["B"], "T": res["T"], "D": res["D"], "N": res["N"], "M": res["M"],
                   "G": res["G"], "io_dtype": "bf16", "gate_dtype": "bf16", "state_dtype": "f32",
                   "accumulate_dtype": "f32", "algorithm": args.algo,
                   "parallelism": "single GPU"},
        "roofline": roof,
        "decode": None if core is None else {
            "us_per_step": round(core["us_per_step"], 2), "tokens_per_s": round(core["tokens_per_s"], 1),
            "steps": core["steps"], "B": core["B"], "M": core["M"], "G": core["G"],
            "bytes_per_step": core["bytes_per_step"], "GB_s": round(core["gbs"], 1),
            "form": "scan-core step (sparc_scan_step): fresh bf16 writes and polar gates each step, "
                    "fp32 state in place, HIP graphs of 100 steps",
            "module": {
                "us_per_step": round(dec["us_per_step"], 2), "tokens_per_s": round(dec["tokens_per_s"], 1),
                "steps": dec["steps"], "bytes_per_step": dec["bytes_per_step"], "GB_s": round(dec["gbs"], 1),
                "form": "SPARCMixer.step (P1 controls and write from x), bf16 x/y, fp32 state in place"}},
        "few_chains_scan": {
            "workload": "complex chunked scan fwd+bwd, few long chains (polar, bf16 I/O, fp32 state)",
            "B": few["B"], "T": few["T"], "D": few["D"], "N": few["N"], "M": few["M"], "G": few["G"],
            "ms_per_step": round(few["ms_step"], 4), "tokens_per_s": round(few["tokens_per_s"], 1),
            "bytes_per_step": few["bytes_fwd"] + few["bytes_bwd"],
            "forward": {"avg_launch_ms": round(few["fwd_ms"], 4), "bytes_per_launch": few["bytes_fwd"],
                        "frac": round(few["fwd_gbs"] / HBM_PEAK_GBS, 4)},
            "backward": {"avg_launch_ms": round(few["bwd_ms"], 4), "bytes_per_launch": few["bytes_bwd"],
                         "frac": round(few["bwd_gbs"] / HBM_PEAK_GBS, 4)},
            "step_frac": round(few["step_gbs"] / HBM_PEAK_GBS, 4)},
        "module": module,
        "p1": p1,
        "cfg3": cfg3,
        "cfg5": cfg5,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
