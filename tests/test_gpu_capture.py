"""Graph capture of the drop-in module's forward and backward.

SPARCMixer forward + backward is captured into a HIP graph with
torch.cuda.graph and replayed several times, with eager work and
synchronisations between the replays; every replay must give the eager run's
output and gradients bit for bit.  The reference launches every kernel on
torch's current stream with no host synchronisation
(sparc-kernal/backward/scan.py:1375-1640), so its path can be captured; so
must this one.  Both forms of the backward at this shape: the one launch
(the chains exchange per-block sums through the workspace; fill kernels, not
memsets, reset it) and, with the one-launch form switched off, the time
pieces (the controls backward of each piece on the library's second stream).

Two orders for the pieces: eager first (the second stream exists when the
capture starts, so the fork and join become graph edges), and capture first
in a fresh process (the library must not create a stream under capture: the
pieces then run on the capturing stream alone, with the same results)."""
import math
import os
import subprocess
import sys

import pytest
import torch

import sparc_amd

pytestmark = pytest.mark.gpu

# B=2, T=1024, width 65536: 1024 chains of 64 modes (no time segments) and
# T a multiple of 8 x 128, so the backward runs in eight time pieces
SHAPE = (2, 1024, 65536)


def _module(width, seed):
    torch.manual_seed(seed)
    m = sparc_amd.SPARCMixer(width)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        m.phase_direction.copy_(0.5 * torch.randn(width + 1, generator=g) / math.sqrt(width))
        m.radial_direction.copy_(0.5 * torch.randn(width + 1, generator=g) / math.sqrt(width))
        m.write_phase_response.copy_(torch.randn(width // 2, generator=g))
        m.write_radial_response.copy_(torch.randn(width // 2, generator=g))
    return m.cuda()


def _inputs(B, T, width, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, width, generator=g).bfloat16().cuda()
    dy = torch.randn(B, T, width, generator=g).bfloat16().cuda()
    dlast = (torch.randn(B, width // 2, generator=g).cuda(), torch.randn(B, width // 2, generator=g).cuda())
    return x, dy, dlast


def _step(m, x, dy, dlast):
    """One forward + backward; the gradients land in x.grad and the
    parameters' .grad (set to None before, so that backward assigns them)."""
    y, (lr, li) = m(x, return_cache=True)
    torch.autograd.backward([y, lr, li], [dy, dlast[0], dlast[1]])
    return y


def _results(m, x, y):
    return [y, x.grad] + [p.grad for p in m.parameters()]


def _clear(m, x):
    x.grad = None
    for p in m.parameters():
        p.grad = None


def _eager(m, x, dy, dlast):
    _clear(m, x)
    y = _step(m, x, dy, dlast)
    torch.cuda.synchronize()
    return [t.detach().clone() for t in _results(m, x, y)]


def _capture_and_replay(m, x, dy, dlast, expect, reps=3):
    _clear(m, x)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            y = _step(m, x, dy, dlast)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    outs = _results(m, x, y)
    for rep in range(reps):
        for t in outs:
            t.detach().fill_(float("nan"))  # a replay must rewrite every output
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(outs, expect)):
            assert torch.equal(got, ref), f"replay {rep}: result {i} differs from the eager run"
        _ = (x.float() * 2).sum().item()  # eager work between replays


@pytest.mark.parametrize("plan", ["auto", "pieces"])
def test_module_fwd_bwd_graph_replays_match_eager(plan):
    B, T, width = SHAPE
    print(f"[case] module fwd+bwd graph capture after eager: B={B} T={T} width={width} bf16 plan={plan}",
          flush=True)
    prev = sparc_amd.set_backward_plan(plan)
    try:
        form = sparc_amd.backward_form(B, T, width // 2, torch.bfloat16)
        assert form == ("one_launch" if plan == "auto" else "pieces")
        m = _module(width, seed=41)
        x, dy, dlast = _inputs(B, T, width, seed=42)
        x.requires_grad_(True)
        expect = _eager(m, x, dy, dlast)       # pieces: creates the library's second stream
        again = _eager(m, x, dy, dlast)
        for a, b in zip(expect, again):
            assert torch.equal(a, b)           # the eager path is deterministic
        _capture_and_replay(m, x, dy, dlast, expect)
    finally:
        sparc_amd.set_backward_plan(prev)


def _capture_first_main():
    """Body of the fresh-process case, with the one-launch backward switched
    off: warm up at a shape without time pieces (which creates no stream),
    capture at the pieced shape, then compare with eager runs made after the
    capture."""
    sparc_amd.set_backward_plan("pieces")
    B, T, width = SHAPE
    m = _module(width, seed=43)
    x, dy, dlast = _inputs(B, T, width, seed=44)
    x.requires_grad_(True)
    xs, dys, dls = _inputs(B, 100, width, seed=45)  # T = 100: no pieces
    xs.requires_grad_(True)
    _eager(m, xs, dys, dls)
    _clear(m, x)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            y = _step(m, x, dy, dlast)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    outs = [t for t in _results(m, x, y)]
    graph.replay()
    torch.cuda.synchronize()
    captured = [t.detach().clone() for t in outs]
    x_eager = x.detach().clone().requires_grad_(True)
    expect = _eager(m, x_eager, dy, dlast)  # now with the second stream
    for i, (got, ref) in enumerate(zip(captured, expect)):
        assert torch.equal(got, ref), f"result {i} of the captured single-stream run differs"
    for rep in range(2):
        for t in outs:
            t.detach().fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(outs, expect)):
            assert torch.equal(got, ref), f"replay {rep}: result {i} differs"
    print("capture-first: ok", flush=True)


def test_module_fwd_bwd_graph_capture_first_in_fresh_process():
    B, T, width = SHAPE
    print(f"[case] module fwd+bwd graph capture before any pieced call (fresh process): B={B} T={T} "
          f"width={width} bf16", flush=True)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
    proc = subprocess.run([sys.executable, os.path.abspath(__file__), "--capture-first"], cwd=root, env=env,
                          capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0, f"child failed ({proc.returncode}):\n{proc.stdout[-2000:]}\n{proc.stderr[-4000:]}"
    assert "capture-first: ok" in proc.stdout


if __name__ == "__main__" and "--capture-first" in sys.argv:
    _capture_first_main()
