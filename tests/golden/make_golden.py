"""Writes tests/golden/p1_eager_golden.npz from the reference's own CPU path.

Run in the build container only (it imports the reference from
/root/reference, which does not exist on the GPU box):

    python tests/golden/make_golden.py

What is exercised (all pure torch on the CPU in the reference):
  * SPARCMixer construction (sparc-kernal/sparc.py:58-88), parameters then
    overwritten with seeded non-trivial values;
  * run_sequence with scan_backend="framework_eager"
    (sparc-kernal/forward/scan.py:1398-1603): make_controls + the CPU branch
    of make_scan_inputs (forward/control.py:129-163), the P1 transition, the
    eager complex scan (forward/scan.py:1355-1375) and the relu(cat) output;
    the last state (the cache) is read from the same branch, called through
    the reference's own functions;
  * torch autograd through that path (gradients of x and every parameter);
  * the eager decode step (forward/decode.py:296-306).
The fixture stores inputs, parameters and outputs as float64 arrays.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

REF = "/root/reference/sparc-kernal"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "p1_eager_golden.npz")


def main() -> None:
    sys.path.insert(0, REF)
    from sparc import SPARCMixer  # noqa: E402  (reference module)

    torch.manual_seed(0)
    g = torch.Generator().manual_seed(1234)
    B, L, width = 2, 24, 16
    M = width // 2
    module = SPARCMixer(width).double()
    with torch.no_grad():
        module.phase_direction.copy_(0.3 * torch.randn(width + 1, generator=g, dtype=torch.float64))
        module.radial_direction.copy_(0.3 * torch.randn(width + 1, generator=g, dtype=torch.float64))
        module.write_phase_response.copy_(torch.randn(M, generator=g, dtype=torch.float64))
        module.write_radial_response.copy_(torch.randn(M, generator=g, dtype=torch.float64))
        module.write_log_gain.add_(0.1 * torch.randn(M, generator=g, dtype=torch.float64))
    module.set_scan_backend("framework_eager")
    x = torch.randn(B, L, width, generator=g, dtype=torch.float64, requires_grad=True)
    # the module call itself (return_cache=True would route to a Triton kernel)
    y_module, _ = module(x, return_cache=False)
    # the same framework_eager branch (forward/scan.py:1584-1602) spelled out
    # with the reference's functions, to also read the last state
    from forward.control import make_scan_inputs
    from forward.scan import _eager_complex_scan
    eta, delta, write_r, write_i = make_scan_inputs(module, x)
    nu, theta = torch.exp(module.nu_log), torch.exp(module.theta_log)
    radius = torch.exp(-nu * torch.exp(eta).unsqueeze(-1))
    phase = theta + (1.0 - radius) * delta.unsqueeze(-1)
    out_r, out_i = _eager_complex_scan(radius * torch.cos(phase), radius * torch.sin(phase),
                                       write_r, write_i)
    y = torch.cat((out_r, out_i), dim=-1).relu()
    assert torch.equal(y, y_module)
    cache = (out_r[:, -1], out_i[:, -1])
    dy = torch.randn(B, L, width, generator=g, dtype=torch.float64)
    dl_r = torch.randn(B, M, generator=g, dtype=torch.float64)
    dl_i = torch.randn(B, M, generator=g, dtype=torch.float64)
    loss = (y * dy).sum() + (cache[0] * dl_r).sum() + (cache[1] * dl_i).sum()
    names = ["nu_log", "theta_log", "phase_direction", "radial_direction", "write_log_gain",
             "write_phase_response", "write_radial_response"]
    params = [getattr(module, n) for n in names]
    grads = torch.autograd.grad(loss, [x] + params)

    # eager decode: continue from the cache for 3 steps
    xs = torch.randn(3, B, width, generator=g, dtype=torch.float64)
    state = (cache[0].detach(), cache[1].detach())
    dec_y, dec_r, dec_i = [], [], []
    with torch.no_grad():
        for t in range(3):
            yt, state = module.step(xs[t], state, segment_pos=None)
            dec_y.append(yt)
            dec_r.append(state[0])
            dec_i.append(state[1])

    out = {"x": x.detach(), "dy": dy, "dlast_re": dl_r, "dlast_im": dl_i, "y": y.detach(),
           "last_re": cache[0].detach(), "last_im": cache[1].detach(), "grad_x": grads[0],
           "decode_x": xs, "decode_y": torch.stack(dec_y), "decode_re": torch.stack(dec_r),
           "decode_im": torch.stack(dec_i)}
    for n, p, gr in zip(names, params, grads[1:]):
        out[n] = p.detach()
        out["grad_" + n] = gr
    np.savez(OUT, **{k: v.numpy() for k, v in out.items()})
    print(f"wrote {OUT}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in out.items()))


if __name__ == "__main__":
    main()
