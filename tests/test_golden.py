"""The oracle against golden vectors written from the reference's own eager
CPU path (tests/golden/make_golden.py): controls, write, P1 transition, scan,
relu(cat) output, last state, autograd gradients of x and of every parameter,
and three eager decode steps.

The reference computes the controls in fp32 even for a float64 module
(``x.float()`` and ``directions.float()`` in make_controls,
forward/control.py:131-134; ``nu_log.float()`` in the CPU write, :150), while
the oracle is float64 throughout, so agreement is to fp32 rounding: 1e-5 of
each tensor's largest magnitude.  A semantic slip (a swapped direction, a
missing scale) moves the results by O(1)."""
import os

import numpy as np
import torch

from oracle import sparc_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "p1_eager_golden.npz")
NAMES = ["nu_log", "theta_log", "phase_direction", "radial_direction", "write_log_gain",
         "write_phase_response", "write_radial_response"]


def close(a, b, rel=1e-5):
    return (a - b).abs().max().item() <= rel * max(b.abs().max().item(), 1e-30)


def load_golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k]) for k in z.files}


def test_oracle_matches_reference_eager_forward_and_gradients():
    gd = load_golden()
    params = O.MixerParams(**{n: gd[n].clone().requires_grad_() for n in NAMES})
    x = gd["x"].clone().requires_grad_()
    y, last = O.mixer_forward(params, x, return_cache=True)
    assert close(y, gd["y"])
    assert close(last[0], gd["last_re"]) and close(last[1], gd["last_im"])
    loss = (y * gd["dy"]).sum() + (last[0] * gd["dlast_re"]).sum() + (last[1] * gd["dlast_im"]).sum()
    grads = torch.autograd.grad(loss, [x] + [getattr(params, n) for n in NAMES])
    assert close(grads[0], gd["grad_x"])
    for n, g in zip(NAMES, grads[1:]):
        assert close(g, gd["grad_" + n]), n


def test_oracle_matches_reference_eager_decode():
    gd = load_golden()
    params = O.MixerParams(**{n: gd[n] for n in NAMES})
    state = (gd["last_re"], gd["last_im"])
    for t in range(gd["decode_x"].shape[0]):
        y, state = O.decode_step(params, gd["decode_x"][t], state)
        assert close(y, gd["decode_y"][t])
        assert close(state[0], gd["decode_re"][t]) and close(state[1], gd["decode_im"][t])
