"""GPU parity of the P1 scan with one gate pair per token (G = 1), which
sparc_scan_forward / sparc_scan_backward run on the one-wave-per-chain
kernels of the fused module path (writes given, states or relu(cat) out,
chunk states every 64 steps; segment resets and reset_first; few chains
split time into segments).

Values, final states and every gradient (eta, delta, nu_log, theta_log, the
writes, h0) against the float64 oracle, to 1e-4 (fp32 I/O) or 2e-2 (bf16
I/O) of max |oracle|; the chunk states against the general chain kernels'
(the same recurrence, other kernels).  The relu cases take the fused forward
and the general backward (which recomputes the states from the chunk states
the fused forward wrote)."""
import pytest
import torch

from sparc_amd import ops
from test_gpu_scan import BF16, F32, check_case, make_case, rel_err

pytestmark = pytest.mark.gpu

CASES = [
    # (id, B, T, M, dtype, extra)
    ("ragged_f32", 2, 200, 256, F32, {}),
    ("bf16", 2, 192, 256, BF16, {}),
    ("lanes_past_M_h0_f32", 3, 77, 132, F32, dict(h0=True, dlast=True)),
    ("h0_dlast_bf16", 2, 150, 128, BF16, dict(h0=True, dlast=True)),
    ("T1_h0_f32", 3, 1, 128, F32, dict(h0=True, dlast=True)),
    ("relu_bf16", 2, 96, 256, BF16, dict(relu=True)),
    ("relu_h0_f32", 2, 130, 128, F32, dict(relu=True, h0=True, dlast=True)),
    # one or two chains: time segments (23 of 136 steps; 20 of 128)
    ("segments_h0_f32", 1, 3000, 64, F32, dict(h0=True, dlast=True)),
    ("segments_bf16", 2, 2500, 128, BF16, dict(dlast=True)),
    ("segments_relu_h0_f32", 1, 1100, 64, F32, dict(relu=True, h0=True)),
    # 1280 chains of 2 modes per lane in the forward
    ("two_modes_per_lane_bf16", 10, 9, 16384, BF16, dict(h0=True, dlast=True)),
    # reset steps (segment_pos == 0: a := 0), reset_first, and both (segment_pos wins)
    ("resets_h0_f32", 2, 200, 256, F32, dict(h0=True, dlast=True, seg=True)),
    ("resets_bf16", 2, 150, 128, BF16, dict(seg=True)),
    ("reset_first_h0_f32", 2, 80, 128, F32, dict(h0=True, dlast=True, reset_first=True)),
    ("resets_and_reset_first_f32", 2, 90, 256, F32, dict(h0=True, seg=True, reset_first=True)),
    ("resets_relu_f32", 2, 130, 128, F32, dict(h0=True, seg=True, relu=True)),
    ("resets_segments_h0_f32", 1, 3000, 64, F32, dict(h0=True, dlast=True, seg=True)),
    ("reset_first_segments_bf16", 2, 2500, 128, BF16, dict(h0=True, dlast=True, reset_first=True)),
    # 512 chains of 256 modes: the wide forward; a partial last block of modes
    # and of steps
    ("wide_h0_dlast_bf16", 8, 70, 16380, BF16, dict(h0=True, dlast=True)),
    ("wide_resets_reset_first_bf16", 8, 70, 16380, BF16, dict(h0=True, dlast=True, seg=True, reset_first=True)),
    ("wide_h0_f32", 8, 37, 16384, F32, dict(h0=True, dlast=True)),
    # an odd number of modes: one mode per lane in both directions (two
    # otherwise), with and without time segments
    ("odd_M_h0_f32", 2, 90, 131, F32, dict(h0=True, dlast=True)),
    ("odd_M_segments_bf16", 1, 1500, 131, BF16, dict(h0=True, dlast=True, seg=True)),
]


@pytest.mark.parametrize("cid,B,T,M,dtype,extra", CASES, ids=[c[0] for c in CASES])
def test_p1_fused_parity(cid, B, T, M, dtype, extra):
    ops.set_algorithm("auto")
    print(f"[case] p1 fused {cid} B={B} T={T} M={M} {dtype}", flush=True)
    case = make_case("p1", B, T, M, 1, dtype, seed=sum(map(ord, cid)) % 1000, **extra)
    check_case(case)


def _forward_raw(case, algorithm):
    ops.set_algorithm(algorithm)
    try:
        init = case["init"]
        h0 = (None, None) if init is None else tuple(t.cuda() for t in init)
        y_re, y_im, cs = ops.scan_forward_raw(
            "p1", case["g0"].cuda(), case["g1"].cuda(), case["w_re"].cuda(), case["w_im"].cuda(),
            case["nu_log"].cuda(), case["theta_log"].cuda(), h0[0], h0[1], None, False, case["relu"])
        torch.cuda.synchronize()
        return y_re, y_im, cs
    finally:
        ops.set_algorithm("auto")


@pytest.mark.parametrize("B,T,M,relu", [(2, 200, 256, False), (1, 3000, 64, False), (2, 130, 128, True)],
                         ids=["ragged", "segments", "relu"])
def test_p1_fused_chunk_states(B, T, M, relu):
    """Every saved chunk state (the state after steps 63, 127, ... and T-1)
    of the fused forward against the general chain forward's."""
    print(f"[case] p1 fused chunk states B={B} T={T} M={M} relu={relu}", flush=True)
    case = make_case("p1", B, T, M, 1, F32, seed=B * 7 + T, h0=True, relu=relu)
    yf_re, yf_im, csf = _forward_raw(case, "auto")
    yc_re, yc_im, csc = _forward_raw(case, "chain")
    assert csf.shape == csc.shape == (B, (T + 63) // 64, M, 2)
    for c in range(csf.shape[1]):
        e = rel_err(csf[:, c], csc[:, c])
        assert e <= 1e-4, f"chunk {c}: rel err {e:.3g}"
    assert rel_err(yf_re, yc_re) <= 1e-4
    if not relu:
        assert rel_err(yf_im, yc_im) <= 1e-4


@pytest.mark.parametrize("dtype,extra", [
    (BF16, dict(h0=True)),
    (F32, dict(h0=True)),
    (BF16, dict(relu=True)),
    (F32, dict(h0=True, seg=True, reset_first=True)),
], ids=["planes_h0_bf16", "planes_h0_f32", "relu_bf16", "resets_h0_f32"])
def test_p1_wide_forward_matches_one_mode_per_lane(dtype, extra):
    """With at least 512 chains of 256 modes the P1 forward runs the wide
    kernel (4 modes per lane, helper waves building the transitions in LDS);
    one batch row alone has too few chains and runs the one-mode-per-lane
    kernel.  Both compute each step value for value: the batched outputs and
    chunk states equal the row-by-row ones bit for bit.  M = 16380 leaves a
    partial last block of modes, T = 70 a partial last block of steps and a
    partial last chunk."""
    B, T, M = 8, 70, 16380
    print(f"[case] p1 wide forward B={B} T={T} M={M} {dtype} {extra}", flush=True)
    case = make_case("p1", B, T, M, 1, dtype, seed=31, **extra)
    segpos = None if case["segpos"] is None else case["segpos"].cuda()
    init = case["init"]

    def fwd(rows):
        h0 = (None, None) if init is None else tuple(t[rows].cuda() for t in init)
        sp = None if segpos is None else segpos[rows]
        return ops.scan_forward_raw(
            "p1", case["g0"][rows].cuda(), case["g1"][rows].cuda(), case["w_re"][rows].cuda(),
            case["w_im"][rows].cuda(), case["nu_log"].cuda(), case["theta_log"].cuda(), h0[0], h0[1], sp,
            case["reset_first"], case["relu"])

    y_re, y_im, cs = fwd(slice(0, B))
    for b in range(B):
        r_re, r_im, rc = fwd(slice(b, b + 1))
        assert torch.equal(y_re[b:b + 1], r_re), f"row {b}: y_re"
        if not case["relu"]:
            assert torch.equal(y_im[b:b + 1], r_im), f"row {b}: y_im"
        assert torch.equal(cs[b:b + 1], rc), f"row {b}: chunk states"


@pytest.mark.parametrize("dtype,extra", [
    (BF16, dict(h0=True, dlast=True)),
    (F32, dict(h0=True, dlast=True)),
    (BF16, dict(h0=True, dlast=True, seg=True, reset_first=True)),
], ids=["h0_dlast_bf16", "h0_dlast_f32", "resets_bf16"])
def test_p1_backward_batched_matches_row_by_row(dtype, extra):
    """The P1 backward of a batch against each of its rows alone: every
    (row, mode) chain runs the same adjoint recurrence value for value
    whatever the batch around it (the batch's forward runs on wide chains,
    one row's on the one-wave kernel; the backward takes the batch in 128-mode
    chains), so dw and dh0 match bit for bit, as does every row's sum over
    time of the per-mode terms; the per-token gradients (sums over the modes,
    grouped otherwise) agree to fp32 rounding.  M = 16380 leaves a partial
    last block of modes, T = 70 a partial last block of steps."""
    B, T, M = 8, 70, 16380
    print(f"[case] p1 backward batched vs rows B={B} T={T} M={M} {dtype} {extra}", flush=True)
    case = make_case("p1", B, T, M, 1, dtype, seed=37, **extra)
    segpos = None if case["segpos"] is None else case["segpos"].cuda()
    init, dl = case["init"], case["dlast"]

    def run(rows):
        h0 = (None, None) if init is None else tuple(t[rows].cuda() for t in init)
        sp = None if segpos is None else segpos[rows]
        args = [case["g0"][rows].cuda(), case["g1"][rows].cuda(), case["w_re"][rows].cuda(),
                case["w_im"][rows].cuda(), case["nu_log"].cuda(), case["theta_log"].cuda()]
        y_re, y_im, cs = ops.scan_forward_raw("p1", *args, h0[0], h0[1], sp, case["reset_first"], False)
        g = ops.scan_backward_raw("p1", args[0], args[1], args[2], args[3], cs, case["dy_re"][rows].cuda(),
                                  case["dy_im"][rows].cuda(), args[4], args[5], h0[0], h0[1], sp,
                                  case["reset_first"], False, dl[0][rows].cuda(), dl[1][rows].cuda(),
                                  want_dh0=init is not None, y_re=y_re, y_im=y_im)
        torch.cuda.synchronize()
        return g

    gb = run(slice(0, B))
    dnu = torch.zeros_like(gb["dnu"])
    dth = torch.zeros_like(gb["dth"])
    for b in range(B):
        gr = run(slice(b, b + 1))
        for k in ("dw_re", "dw_im", "dh0_re", "dh0_im"):
            if gb[k] is not None:
                assert torch.equal(gb[k][b:b + 1], gr[k]), f"row {b}: {k}"
        for k in ("dg0", "dg1"):
            e = rel_err(gb[k][b:b + 1], gr[k])
            assert e <= 1e-5, f"row {b}: {k} rel err {e:.3g}"
        dnu += gr["dnu"]
        dth += gr["dth"]
    assert rel_err(gb["dnu"], dnu) <= 1e-5 and rel_err(gb["dth"], dth) <= 1e-5
