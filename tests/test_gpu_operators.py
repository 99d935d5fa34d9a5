"""GPU parity of the reference-named operators (sparc_amd.ops, mirroring
sparc-kernal/backward/scan.py:1643-1877) called with valid inputs: values and
gradients against the float64 oracle, plus the reference's return structure,
output and gradient dtypes, and no_grad behaviour of the *_with_last forms.

Tolerance: max |gpu - oracle| / max |oracle| <= 1e-4 (fp32 I/O) or 2e-2
(bf16 I/O), the oracle run in float64 on the same (rounded) inputs."""
import math

import pytest
import torch

from oracle import sparc_oracle as O
from sparc_amd import ops

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16
TOL = {F32: 1e-4, BF16: 2e-2}


def rel_err(got, ref):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    return (got - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)


def leaf(t, device="cuda"):
    return t.detach().clone().to(device).requires_grad_()


def p1_inputs(B, L, M, dtype, seed):
    """P1 scan inputs: eta, delta [B, L] fp32; nu_log, theta_log [M] fp32
    (the module's init); writes [B, L, M] in ``dtype``."""
    g = torch.Generator().manual_seed(seed)
    eta = (O.LOG16 * torch.tanh(0.5 * torch.randn(B, L, generator=g))).float()
    delta = (O.HALF_PI * torch.tanh(torch.randn(B, L, generator=g))).float()
    p = O.init_params(2 * M, generator=g)
    br = torch.randn(B, L, M, generator=g).to(dtype)
    bi = torch.randn(B, L, M, generator=g).to(dtype)
    return dict(eta=eta, delta=delta, nu_log=p.nu_log.float(), theta_log=p.theta_log.float(), br=br, bi=bi)


def oracle_p1(inp, h0=None, segment_pos=None, reset_first=False, relu=False):
    d = {k: v.double().requires_grad_() for k, v in inp.items()}
    h0d = None if h0 is None else tuple(t.double().requires_grad_() for t in h0)
    y, last = O.grouped_scan_forward("p1", d["eta"][..., None], d["delta"][..., None], d["br"], d["bi"],
                                     d["nu_log"], d["theta_log"], h0=h0d, segment_pos=segment_pos,
                                     reset_first=reset_first, relu_output=relu)
    return d, h0d, y, last


def check_grads(got_leaves, ref_leaves, tol, names):
    """Each gradient in its input's dtype, within ``tol`` or, for a gradient
    stored in bf16, the bf16 tolerance (its own rounding is 2^-9)."""
    for n, a, b in zip(names, got_leaves, ref_leaves):
        assert a.grad is not None, f"no gradient for {n}"
        assert a.grad.dtype == a.dtype, f"{n}: gradient dtype {a.grad.dtype} != {a.dtype}"
        e = rel_err(a.grad, b.grad)
        t = max(tol, TOL[a.dtype])
        assert e <= t, f"{n}: gradient rel err {e:.3g} > {t}"


P1_NAMES = ["eta", "delta", "nu_log", "theta_log", "br", "bi"]


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_sparc_scan(dtype):
    """``sparc_scan`` (backward/scan.py:1658-1661): (out_r, out_i) in the
    writes' dtype, gradients of every input."""
    print(f"[case] sparc_scan B=2 L=100 M=64 {dtype}", flush=True)
    inp = p1_inputs(2, 100, 64, dtype, seed=1)
    x = {k: leaf(v) for k, v in inp.items()}
    out = ops.sparc_scan(*(x[k] for k in P1_NAMES))
    assert isinstance(out, tuple) and len(out) == 2 and out[0].dtype == dtype
    d, _, (yr, yi), _ = oracle_p1(inp)
    g = torch.Generator().manual_seed(2)
    dr, di = torch.randn(yr.shape, generator=g), torch.randn(yi.shape, generator=g)
    ((out[0].float() * dr.cuda()).sum() + (out[1].float() * di.cuda()).sum()).backward()
    ((yr * dr.double()).sum() + (yi * di.double()).sum()).backward()
    assert rel_err(out[0], yr) <= TOL[dtype] and rel_err(out[1], yi) <= TOL[dtype]
    check_grads([x[k] for k in P1_NAMES], [d[k] for k in P1_NAMES], TOL[dtype], P1_NAMES)


def test_sparc_scan_with_last_is_no_grad():
    """``sparc_scan_with_last`` (backward/scan.py:1857-1877) runs under
    no_grad: four outputs, last state fp32, nothing requires grad."""
    print("[case] sparc_scan_with_last B=2 L=70 M=64 f32", flush=True)
    inp = p1_inputs(2, 70, 64, F32, seed=3)
    x = {k: leaf(v) for k, v in inp.items()}
    out = ops.sparc_scan_with_last(*(x[k] for k in P1_NAMES))
    assert len(out) == 4 and not any(t.requires_grad for t in out)
    assert out[2].dtype == F32 and out[2].shape == (2, 64)
    _, _, (yr, yi), (lr, li) = oracle_p1(inp)
    for a, b in zip(out, (yr, yi, lr, li)):
        assert rel_err(a, b) <= 1e-4


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_sparc_tiled_serial_scan(dtype):
    """``sparc_tiled_serial_scan`` (backward/scan.py:1664-1687): h0, segment
    resets and reset_first (segment_pos wins), a ragged length; outputs
    (out_r, out_i, last_r, last_i) with gradients of every input, of h0 and
    through the last state."""
    print(f"[case] sparc_tiled_serial_scan B=3 L=77 M=64 {dtype}", flush=True)
    B, L, M = 3, 77, 64
    inp = p1_inputs(B, L, M, dtype, seed=5)
    g = torch.Generator().manual_seed(6)
    h0 = (torch.randn(B, M, generator=g), torch.randn(B, M, generator=g))
    seg = torch.arange(L, dtype=torch.int32).repeat(B, 1) + 1
    seg[0, 30:] = torch.arange(L - 30, dtype=torch.int32)     # row 0: a segment starts at 30
    seg[2, 0] = 0                                              # row 2: starts at 0 (drops h0)
    x = {k: leaf(v) for k, v in inp.items()}
    xh0 = tuple(leaf(t) for t in h0)
    out = ops.sparc_tiled_serial_scan(*(x[k] for k in P1_NAMES), segment_pos=seg.cuda(),
                                      initial_state=xh0, block_size=64, reset_first=True)
    assert len(out) == 4 and out[0].dtype == dtype and out[2].dtype == F32
    d, h0d, (yr, yi), (lr, li) = oracle_p1(inp, h0=h0, segment_pos=seg, reset_first=True)
    ws = [torch.randn(t.shape, generator=g) for t in (yr, yi, lr, li)]
    sum((o.float() * w.cuda()).sum() for o, w in zip(out, ws)).backward()
    sum((o * w.double()).sum() for o, w in zip((yr, yi, lr, li), ws)).backward()
    for a, b in zip(out, (yr, yi, lr, li)):
        assert rel_err(a, b) <= TOL[dtype]
    check_grads([x[k] for k in P1_NAMES] + list(xh0), [d[k] for k in P1_NAMES] + list(h0d),
                TOL[dtype], P1_NAMES + ["h0_re", "h0_im"])
    assert xh0[0].grad[2].abs().max().item() == 0     # row 2 reset at t = 0
    with pytest.raises(ValueError):
        ops.sparc_tiled_serial_scan(*(x[k] for k in P1_NAMES), block_size=100)


@pytest.mark.parametrize("relu", [False, True], ids=["planes", "fused_relu"])
@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_sparc_chunk_scan(relu, dtype):
    """``sparc_chunk_scan`` (backward/scan.py:1703-1751): (out_r, out_i), or
    relu(cat) [B, L, 2M] with fused_output_relu; the reference's knobs are
    validated and do not change the result."""
    print(f"[case] sparc_chunk_scan B=2 L=128 M=64 relu={relu} {dtype}", flush=True)
    B, L, M = 2, 128, 64
    inp = p1_inputs(B, L, M, dtype, seed=7)
    x = {k: leaf(v) for k, v in inp.items()}
    out = ops.sparc_chunk_scan(*(x[k] for k in P1_NAMES), chunk_size=32, hierarchical_prefix=True,
                               prefix_group_size=64, mode_block_size=64, fused_output_relu=relu)
    d, _, y, _ = oracle_p1(inp, relu=relu)
    g = torch.Generator().manual_seed(8)
    if relu:
        assert torch.is_tensor(out) and out.shape == (B, L, 2 * M) and out.dtype == dtype
        # no output gradient where |h| is within the I/O rounding of 0: there
        # the relu mask may differ from float64
        with torch.no_grad():
            (hr, hi), _ = O.grouped_scan_forward("p1", inp["eta"].double()[..., None],
                                                 inp["delta"].double()[..., None], inp["br"].double(),
                                                 inp["bi"].double(), inp["nu_log"].double(),
                                                 inp["theta_log"].double())
            h = torch.cat((hr, hi), -1)
            band = 1e-3 if dtype == F32 else 2e-2
            mask = (h.abs() > band * h.abs().max()).double()
        dy = torch.randn(y.shape, generator=g, dtype=torch.float64) * mask
        (out.float() * dy.float().cuda()).sum().backward()
        (y * dy).sum().backward()
        assert rel_err(out, y) <= TOL[dtype]
    else:
        assert isinstance(out, tuple) and len(out) == 2 and out[0].dtype == dtype
        dr, di = torch.randn(y[0].shape, generator=g), torch.randn(y[1].shape, generator=g)
        ((out[0].float() * dr.cuda()).sum() + (out[1].float() * di.cuda()).sum()).backward()
        ((y[0] * dr.double()).sum() + (y[1] * di.double()).sum()).backward()
        assert rel_err(out[0], y[0]) <= TOL[dtype] and rel_err(out[1], y[1]) <= TOL[dtype]
    check_grads([x[k] for k in P1_NAMES], [d[k] for k in P1_NAMES], TOL[dtype], P1_NAMES)
    with pytest.raises(ValueError, match="divide length"):
        ops.sparc_chunk_scan(*(x[k] for k in P1_NAMES), chunk_size=48)


@pytest.mark.parametrize("case", ["chunk", "h0", "segments", "ragged", "chunk_relu", "ragged_relu"])
def test_sparc_training_scan_dispatch(case):
    """``sparc_training_scan_dispatch`` (backward/scan.py:1754-1818): the chunk
    path, and the tiled-serial fallback for h0, segment resets or a partial
    last chunk, each with and without fused_output_relu."""
    print(f"[case] sparc_training_scan_dispatch {case}", flush=True)
    B, M = 2, 64
    L = 100 if case.startswith("ragged") else 96
    relu = case.endswith("relu")
    inp = p1_inputs(B, L, M, F32, seed=11)
    g = torch.Generator().manual_seed(12)
    h0 = (torch.randn(B, M, generator=g), torch.randn(B, M, generator=g)) if case == "h0" else None
    seg = None
    if case == "segments":
        seg = torch.arange(L, dtype=torch.int32).repeat(B, 1) + 1
        seg[1, 40:] = torch.arange(L - 40, dtype=torch.int32)
    x = {k: leaf(v) for k, v in inp.items()}
    xh0 = None if h0 is None else tuple(leaf(t) for t in h0)
    out = ops.sparc_training_scan_dispatch(*(x[k] for k in P1_NAMES), chunk_size=16,
                                           segment_pos=None if seg is None else seg.cuda(),
                                           initial_state=xh0, fused_output_relu=relu)
    d, h0d, y, _ = oracle_p1(inp, h0=h0, segment_pos=seg, relu=relu)
    if relu:
        assert torch.is_tensor(out) and out.shape == (B, L, 2 * M)
        with torch.no_grad():
            yp, _ = O.grouped_scan_forward("p1", inp["eta"].double()[..., None],
                                           inp["delta"].double()[..., None], inp["br"].double(),
                                           inp["bi"].double(), inp["nu_log"].double(),
                                           inp["theta_log"].double())
            h = torch.cat(yp, -1)
            mask = (h.abs() > 1e-3 * h.abs().max()).double()
        dy = torch.randn(y.shape, generator=g, dtype=torch.float64) * mask
        (out * dy.float().cuda()).sum().backward()
        (y * dy).sum().backward()
        assert rel_err(out, y) <= 1e-4
    else:
        assert isinstance(out, tuple) and len(out) == 2
        dr, di = torch.randn(y[0].shape, generator=g), torch.randn(y[1].shape, generator=g)
        ((out[0] * dr.cuda()).sum() + (out[1] * di.cuda()).sum()).backward()
        ((y[0] * dr.double()).sum() + (y[1] * di.double()).sum()).backward()
        assert rel_err(out[0], y[0]) <= 1e-4 and rel_err(out[1], y[1]) <= 1e-4
    got = [x[k] for k in P1_NAMES] + (list(xh0) if xh0 else [])
    ref = [d[k] for k in P1_NAMES] + (list(h0d) if h0d else [])
    check_grads(got, ref, 1e-4, P1_NAMES + ["h0_re", "h0_im"])


def cart_inputs(B, L, M, a_dtype, b_dtype, seed, lo=0.95, hi=0.9999):
    g = torch.Generator().manual_seed(seed)
    r = lo + (hi - lo) * torch.rand(B, L, M, generator=g, dtype=torch.float64)
    phi = (torch.rand(B, L, M, generator=g, dtype=torch.float64) * 2 - 1) * 0.3
    ar, ai = (r * torch.cos(phi)).to(a_dtype), (r * torch.sin(phi)).to(a_dtype)
    br = torch.randn(B, L, M, generator=g).to(b_dtype)
    bi = torch.randn(B, L, M, generator=g).to(b_dtype)
    return ar, ai, br, bi


@pytest.mark.parametrize("a_dtype,b_dtype", [(F32, F32), (BF16, BF16), (F32, BF16), (BF16, F32)],
                         ids=["f32", "bf16", "a32_b16", "a16_b32"])
def test_complex_scan(a_dtype, b_dtype):
    """``complex_scan`` (backward/scan.py:1653-1655, _ComplexScan :887-919)
    per-element transition.  The transition keeps its own dtype, as the
    reference loads ``a`` in its dtype and upcasts it (forward/scan.py:
    707-710): outputs in the writes' dtype, each gradient in its input's."""
    print(f"[case] complex_scan B=2 L=1024 M=96 a={a_dtype} b={b_dtype}", flush=True)
    # bf16 rounding may raise |a| by 2^-9: keep |a| well below 1 there.  The
    # fp32-a, bf16-b case takes slow modes, where a transition rounded to bf16
    # would move the outputs by more than the bf16 tolerance
    mixed = a_dtype == F32 and b_dtype == BF16
    lo, hi = (0.9, 0.99) if a_dtype == BF16 else ((0.995, 0.9999) if mixed else (0.95, 0.9999))
    ar, ai, br, bi = cart_inputs(2, 1024, 96, a_dtype, b_dtype, seed=13, lo=lo, hi=hi)
    x = [leaf(t) for t in (ar, ai, br, bi)]
    out = ops.complex_scan(*x)
    assert isinstance(out, tuple) and len(out) == 2 and out[0].dtype == b_dtype
    d = [t.double().requires_grad_() for t in (ar, ai, br, bi)]
    (yr, yi), _ = O.complex_scan(*d)
    g = torch.Generator().manual_seed(14)
    dr, di = torch.randn(yr.shape, generator=g), torch.randn(yi.shape, generator=g)
    ((out[0].float() * dr.cuda()).sum() + (out[1].float() * di.cuda()).sum()).backward()
    ((yr * dr.double()).sum() + (yi * di.double()).sum()).backward()
    tol = TOL[b_dtype]
    assert rel_err(out[0], yr) <= tol and rel_err(out[1], yi) <= tol
    check_grads(x, d, tol, ["ar", "ai", "br", "bi"])
    if mixed:
        # fp32 transitions: the outputs are at their own bf16 rounding (2^-9
        # of each value); with a rounded to bf16 the oracle lands > 2e-2 away
        assert max(rel_err(out[0], yr), rel_err(out[1], yi)) <= 5e-3
        (cr, ci), _ = O.complex_scan(ar.bfloat16().double(), ai.bfloat16().double(), br.double(), bi.double())
        assert min(rel_err(cr, yr), rel_err(ci, yi)) > 2e-2


def test_complex_scan_with_last_is_no_grad():
    print("[case] complex_scan_with_last B=2 L=300 M=64 a=f32 b=bf16", flush=True)
    ar, ai, br, bi = cart_inputs(2, 300, 64, F32, BF16, seed=15)
    out = ops.complex_scan_with_last(*(leaf(t) for t in (ar, ai, br, bi)))
    assert len(out) == 4 and not any(t.requires_grad for t in out)
    assert out[0].dtype == BF16 and out[2].dtype == F32
    (yr, yi), (lr, li) = O.complex_scan(*(t.double() for t in (ar, ai, br, bi)))
    for a, b in zip(out, (yr, yi, lr, li)):
        assert rel_err(a, b) <= 2e-2


def real_inputs(B, L, W, a_dtype, b_dtype, seed, lo=0.95, hi=0.9999):
    g = torch.Generator().manual_seed(seed)
    a = (lo + (hi - lo) * torch.rand(B, L, W, generator=g, dtype=torch.float64)).to(a_dtype)
    b = torch.randn(B, L, W, generator=g).to(b_dtype)
    return a, b


@pytest.mark.parametrize("op", ["real_scan", "real_chunk_scan"])
@pytest.mark.parametrize("a_dtype,b_dtype", [(F32, F32), (BF16, BF16), (F32, BF16)],
                         ids=["f32", "bf16", "a32_b16"])
def test_real_scans(op, a_dtype, b_dtype):
    """``real_scan`` / ``real_chunk_scan`` (backward/scan.py:1643-1650) over
    2048 steps with a in [0.95, 0.9999], or [0.995, 0.9999] for fp32 ``a``
    beside bf16 ``b``: there the retention stays fp32, where bf16 would round
    0.9999 to 1.0 (an undamped accumulator) and move the outputs by about
    5e-2."""
    print(f"[case] {op} B=2 L=2048 W=128 a={a_dtype} b={b_dtype}", flush=True)
    mixed = a_dtype == F32 and b_dtype == BF16
    a, b = real_inputs(2, 2048, 128, a_dtype, b_dtype, seed=17, lo=0.995 if mixed else 0.95)
    xa, xb = leaf(a), leaf(b)
    out = ops.real_scan(xa, xb) if op == "real_scan" else ops.real_chunk_scan(xa, xb, chunk_size=64)
    assert torch.is_tensor(out) and out.dtype == b_dtype and out.shape == b.shape
    da, db = a.double().requires_grad_(), b.double().requires_grad_()
    y, _ = O.real_scan(da, db)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(18))
    (out.float() * dy.cuda()).sum().backward()
    (y * dy.double()).sum().backward()
    tol = TOL[b_dtype]
    e = rel_err(out, y)
    assert e <= tol, f"output rel err {e:.3g}"
    check_grads([xa, xb], [da, db], tol, ["a", "b"])
    if mixed:
        # fp32 retention: the outputs are at their own bf16 rounding; with a
        # rounded to bf16 the oracle lands about 5e-2 away
        assert e <= 5e-3, f"output rel err {e:.3g}"
        yb, _ = O.real_scan(a.bfloat16().double(), b.double())
        assert rel_err(yb, y) > 2e-2


def test_real_scan_with_last_is_no_grad():
    print("[case] real_scan_with_last B=2 L=500 W=64 a=f32 b=bf16", flush=True)
    a, b = real_inputs(2, 500, 64, F32, BF16, seed=19)
    out = ops.real_scan_with_last(leaf(a), leaf(b))
    assert len(out) == 2 and not any(t.requires_grad for t in out)
    assert out[0].dtype == BF16 and out[1].dtype == F32 and out[1].shape == (2, 64)
    y, last = O.real_scan(a.double(), b.double())
    assert rel_err(out[0], y) <= 2e-2 and rel_err(out[1], last) <= 2e-2


@pytest.mark.parametrize("transition", ["polar", "cartesian", "real"])
def test_grouped_fp32_gates_bf16_writes_every_algorithm(transition):
    """fp32 gates shared by groups of modes beside bf16 writes (the general
    kernels; lane-shared fast paths read gates in the I/O dtype and are not
    used for this case) under each algorithm, forward and backward."""
    M, G = 256, 16
    for algo in ("lookback", "chain", "serial"):
        print(f"[case] grouped fp32 gates {transition} B=2 T=300 M={M} G={G} bf16 writes algo={algo}",
              flush=True)
        ops.set_algorithm(algo)
        try:
            g = torch.Generator().manual_seed(21)
            r = 0.95 + 0.0499 * torch.rand(2, 300, G, generator=g)
            phi = (torch.rand(2, 300, G, generator=g) * 2 - 1) * math.pi
            if transition == "polar":
                g0, g1 = r, phi
            elif transition == "cartesian":
                g0, g1 = r * torch.cos(phi), r * torch.sin(phi)
            else:
                g0, g1 = r, None
            wr = torch.randn(2, 300, M, generator=g).bfloat16()
            wi = torch.randn(2, 300, M, generator=g).bfloat16() if transition != "real" else None
            xs = [leaf(t) for t in (g0, g1, wr, wi) if t is not None]
            it = iter(xs)
            xg0 = next(it)
            xg1 = next(it) if g1 is not None else None
            xwr = next(it)
            xwi = next(it) if wi is not None else None
            y, last = ops.chunk_scan(transition, xg0, xg1, xwr, xwi)
            ds = [t.double().requires_grad_() for t in (g0, g1, wr, wi) if t is not None]
            it = iter(ds)
            dg0 = next(it)
            dg1 = next(it) if g1 is not None else None
            dwr = next(it)
            dwi = next(it) if wi is not None else None
            yo, lo = O.grouped_scan_forward(transition, dg0, dg1, dwr, dwi)
            ys = y if isinstance(y, tuple) else (y,)
            yos = yo if isinstance(yo, tuple) else (yo,)
            gen = torch.Generator().manual_seed(22)
            dys = [torch.randn(t.shape, generator=gen) for t in yos]
            sum((a.float() * w.cuda()).sum() for a, w in zip(ys, dys)).backward()
            sum((a * w.double()).sum() for a, w in zip(yos, dys)).backward()
            for a, b in zip(ys, yos):
                assert rel_err(a, b) <= 2e-2, f"{algo}: output rel err {rel_err(a, b):.3g}"
            names = ["g0", "g1", "w_re", "w_im"] if transition != "real" else ["g0", "w_re"]
            check_grads(xs, ds, 2e-2, names)
            assert xg0.grad.dtype == F32
        finally:
            ops.set_algorithm("auto")


@pytest.mark.parametrize("transition", ["polar", "cartesian", "real"])
def test_scan_step_fp32_gates_bf16_writes(transition):
    """The single step (sparc_scan_step) with fp32 gates beside bf16 writes
    equals a one-step scan from the state."""
    print(f"[case] scan step fp32 gates {transition} B=4 M=256 G=16 bf16 writes", flush=True)
    B, M, G = 4, 256, 16
    g = torch.Generator().manual_seed(23)
    r = 0.9 + 0.0999 * torch.rand(B, G, generator=g)
    phi = (torch.rand(B, G, generator=g) * 2 - 1) * math.pi
    g0, g1 = {"polar": (r, phi), "cartesian": (r * torch.cos(phi), r * torch.sin(phi)),
              "real": (r, None)}[transition]
    wr = torch.randn(B, M, generator=g).bfloat16()
    wi = torch.randn(B, M, generator=g).bfloat16() if transition != "real" else None
    h = (torch.randn(B, M, generator=g), torch.randn(B, M, generator=g))
    if transition == "real":
        state = h[0].cuda().contiguous()
        ops.scan_step("real", g0.cuda(), None, wr.cuda(), None, state)
        exp, _ = O.grouped_scan_forward("real", g0.double()[:, None], None, wr.double()[:, None], None,
                                        h0=h[0].double())
        assert rel_err(state, exp[:, 0]) <= 1e-5
        return
    state = (h[0].cuda().contiguous(), h[1].cuda().contiguous())
    ops.scan_step(transition, g0.cuda(), g1.cuda(), wr.cuda(), wi.cuda(), state)
    (er, ei), _ = O.grouped_scan_forward(transition, g0.double()[:, None], g1.double()[:, None],
                                         wr.double()[:, None], wi.double()[:, None],
                                         h0=(h[0].double(), h[1].double()))
    assert rel_err(state[0], er[:, 0]) <= 1e-5 and rel_err(state[1], ei[:, 0]) <= 1e-5
