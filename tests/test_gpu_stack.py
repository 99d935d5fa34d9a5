"""The SPARC block stack (the 12-layer training configuration's model) on the
GPU against a float64 CPU stack with the oracle mixer: output and every
parameter gradient, fp32 (tolerance 1e-4), and one bf16 training step."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import sparc_oracle as O
from sparc_amd.stack import SPARCStack

pytestmark = pytest.mark.gpu

MIXER = ["nu_log", "theta_log", "phase_direction", "radial_direction", "write_log_gain",
         "write_phase_response", "write_radial_response"]


def rel_err(got, ref):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    return (got - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)


def reference_stack(model, x, relu_masks=None, write_dtype=None, states=None):
    """float64 CPU restatement of SPARCStack.forward with the oracle mixer;
    returns the output and the leaf tensors by parameter name.

    relu_masks[i] (0/1, the shape of block i's mixer output) replaces block
    i's relu(cat(h_re, h_im)) by cat(h_re, h_im) * mask: the GPU's own relu
    decisions, so that states within rounding of 0 (where float64 and the
    GPU may decide differently) route the gradient the way the GPU did.
    states[i] receives block i's cat(h_re, h_im) (detached).  write_dtype
    models the rounding of the write to x's dtype (oracle mixer_forward)."""
    leaves = {n: p.detach().double().cpu().clone().requires_grad_() for n, p in model.named_parameters()}
    h = x
    for i, blk in enumerate(model.blocks):
        pre = f"blocks.{i}."
        u = F.rms_norm(h, (h.shape[-1],), leaves[pre + "norm.weight"], blk.norm.eps)
        u = u @ leaves[pre + "in_proj.weight"].T
        p = O.MixerParams(**{n: leaves[pre + "mixer." + n] for n in MIXER})
        if relu_masks is None and states is None:
            y = O.mixer_forward(p, u, write_dtype=write_dtype)[0]
        else:
            eta, delta = O.controls(u, p.phase_direction, p.radial_direction)
            wr, wi = O.write(u, eta, delta, p.nu_log, p.write_log_gain, p.write_phase_response,
                             p.write_radial_response)
            if write_dtype is not None:
                wr, wi = wr.to(write_dtype).to(wr.dtype), wi.to(write_dtype).to(wi.dtype)
            ar, ai = O.p1_transition(eta[..., None], delta[..., None], p.nu_log, p.theta_log)
            (hr, hi), _ = O.complex_scan(ar, ai, wr, wi)
            hc = torch.cat((hr, hi), dim=-1)
            if states is not None:
                states[i] = hc.detach()
            y = hc.relu() if relu_masks is None else hc * relu_masks[i]
        h = h + y @ leaves[pre + "out_proj.weight"].T
    return F.rms_norm(h, (h.shape[-1],), leaves["norm.weight"], model.norm.eps), leaves


@pytest.mark.parametrize("fold", [True, False], ids=["folded_controls", "separate"])
def test_stack_fp32_matches_oracle_stack(fold, monkeypatch):
    print(f"[case] stack fp32 2 layers d_model=16 N=4 B=2 T=50 fold={fold}", flush=True)
    from sparc_amd import stack
    monkeypatch.setattr(stack, "fuse_projection", fold)
    torch.manual_seed(0)
    model = SPARCStack(2, 16, 4)
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for blk in model.blocks:  # switch the controllers and write responses on
            w = blk.mixer.width
            blk.mixer.phase_direction.copy_(0.5 * torch.randn(w + 1, generator=g) / math.sqrt(w))
            blk.mixer.radial_direction.copy_(0.5 * torch.randn(w + 1, generator=g) / math.sqrt(w))
            blk.mixer.write_phase_response.copy_(torch.randn(w // 2, generator=g))
            blk.mixer.write_radial_response.copy_(torch.randn(w // 2, generator=g))
            blk.norm.weight.copy_(1.0 + 0.1 * torch.randn(16, generator=g))
    x = torch.randn(2, 50, 16, generator=g)
    dy = torch.randn(2, 50, 16, generator=g)
    ref, leaves = reference_stack(model, x.double())
    ref_grads = torch.autograd.grad((ref * dy.double()).sum(), list(leaves.values()), allow_unused=True)
    m = model.cuda()
    out = m(x.cuda())
    names = [n for n, _ in m.named_parameters()]
    grads = torch.autograd.grad((out * dy.cuda()).sum(), list(m.parameters()), allow_unused=True)
    assert rel_err(out, ref) <= 1e-4
    for n, a, b in zip(names, grads, ref_grads):
        if b is None or b.abs().max() == 0:  # energy_response: inactive
            assert a is None or a.abs().max().item() == 0, n
            continue
        assert rel_err(a, b) <= 1e-4, f"{n}: {rel_err(a, b):.3g}"


@pytest.mark.parametrize("fold", [True, False], ids=["folded_controls", "separate"])
def test_stack_bf16_training_step(fold, monkeypatch):
    """One bf16 training step (forward, backward, AdamW) at a reduced cfg5
    shape: finite loss and gradients, parameters updated."""
    print(f"[case] stack bf16 step 2 layers d_model=64 N=16 B=4 T=128 fold={fold}", flush=True)
    from sparc_amd import stack
    monkeypatch.setattr(stack, "fuse_projection", fold)
    torch.manual_seed(0)
    model = SPARCStack(2, 64, 16).cuda().to(torch.bfloat16)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    x = torch.randn(4, 128, 64, device="cuda", dtype=torch.bfloat16)
    before = model.blocks[0].in_proj.weight.detach().clone()
    loss = model(x).float().square().mean()
    loss.backward()
    assert math.isfinite(loss.item())
    for n, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), n
    opt.step()
    assert not torch.equal(before, model.blocks[0].in_proj.weight)


def test_tuned_gemms_match_default():
    """The stack's TunableOp file is accepted on this GPU, and one block at the
    cfg5 shape (B=16, T=2048, d_model=768, N=16, bf16) gives the same output
    and input gradient with the recorded GEMM solutions as with torch's
    defaults (tolerance 2e-2, bf16), with a fused AdamW step after."""
    print("[case] stack tuned gemms 1 layer B=16 T=2048 d_model=768 N=16 bf16", flush=True)
    from sparc_amd.stack import use_default_gemms, use_tuned_gemms
    torch.manual_seed(0)
    model = SPARCStack(1, 768, 16).cuda().to(torch.bfloat16)
    x = torch.randn(16, 2048, 768, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    dy = torch.randn_like(x)

    def run():
        out = model(x)
        (gx,) = torch.autograd.grad(out, [x], dy)
        return out.detach(), gx

    ref, ref_gx = run()
    try:
        assert use_tuned_gemms()
        got, got_gx = run()
        opt = torch.optim.AdamW(model.parameters(), lr=1e-3, fused=True)
        model(x).float().square().mean().backward()
        opt.step()
        torch.cuda.synchronize()
    finally:
        use_default_gemms()
    assert rel_err(got, ref) <= 2e-2
    assert rel_err(got_gx, ref_gx) <= 2e-2
    for n, p in model.named_parameters():
        assert torch.isfinite(p.float()).all(), n


def _switch_on(model, g):
    """Random controller directions, write responses and norm weights (the
    init leaves the controllers off)."""
    with torch.no_grad():
        for blk in model.blocks:
            w = blk.mixer.width
            blk.mixer.phase_direction.copy_(0.5 * torch.randn(w + 1, generator=g) / math.sqrt(w))
            blk.mixer.radial_direction.copy_(0.5 * torch.randn(w + 1, generator=g) / math.sqrt(w))
            blk.mixer.write_phase_response.copy_(torch.randn(w // 2, generator=g))
            blk.mixer.write_radial_response.copy_(torch.randn(w // 2, generator=g))
            blk.norm.weight.copy_(1.0 + 0.1 * torch.randn(blk.norm.weight.shape[0], generator=g))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_cfg5_block_full_size_row_against_float64(dtype):
    """One block of the cfg5 stack (and its final norm) at the full shape:
    B=16, T=2048, d_model=768, N=16 (mixer width 24576), folded controls,
    controllers and write responses switched on.  The output gradient is
    nonzero on the last batch row only, so the GPU's input and parameter
    gradients are exactly that row's, which a float64 CPU restatement of the
    block (oracle mixer, the same parameters) computes.  The restatement
    takes the GPU's relu decisions (its mixer output > 0) for the relu: a
    state within rounding of 0 may fall either side, and the output gradient
    then flows through it on one side only; the test checks that every such
    disagreement lies within that band of 0 (1e-5 of the largest state for
    fp32, 2e-2 for bf16).  Outputs, the input gradient and every parameter
    gradient within 1e-4 (fp32) and 2e-2 (bf16, the write rounded to bf16
    as the fused path and the reference do)."""
    print(f"[case] cfg5 block full size B=16 T=2048 d_model=768 N=16 {dtype}", flush=True)
    tol, band = (1e-4, 1e-5) if dtype == torch.float32 else (2e-2, 2e-2)
    torch.manual_seed(0)
    model = SPARCStack(1, 768, 16)
    g = torch.Generator().manual_seed(5)
    _switch_on(model, g)
    model = model.to(dtype)
    row = 15
    x = torch.randn(16, 2048, 768, generator=g).to(dtype)
    dy = torch.zeros(16, 2048, 768)
    dy[row] = torch.randn(2048, 768, generator=g)
    dy = dy.to(dtype)
    m = SPARCStack(1, 768, 16)
    m.load_state_dict(model.state_dict())
    m = m.to(dtype).cuda()
    seen = {}
    hook = m.blocks[0].out_proj.register_forward_hook(
        lambda mod, inp, out: seen.__setitem__("y", inp[0][row].detach().cpu()))
    xg = x.cuda().requires_grad_()
    out = m(xg)
    hook.remove()
    params = list(m.parameters())
    names = [n for n, _ in m.named_parameters()]
    grads = torch.autograd.grad(out, [xg] + params, dy.cuda(), allow_unused=True)
    torch.cuda.synchronize()
    out_row = out[row].detach().cpu()
    grads = [None if t is None else t.detach().cpu() for t in grads]
    del out, xg, m
    torch.cuda.empty_cache()
    print("[case] gpu done; float64 reference of the last row", flush=True)
    mask = (seen["y"] > 0).double()[None]
    states = {}
    xr = x[row:row + 1].double().requires_grad_()
    ref, leaves = reference_stack(model, xr, relu_masks={0: mask}, states=states,
                                  write_dtype=torch.bfloat16 if dtype == torch.bfloat16 else None)
    h = states[0]
    flip = mask != (h > 0).double()
    flips = int(flip.sum())
    worst = h[flip].abs().max().item() / h.abs().max().item() if flips else 0.0
    print(f"[case] relu decisions differing from float64: {flips} (largest |state| among them "
          f"{worst:.2e} of the largest)", flush=True)
    assert worst <= band, "a relu decision differs away from 0"
    errs = {"out": rel_err(out_row, ref[0])}
    ref_grads = torch.autograd.grad((ref * dy[row:row + 1].double()).sum(), [xr] + list(leaves.values()),
                                    allow_unused=True)
    errs["x"] = rel_err(grads[0][row], ref_grads[0][0])
    for n, a, b in zip(names, grads[1:], ref_grads[1:]):
        if b is None or b.abs().max() == 0:  # energy_response: inactive
            assert a is None or a.abs().max().item() == 0, n
            continue
        errs[n] = rel_err(a, b)
    print("[case] rel errors: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v <= tol, f"{k}: {v:.3g}"
