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


def reference_stack(model, x):
    """float64 CPU restatement of SPARCStack.forward with the oracle mixer;
    returns the output and the leaf tensors by parameter name."""
    leaves = {n: p.detach().double().cpu().clone().requires_grad_() for n, p in model.named_parameters()}
    h = x
    for i, blk in enumerate(model.blocks):
        pre = f"blocks.{i}."
        u = F.rms_norm(h, (h.shape[-1],), leaves[pre + "norm.weight"], blk.norm.eps)
        u = u @ leaves[pre + "in_proj.weight"].T
        p = O.MixerParams(**{n: leaves[pre + "mixer." + n] for n in MIXER})
        y = O.mixer_forward(p, u)[0]
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
