"""The recipe of ``gemm_stack_gfx950.csv`` beside it: writes a TunableOp
results file for the GEMMs of one training step of the 12-layer block stack
(d_model 768, N=16, B=16, T=2048, bf16, AdamW) on the current GPU.  It is
kept in the package so that the committed file can be regenerated for
another ROCm, torch or GPU (the reader rejects files whose validator lines do
not match); nothing imports it at run time:

    python -m sparc_amd.tuning.tune_stack_gemms [OUT.csv]

Every GEMM shape of the step (the four projection products per block and the
small fp32 products of the folded controls) is timed over the hipBLASLt and
rocBLAS solutions torch offers, and the fastest is recorded.  The file's
validator lines pin the torch, HIP, hipBLASLt and rocBLAS versions and the
GPU architecture; ``sparc_amd.stack.use_tuned_gemms`` reads it back.  A run
takes a few minutes.
"""
import os
import sys

import torch
import torch.cuda.tunable as tn

from sparc_amd.stack import SPARCStack


def main(out: str) -> None:
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    model = SPARCStack(12, 768, 16).to(dev).to(torch.bfloat16)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)
    x = torch.randn(16, 2048, 768, device=dev, dtype=torch.bfloat16)
    tn.enable(True)
    tn.tuning_enable(True)
    tn.set_max_tuning_iterations(10)
    tn.set_max_tuning_duration(30)
    tn.set_filename(out)
    opt.zero_grad(set_to_none=True)
    model(x).float().square().mean().backward()
    opt.step()
    torch.cuda.synchronize(dev)
    for r in tn.get_results():
        print(*r, sep=",", flush=True)
    # the results file is written when the process exits (tuning enabled)


if __name__ == "__main__":
    main(os.path.abspath(sys.argv[1] if len(sys.argv) > 1 else "gemm_stack.csv"))
