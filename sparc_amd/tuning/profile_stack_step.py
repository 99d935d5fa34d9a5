"""Where one training step of the 12-layer block stack spends its time
(d_model 768, N=16, B=16, T=2048, bf16, AdamW; the stack's tuned GEMM
solutions when the file's library versions match).  Prints a markdown table
of the GEMMs (shape, calls, average time, TFLOP/s and fraction of MI355X's
dense bf16 peak) and of the other device kernels by total time; nothing
imports it at run time:

    python -m sparc_amd.tuning.profile_stack_step

Times come from torch.profiler (device activity, shapes recorded) over one
step after warm-up; the step time printed first is wall clock over three
un-profiled steps.
"""
import collections
import time

import torch
from torch.profiler import ProfilerActivity, profile

from sparc_amd.stack import SPARCStack, use_tuned_gemms

BF16_DENSE_PEAK = 2.5e15  # MI355X dense bf16 MFMA, FLOP/s


def _self_device_us(evt) -> float:
    t = getattr(evt, "self_device_time_total", None)
    return float(evt.self_cuda_time_total if t is None else t)


def main() -> None:
    dev = torch.device("cuda", 0)
    L, d_model, N, B, T = 12, 768, 16, 16, 2048
    torch.manual_seed(0)
    model = SPARCStack(L, d_model, N).to(dev).to(torch.bfloat16)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)
    tuned = use_tuned_gemms()
    x = torch.randn(B, T, d_model, device=dev, dtype=torch.bfloat16)

    def step():
        opt.zero_grad(set_to_none=True)
        model(x).float().square().mean().backward()
        opt.step()

    for _ in range(3):
        step()
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(3):
        step()
    torch.cuda.synchronize(dev)
    print(f"step: {(time.perf_counter() - t0) * 1e3 / 3:.2f} ms (wall clock, mean of 3; tuned GEMMs: {tuned})",
          flush=True)

    with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA], record_shapes=True) as prof:
        step()
        torch.cuda.synchronize(dev)

    print("\n| GEMM (M x N x K) | dtype | calls | avg (us) | TFLOP/s | % of dense peak |\n|---|---|---:|---:|---:|---:|")
    gemm_us = 0.0
    for e in sorted(prof.key_averages(group_by_input_shape=True), key=lambda e: -_self_device_us(e)):
        us = _self_device_us(e)
        if e.key not in ("aten::mm", "aten::addmm") or us <= 0:
            continue
        shapes = e.input_shapes if e.key == "aten::mm" else e.input_shapes[1:]
        (m, k), (_, n) = shapes[0], shapes[1]
        flop = 2.0 * m * n * k * e.count
        rate = flop / (us * 1e-6)
        gemm_us += us
        print(f"| {m} x {n} x {k} ({e.key}) | {'fp32' if min(m, n, k) <= 2 else 'bf16'} | {e.count} | "
              f"{us / e.count:.1f} | {rate / 1e12:.0f} | {100 * rate / BF16_DENSE_PEAK:.1f} |")
    print(f"\nGEMM device time in the step: {gemm_us / 1e3:.2f} ms", flush=True)

    kernels = collections.defaultdict(lambda: [0, 0.0])
    total = 0.0
    for e in prof.events():
        if e.device_type != torch.autograd.DeviceType.CUDA:
            continue
        us = e.device_time_total if hasattr(e, "device_time_total") else e.cuda_time_total
        kernels[e.name][0] += 1
        kernels[e.name][1] += us
        total += us
    print(f"device time of every kernel in the step: {total / 1e3:.2f} ms\n")
    print("| kernel | launches | total (ms) | avg (us) |\n|---|---:|---:|---:|")
    for name, (cnt, us) in sorted(kernels.items(), key=lambda kv: -kv[1][1])[:30]:
        print(f"| `{name[:90]}` | {cnt} | {us / 1e3:.2f} | {us / cnt:.1f} |")


if __name__ == "__main__":
    main()
