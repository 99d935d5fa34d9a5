"""The allocation-free decode entry point (sparc_decode_step_prepared_noalloc)
against the workspace one it shares its kernels with
(sparc_decode_step_prepared): bit-identical outputs and new states on two
calls in a row, the second with a smaller batch (the library's scratch keeps
the first call's partial sums; the second must not read them), and a host-side
rejection of a batch beyond the scratch limit.  Called through the C ABI."""
import ctypes

import pytest
import torch

from sparc_amd import _lib

pytestmark = pytest.mark.gpu

NOALLOC_MAX_ROWS = 4096


def _consts(lib, modes, g):
    nu_log = (torch.randn(modes, generator=g) - 2.0).cuda()
    theta_log = torch.randn(modes, generator=g).cuda()
    wlg = (-0.1 * torch.rand(modes, generator=g)).cuda()
    wpr = torch.randn(modes, generator=g).cuda()
    wrr = torch.randn(modes, generator=g).cuda()
    consts = torch.empty(modes, 8, device="cuda")
    P = _lib.ptr
    _lib.check(lib.sparc_decode_prepare(modes, P(nu_log), P(theta_log), P(wlg), P(wpr), P(wrr), P(consts),
                                        _lib.stream_of(consts.device)), "sparc_decode_prepare")
    return consts


def _step_inputs(batch, modes, dtype, g):
    width = 2 * modes
    x = torch.randn(batch, width, generator=g).to(dtype).cuda()
    pdir = (0.5 * torch.randn(width + 1, generator=g) / width ** 0.5).cuda()
    rdir = (0.5 * torch.randn(width + 1, generator=g) / width ** 0.5).cuda()
    st_re = (0.1 * torch.randn(batch, modes, generator=g)).cuda()
    st_im = (0.1 * torch.randn(batch, modes, generator=g)).cuda()
    return x, pdir, rdir, st_re, st_im


def _run(lib, noalloc, batch, modes, dtype, x, pdir, rdir, consts, st_re, st_im):
    P = _lib.ptr
    new_re, new_im = torch.empty_like(st_re), torch.empty_like(st_im)
    y = torch.empty_like(x)
    stream = _lib.stream_of(x.device)
    args = (batch, modes, _lib.io_code(dtype), P(x), P(pdir), P(rdir), P(consts), P(st_re), P(st_im),
            P(new_re), P(new_im), P(y))
    if noalloc:
        _lib.check(lib.sparc_decode_step_prepared_noalloc(*args, stream), "noalloc")
    else:
        ws = torch.empty(lib.sparc_decode_workspace_bytes(batch, modes), dtype=torch.uint8, device="cuda")
        _lib.check(lib.sparc_decode_step_prepared(*args, P(ws), ws.numel(), stream), "prepared")
    return y, new_re, new_im


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_noalloc_decode_matches_workspace_entry_point(dtype):
    lib = _lib.load()
    g = torch.Generator().manual_seed(7)
    modes = 1024
    consts = _consts(lib, modes, g)
    for batch in (96, 24):      # the second call smaller than the first
        print(f"[case] no-alloc decode B={batch} M={modes} {dtype}", flush=True)
        x, pdir, rdir, st_re, st_im = _step_inputs(batch, modes, dtype, g)
        ref = _run(lib, False, batch, modes, dtype, x, pdir, rdir, consts, st_re, st_im)
        got = _run(lib, True, batch, modes, dtype, x, pdir, rdir, consts, st_re, st_im)
        torch.cuda.synchronize()
        for a, b, n in zip(got, ref, ("y", "new_re", "new_im")):
            assert torch.equal(a, b), f"B={batch}: {n} differs from the workspace entry point"


def test_noalloc_decode_rejects_batch_beyond_limit():
    """Checked on the host before anything is launched: no pointer is read."""
    lib = _lib.load()
    P = _lib.ptr
    dummy = torch.zeros(16, device="cuda")
    st = lib.sparc_decode_step_prepared_noalloc(NOALLOC_MAX_ROWS + 1, 1024, 1, *([P(dummy)] * 9),
                                                _lib.stream_of(dummy.device))
    assert st == 1 and b"scratch limit" in lib.sparc_last_error()
