"""fagq_mla_bwd_launch_noalloc (the MLA backward with its workspace in a
library-owned per-GPU array, for callers that cannot allocate) against
fagq_mla_bwd_launch with a caller workspace: the same kernels on the same
inputs, so dq and dc must be bit-identical.  Two calls in a row, the second
smaller, check that the array's leftover contents from a larger call do not
leak into a later one.  (That a call beyond the array's size is refused is a
CPU test, in test_launch_failure.py.)"""
import ctypes

import pytest
import torch

from tests.gpu_util import note

pytestmark = pytest.mark.gpu


def run_pair(pkg, dev, B, H, S, D, grad_dtype, seed):
    from fagq_mi355x import _lib
    from fagq_mi355x.workloads import MlaWorkload, make_mla_inputs
    w = MlaWorkload(f"noalloc_b{B}h{H}s{S}d{D}", B, H, S, D, grad_dtype, seed=seed)
    q, c, out, do, lse = make_mla_inputs(w, device=dev)
    lib = _lib.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    code = 1 if grad_dtype == torch.bfloat16 else 0
    note(f"case noalloc B={B} H={H} S={S} D={D} {grad_dtype}")
    # reference: the workspace entry point
    ws = torch.empty(lib.fagq_mla_bwd_workspace_bytes(B, S, D), dtype=torch.uint8, device=dev)
    dq0 = torch.full((B, H, S, D), 7.0, dtype=grad_dtype, device=dev)
    dc0 = torch.full((B, S, D), 7.0, dtype=grad_dtype, device=dev)
    _lib.check(lib.fagq_mla_bwd_launch(P(q), P(c), P(out), P(do), P(lse), P(dq0), P(dc0), P(ws),
                                       ws.numel(), B, H, S, D, w.sm_scale, code, code, st),
               "fagq_mla_bwd_launch")
    dq1 = torch.full_like(dq0, -3.0)
    dc1 = torch.full_like(dc0, -3.0)
    _lib.check(lib.fagq_mla_bwd_launch_noalloc(P(q), P(c), P(out), P(do), P(lse), P(dq1), P(dc1),
                                               B, H, S, D, w.sm_scale, code, code, st),
               "fagq_mla_bwd_launch_noalloc")
    torch.cuda.synchronize(dev)
    assert torch.equal(dq1.view(torch.uint8) if grad_dtype == torch.bfloat16 else dq1.view(torch.int32),
                       dq0.view(torch.uint8) if grad_dtype == torch.bfloat16 else dq0.view(torch.int32))
    assert torch.equal(dc1.view(torch.uint8) if grad_dtype == torch.bfloat16 else dc1.view(torch.int32),
                       dc0.view(torch.uint8) if grad_dtype == torch.bfloat16 else dc0.view(torch.int32))


def test_noalloc_matches_workspace_entry_point_twice(pkg, gpu):
    # A larger call (16 MiB of the array), then a smaller one with another
    # head split and scan-block layout.
    run_pair(pkg, gpu, 2, 32, 4096, 512, torch.bfloat16, seed=1)
    run_pair(pkg, gpu, 1, 8, 300, 256, torch.float32, seed=2)

