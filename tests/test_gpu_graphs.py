"""The operator and the allocation-free MLA entry point under HIP-graph capture,
as a serving loop records them: captured once, replayed several times with the
inputs changed in place by eager work between replays, every replay checked bit
for bit against an eager call on the same inputs.  Neither records a memset:
the quantizer uses no scratch, and the MLA kernels write every workspace word
they read."""
import ctypes

import pytest
import torch

from tests.gpu_util import note

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.uint8)


@pytest.mark.parametrize("M,D,qdt,col,ue8m0", [
    (4, 8192, torch.int8, False, False),          # decode-sized, 16 waves per row
    (256, 7168, torch.float8_e4m3fn, True, False),
    (130, 5120, torch.float8_e4m3fn, True, True)])
def test_quantizer_graph_replays_match_eager(pkg, gpu, M, D, qdt, col, ue8m0):
    note(f"case graph capture quantizer M={M} D={D} {qdt} col={col} ue8m0={ue8m0}")
    g = torch.Generator(device="cpu").manual_seed(M + D)
    rnd = "rne" if qdt == torch.int8 else None
    x = torch.randn(M, D, generator=g).bfloat16().to(gpu)
    r = torch.randn(M, D, generator=g).bfloat16().to(gpu)
    w = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(gpu)
    ro = torch.empty_like(r)
    q = torch.empty(M, D, dtype=qdt, device=gpu)
    sc = pkg.empty_scales(M, D // 128, ue8m0=ue8m0, col_major=col, device=gpu)

    def call(ro_, q_, sc_):
        pkg.fused_add_rmsnorm_group_quant(x, r, w, ro_, None, q_, sc_, 1e-6, 128, rounding=rnd)

    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        call(ro, q, sc)                                # warm-up outside the capture
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call(ro, q, sc)
    torch.cuda.synchronize(gpu)

    for rep in range(REPLAYS):
        # eager work between replays: new inputs written in place
        x.copy_((torch.randn(M, D, generator=g) * (rep + 1)).bfloat16())
        r.copy_(torch.randn(M, D, generator=g).bfloat16())
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        ro_e, q_e = torch.empty_like(ro), torch.empty_like(q)
        sc_e = pkg.empty_scales(M, D // 128, ue8m0=ue8m0, col_major=col, device=gpu)
        call(ro_e, q_e, sc_e)
        torch.cuda.synchronize(gpu)
        for a, b in ((ro, ro_e), (q, q_e), (sc, sc_e)):
            assert torch.equal(_bits(a), _bits(b)), f"replay {rep}"


def test_mla_noalloc_graph_replays_match_eager(pkg, gpu):
    """fagq_mla_bwd_launch_noalloc (three kernels, the library's own workspace)
    captured once and replayed with new dO between replays, against the
    caller-workspace entry point run eagerly."""
    from fagq_mi355x import _lib
    from fagq_mi355x.workloads import MlaWorkload, make_mla_inputs
    B, H, S, D = 1, 16, 512, 512
    w = MlaWorkload("graph", B, H, S, D, torch.bfloat16, seed=3)
    note(f"case graph capture mla noalloc B={B} H={H} S={S} D={D}")
    q, c, out, do, lse = make_mla_inputs(w, device=gpu)
    lib = _lib.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    dq = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=gpu)
    dc = torch.empty(B, S, D, dtype=torch.bfloat16, device=gpu)

    def noalloc(stream):
        _lib.check(lib.fagq_mla_bwd_launch_noalloc(P(q), P(c), P(out), P(do), P(lse), P(dq), P(dc),
                                                   B, H, S, D, w.sm_scale, 1, 1,
                                                   ctypes.c_void_p(stream.cuda_stream)),
                   "fagq_mla_bwd_launch_noalloc")

    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    noalloc(side)                                      # warm-up (device check, symbol lookup)
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        noalloc(side)
    torch.cuda.synchronize(gpu)

    ws = torch.empty(lib.fagq_mla_bwd_workspace_bytes(B, S, D), dtype=torch.uint8, device=gpu)
    g = torch.Generator(device="cpu").manual_seed(9)
    for rep in range(REPLAYS):
        do.copy_((torch.randn(B, H, S, D, generator=g) * (rep + 1)).bfloat16())
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        dq_e, dc_e = torch.empty_like(dq), torch.empty_like(dc)
        st = torch.cuda.current_stream(gpu)
        _lib.check(lib.fagq_mla_bwd_launch(P(q), P(c), P(out), P(do), P(lse), P(dq_e), P(dc_e),
                                           P(ws), ws.numel(), B, H, S, D, w.sm_scale, 1, 1,
                                           ctypes.c_void_p(st.cuda_stream)),
                   "fagq_mla_bwd_launch")
        torch.cuda.synchronize(gpu)
        assert torch.equal(_bits(dq), _bits(dq_e)), f"replay {rep}: dq"
        assert torch.equal(_bits(dc), _bits(dc_e)), f"replay {rep}: dc"
