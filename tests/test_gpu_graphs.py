"""The allocation-free entry points under HIP-graph capture, as a serving loop
records them: the operator (bf16 and typed), the multi-input form, DSA top-k,
the fp8 GEMM and the allocation-free MLA backward, each captured once, replayed
several times with inputs changed in place by eager work between replays, every
replay checked bit for bit against an eager call on the same inputs.  None
records a memset: these kernels use no scratch, and the MLA kernels write every
workspace word they read."""
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


@pytest.mark.parametrize("S,gdt", [
    (512, torch.bfloat16),       # 128 row workgroups x 8 head groups: the wide K1
    (8192, torch.float32)])      # 2048 row workgroups: the one-head-in-flight fp32 K1
def test_mla_noalloc_graph_replays_match_eager(pkg, gpu, S, gdt):
    """fagq_mla_bwd_launch_noalloc (three kernels, the library's own workspace)
    captured once and replayed with new dO between replays, against the
    caller-workspace entry point run eagerly."""
    from fagq_mi355x import _lib
    from fagq_mi355x.workloads import MlaWorkload, make_mla_inputs
    B, H, D = 1, 16, 512
    code = 1 if gdt == torch.bfloat16 else 0            # FAGQ_MLA_BF16 / FAGQ_MLA_F32
    w = MlaWorkload("graph", B, H, S, D, gdt, seed=3)
    note(f"case graph capture mla noalloc B={B} H={H} S={S} D={D} grads {gdt}")
    q, c, out, do, lse = make_mla_inputs(w, device=gpu)
    lib = _lib.load()
    assert lib.fagq_mla_bwd_workspace_bytes(B, S, D) <= 32 << 20   # FAGQ_MLA_SCRATCH_BYTES
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    dq = torch.empty(B, H, S, D, dtype=gdt, device=gpu)
    dc = torch.empty(B, S, D, dtype=gdt, device=gpu)

    def noalloc(stream):
        _lib.check(lib.fagq_mla_bwd_launch_noalloc(P(q), P(c), P(out), P(do), P(lse), P(dq), P(dc),
                                                   B, H, S, D, w.sm_scale, code, code,
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
                                           P(ws), ws.numel(), B, H, S, D, w.sm_scale, code, code,
                                           ctypes.c_void_p(st.cuda_stream)),
                   "fagq_mla_bwd_launch")
        torch.cuda.synchronize(gpu)
        assert torch.equal(_bits(dq), _bits(dq_e)), f"replay {rep}: dq"
        assert torch.equal(_bits(dc), _bits(dc_e)), f"replay {rep}: dc"


def _replays_match_eager(gpu, call, refresh, outs, label):
    """Captures call(stream) once, then for each replay: refresh() rewrites the
    inputs in place (eager work), the graph replays, and an eager call on the
    same inputs must reproduce every output bit for bit."""
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        call(side)                                      # warm-up outside the capture
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call(side)
    torch.cuda.synchronize(gpu)
    for rep in range(REPLAYS):
        refresh(rep)
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        got = [o.clone() for o in outs]
        for o in outs:
            o.fill_(0)
        call(torch.cuda.current_stream(gpu))
        torch.cuda.synchronize(gpu)
        for i, (a, b) in enumerate(zip(got, outs)):
            assert torch.equal(_bits(a), _bits(b)), f"{label}: replay {rep}, output {i}"


@pytest.mark.parametrize("at,rt", [(torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
def test_typed_graph_replays_match_eager(pkg, gpu, at, rt):
    M, D = 256, 7168
    note(f"case graph capture typed M={M} D={D} x={at} residual={rt}")
    g = torch.Generator(device="cpu").manual_seed(5)
    x = torch.randn(M, D, generator=g).to(at).to(gpu)
    r = torch.randn(M, D, generator=g).to(rt).to(gpu)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(at).to(gpu)
    ro, norm = torch.empty_like(r), torch.empty_like(x)
    q = torch.empty(M, D, dtype=torch.float8_e4m3fn, device=gpu)
    sc = pkg.empty_scales(M, D // 128, col_major=True, device=gpu)

    def call(stream):
        with torch.cuda.stream(stream):
            pkg.fused_add_rmsnorm_group_quant(x, r, w, ro, norm, q, sc, 1e-6, 128)

    def refresh(rep):
        x.copy_((torch.randn(M, D, generator=g) * (rep + 1)).to(at))

    _replays_match_eager(gpu, call, refresh, [ro, norm, q, sc], "typed")


@pytest.mark.parametrize("P_", [4, 8])       # 2-step and 4-step waves
def test_parts_graph_replays_match_eager(pkg, gpu, P_):
    from fagq_mi355x import _lib
    M, D = 512, 7168
    note(f"case graph capture parts P={P_} M={M} D={D}")
    g = torch.Generator(device="cpu").manual_seed(6)
    parts = [torch.randn(M, D, generator=g).bfloat16().to(gpu) for _ in range(P_)]
    r = torch.randn(M, D, generator=g).bfloat16().to(gpu)
    w = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(gpu)
    ro = torch.empty_like(r)
    q = torch.empty(M, D, dtype=torch.float8_e4m3fn, device=gpu)
    sc = pkg.empty_scales(M, D // 128, col_major=True, device=gpu)
    lib = _lib.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    ptrs = (ctypes.c_void_p * P_)(*[t.data_ptr() for t in parts])

    def call(stream):
        _lib.check(lib.fagq_launch_parts(ptrs, P_, P(r), P(w), P(ro), P(q), P(sc), M, D, 128, 1e-6,
                                         _lib.Q_FP8_E4M3FN, _lib.SCALE_F32, _lib.LAYOUT_COL_MAJOR,
                                         _lib.ROUND_RNE, ctypes.c_void_p(stream.cuda_stream)),
                   "fagq_launch_parts")

    def refresh(rep):
        parts[rep % P_].copy_((torch.randn(M, D, generator=g) * (rep + 1)).bfloat16())

    _replays_match_eager(gpu, call, refresh, [ro, q, sc], "parts")


def test_dsa_graph_replays_match_eager(pkg, gpu):
    B, H, Q, NB, bs, k = 2, 4, 64, 4096, 64, 128
    note(f"case graph capture dsa B={B} H={H} Q={Q} NB={NB} k={k}")
    g = torch.Generator(device="cpu").manual_seed(7)
    s = torch.randn(B, H, Q, NB, generator=g).to(gpu)
    pt = torch.randint(0, 1 << 20, (B, NB), generator=g, dtype=torch.int32).to(gpu)
    pos = torch.randint(0, NB * bs, (B, Q), generator=g, dtype=torch.int32).to(gpu)
    kv = torch.full((B,), NB * bs, dtype=torch.int32).to(gpu)
    ob = torch.empty(B, H, Q, k, dtype=torch.int32, device=gpu)
    op = torch.empty_like(ob)

    def call(stream):
        with torch.cuda.stream(stream):
            pkg.dsa_topk_page_table_transform(s, pt, pos, kv, ob, op, bs, k)

    def refresh(rep):
        s.copy_(torch.randn(B, H, Q, NB, generator=g) * (rep + 1))

    _replays_match_eager(gpu, call, refresh, [ob, op], "dsa")


def test_gemm_graph_replays_match_eager(pkg, gpu):
    from tests.test_gpu_gemm import make
    M, N, K = 512, 2112, 1024
    note(f"case graph capture gemm M={M} N={N} K={K}")
    a_q, a_s, b_q, b_s = [t.to(gpu) for t in make(M, N, K, "f32", "f32", True, seed=8)]
    out = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    g = torch.Generator(device="cpu").manual_seed(8)

    def call(stream):
        with torch.cuda.stream(stream):
            pkg.fp8_block_scaled_gemm(a_q, a_s.t(), b_q, b_s, out=out)

    def refresh(rep):
        a_s.copy_(torch.exp(torch.empty(a_s.shape).uniform_(-4, 2, generator=g)))

    _replays_match_eager(gpu, call, refresh, [out], "gemm")
