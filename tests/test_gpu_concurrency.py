"""Two host threads, each with its own stream and buffers, call the library
at once through the C ABI (ctypes releases the GIL for the call): the
operator on a prefill-shaped route in one thread and on the decode route plus
the DSA transform in the other.  Every output must equal the one a single
call on the default stream produced: no call shares state with another
beyond its arguments, as include/fagq.h states."""
import ctypes
import threading

import pytest
import torch

from tests.gpu_util import note

pytestmark = pytest.mark.gpu

P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())


def raw(t):
    """The bytes of an output (column-major scales are a transposed view)."""
    return (t if t.is_contiguous() else t.t()).view(torch.uint8)


def quant_call(lib, _lib, bufs, stream):
    x, r, g, ro, q, sc, M, D, fp8, col = bufs
    return lib.fagq_launch(P(x), P(r), P(g), P(ro), None, P(q), P(sc), M, D, 128, 1e-6,
                           _lib.Q_FP8_E4M3FN if fp8 else _lib.Q_INT8, _lib.SCALE_F32,
                           _lib.LAYOUT_COL_MAJOR if col else _lib.LAYOUT_ROW_MAJOR, _lib.ROUND_RNE,
                           ctypes.c_void_p(stream))


def dsa_call(lib, bufs, stream):
    s, pt, pos, kv, ob, op, B, H, Q, NB, bs, k = bufs
    return lib.fagq_dsa_topk_launch(P(s), 0, P(pt), P(pos), P(kv), 0, P(ob), P(op), B, H, Q, NB, bs,
                                    k, ctypes.c_void_p(stream))


def test_two_threads_two_streams(pkg, gpu):
    from fagq_mi355x import _lib
    lib = pkg.load_library()
    g = torch.Generator().manual_seed(77)

    def quant_bufs(M, D, fp8, col):
        x = torch.randn(M, D, generator=g).bfloat16().to(gpu)
        r = torch.randn(M, D, generator=g).bfloat16().to(gpu)
        w = (1.0 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(gpu)
        q = torch.empty(M, D, dtype=torch.float8_e4m3fn if fp8 else torch.int8, device=gpu)
        sc = pkg.empty_scales(M, D // 128, col_major=col, device=gpu)
        return (x, r, w, torch.empty_like(r), q, sc, M, D, fp8, col)

    big = quant_bufs(2048, 7168, True, True)      # two rows per workgroup, wide scale stores
    small = quant_bufs(4, 8192, False, False)     # decode route
    B, H, Q, NB, bs, k = 1, 4, 64, 2048, 64, 128
    s = torch.randn(B, H, Q, NB, generator=g).to(gpu)
    pt = torch.randperm(B * NB, generator=g).int().view(B, NB).to(gpu)
    pos = torch.arange(NB * bs - Q, NB * bs).view(B, Q).int().to(gpu)
    kv = torch.full((B,), NB * bs, dtype=torch.int32).to(gpu)
    dsa = (s, pt, pos, kv, torch.empty(B, H, Q, k, dtype=torch.int32, device=gpu),
           torch.empty(B, H, Q, k, dtype=torch.int32, device=gpu), B, H, Q, NB, bs, k)

    # Reference outputs: one call each on the default stream.
    default = torch.cuda.current_stream(gpu).cuda_stream
    assert quant_call(lib, _lib, big, default) == 0
    assert quant_call(lib, _lib, small, default) == 0
    assert dsa_call(lib, dsa, default) == 0
    torch.cuda.synchronize(gpu)
    outs = (big[3], big[4], big[5], small[3], small[4], small[5], dsa[4], dsa[5])
    want = [raw(t).clone() for t in outs]
    for t in outs:
        raw(t).fill_(0xcd)
    torch.cuda.synchronize(gpu)

    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    status = [[], []]

    def worker(i):
        st = streams[i].cuda_stream
        for _ in range(25):
            if i == 0:
                status[0].append(quant_call(lib, _lib, big, st))
            else:
                status[1].append(quant_call(lib, _lib, small, st))
                status[1].append(dsa_call(lib, dsa, st))

    note("two host threads, two streams: the operator (2048 x 7168, 4 x 8192) and DSA")
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize(gpu)
    assert status[0] == [0] * 25 and status[1] == [0] * 50
    for a, b in zip(outs, want):
        assert torch.equal(raw(a), b)
