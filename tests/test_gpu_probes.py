"""The library's ceiling probes (include/fagq_diag.h) move and compute what
their descriptions say, so the bandwidth and issue-rate figures bench.py prints
for them are figures of that work: copy, write and the operator-mix stream on
ragged sizes (a partial last workgroup), and both shapes of the MFMA probe."""
import ctypes

import numpy as np
import pytest
import torch

from tests.gpu_util import note

pytestmark = pytest.mark.gpu

CHUNK = 512 * 16          # bytes one probe workgroup moves per stream


def _stream(pkg, gpu, src, dst, nbytes, mode):
    from fagq_mi355x import _lib
    lib = _lib.load()
    st = lib.fagq_diag_stream(ctypes.c_void_p(src.data_ptr()) if src is not None else None,
                              ctypes.c_void_p(dst.data_ptr()), nbytes, mode,
                              ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream))
    assert st == 0, st
    torch.cuda.synchronize(gpu)


@pytest.mark.parametrize("nbytes", [16, CHUNK, 3 * CHUNK + 48])
def test_copy_and_write_probes(pkg, gpu, nbytes):
    from fagq_mi355x import _lib
    note(f"case stream probes copy/write bytes={nbytes}")
    g = torch.Generator().manual_seed(nbytes)
    src = torch.randint(0, 256, (nbytes,), generator=g, dtype=torch.uint8).to(gpu)
    dst = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device=gpu)
    _stream(pkg, gpu, src, dst, nbytes, _lib.STREAM_COPY)
    out = dst.cpu().numpy()
    assert np.array_equal(out[:nbytes], src.cpu().numpy())
    assert (out[nbytes:] == 0xA5).all()                       # nothing past the end
    dst.fill_(0xA5)
    _stream(pkg, gpu, None, dst, nbytes, _lib.STREAM_WRITE)
    words = dst.cpu().numpy()[:nbytes].view(np.uint32).reshape(-1, 4)
    chunk = np.arange(words.shape[0])
    assert np.array_equal(words[:, 0], (chunk // 512 * CHUNK).astype(np.uint32))   # block base
    assert np.array_equal(words[:, 1], (chunk % 512).astype(np.uint32))            # thread
    assert (words[:, 2] == 2).all() and (words[:, 3] == 3).all()
    assert (dst.cpu().numpy()[nbytes:] == 0xA5).all()


@pytest.mark.parametrize("nbytes", [32, CHUNK, 5 * CHUNK + 96])
def test_operator_mix_probe(pkg, gpu, nbytes):
    """x = src[0, n), residual = src[n, 2n) read; dst[0, n) = x ^ residual and
    dst[n, 1.5n) = per 16-byte chunk (w0 ^ w1, w2 ^ w3) of that."""
    from fagq_mi355x import _lib
    note(f"case stream probe opmix bytes={nbytes}")
    g = torch.Generator().manual_seed(nbytes + 1)
    src = torch.randint(0, 256, (2 * nbytes,), generator=g, dtype=torch.uint8).to(gpu)
    total = nbytes + nbytes // 2
    dst = torch.full((total + 64,), 0x5A, dtype=torch.uint8, device=gpu)
    _stream(pkg, gpu, src, dst, nbytes, _lib.STREAM_OPMIX)
    s = src.cpu().numpy()
    x, r = s[:nbytes].view(np.uint32), s[nbytes:].view(np.uint32)
    mix = (x ^ r).reshape(-1, 4)
    out = dst.cpu().numpy()
    assert np.array_equal(out[:nbytes].view(np.uint32), mix.reshape(-1))
    codes = out[nbytes:total].view(np.uint32).reshape(-1, 2)
    assert np.array_equal(codes[:, 0], mix[:, 0] ^ mix[:, 1])
    assert np.array_equal(codes[:, 1], mix[:, 2] ^ mix[:, 3])
    assert (out[total:] == 0x5A).all()


def test_mfma_rate_probe_shapes(pkg, gpu):
    """Both instruction shapes run, write every thread's word, and repeat bit for
    bit from launch to launch (the operand bytes are arbitrary fp8 codes, NaN
    included: the probe measures issue rate, not values)."""
    from fagq_mi355x import _lib
    lib = _lib.load()
    note("case mfma rate probe, both shapes")
    outs = []
    for shape in (0, 1):
        out = torch.full((4 * 256,), 0x7fa5a5a5, dtype=torch.int32, device=gpu)
        for _ in range(2):
            st = lib.fagq_diag_mfma_rate(ctypes.c_void_p(out.data_ptr()), 4, 3, shape,
                                         ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream))
            assert st == 0, st
            torch.cuda.synchronize(gpu)
            outs.append(out.cpu().clone())
        assert torch.equal(outs[-1], outs[-2])
        assert (outs[-1] != 0x7fa5a5a5).all()
