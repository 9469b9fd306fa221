"""The ceiling probes (libfagq_probe.so, include/fagq_probe.h) move and compute what
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
    lib = _lib.load_probe()
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
    lib = _lib.load_probe()
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


def _lds_probe_addr(pattern: int, lane: int) -> int:
    """Byte address each lane reads, as include/fagq_diag.h states it."""
    r, c = lane % 16, 2 * (lane // 16) + (1 if pattern == 2 else 0)
    f = ((r >> 1) & 1) | (r & 4)
    return {0: 16 * lane, 1: 128 * r + 16 * (c ^ f), 2: 128 * r + 16 * (c ^ f),
            3: 128 * r + 16 * (c ^ ((r >> 1) & 7)), 4: 128 * r + 16 * (c ^ (r & 7)),
            5: 128 * r + 16 * c}[pattern]


@pytest.mark.parametrize("pattern", range(6))
def test_lds_read_probe_addresses(pkg, gpu, pattern):
    """Every thread returns the four 32-bit words at its documented address."""
    from fagq_mi355x import _lib
    lib = _lib.load_probe()
    note(f"case lds read probe pattern={pattern}")
    blocks = 3
    out = torch.full((blocks * 256 * 4,), -1, dtype=torch.int32, device=gpu)
    st = lib.fagq_diag_lds_read(ctypes.c_void_p(out.data_ptr()), blocks, 2, pattern,
                                ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream))
    assert st == 0, st
    torch.cuda.synchronize(gpu)
    got = out.cpu().numpy().view(np.uint32).reshape(blocks, 256, 4)
    words = (np.arange(4096, dtype=np.uint64) * 0x9E3779B1 % (1 << 32)).astype(np.uint32)
    for t in range(256):
        w0 = _lds_probe_addr(pattern, t % 64) // 4
        assert np.array_equal(got[:, t], np.broadcast_to(words[w0:w0 + 4], (blocks, 4))), t


def test_lds_read_probe_fragment_patterns_cover_rows():
    """The fragment patterns read 16 distinct rows at one logical chunk per 16
    lanes, every 16-byte chunk of each row once over the two halves (1, 2) -
    the access the GEMM's operand reads make (CPU check of the address map)."""
    for lanes in (range(0, 16), range(16, 32), range(32, 48), range(48, 64)):
        rows = {_lds_probe_addr(1, l) // 128 for l in lanes}
        assert rows == set(range(16))
    for r in range(16):
        chunks = sorted((_lds_probe_addr(p, l) % 128) // 16 for p in (1, 2) for l in range(64)
                        if l % 16 == r)
        assert chunks == list(range(8))
