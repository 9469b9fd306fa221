"""The device number-format encoders (gfx950 v_cvt_pk_fp8_f32 for OCP fp8
e4m3fn; rint + cvt for int8) against the oracle's encoders, exhaustively
over every fp32 in the binades where the codes change, through the
fagq_diag_encode entry point."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import note

pytestmark = pytest.mark.gpu


def binade(e: int) -> np.ndarray:
    base = np.uint32((e + 127) << 23)
    u = base | np.arange(1 << 23, dtype=np.uint32)
    return np.concatenate([u, u | np.uint32(0x80000000)]).view(np.float32)


def device_encode(pkg, dev, f: np.ndarray, q_format: int, rounding: int,
                  clamp: bool = True) -> np.ndarray:
    from fagq_mi355x import _lib
    src = torch.from_numpy(f).to(dev)
    out = torch.empty(f.size, dtype=torch.uint8, device=dev)
    st = pkg.load_library().fagq_diag_encode(
        ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(out.data_ptr()), f.size, q_format,
        rounding, int(clamp), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    _lib.check(st, "fagq_diag_encode")
    torch.cuda.synchronize(dev)
    return out.cpu().numpy()


def test_fp8_encoder_exhaustive(pkg, gpu):
    from fagq_mi355x import _lib
    for e in range(-12, 10):
        f = binade(e)
        note(f"case fp8 encoder binade 2^{e}")
        got = device_encode(pkg, gpu, f, _lib.Q_FP8_E4M3FN, _lib.ROUND_RNE)
        ref = oracle.encode(f, oracle.Q_FP8, oracle.R_RNE)
        bad = got != ref
        assert not bad.any(), (e, f[bad][:4], got[bad][:4], ref[bad][:4])


def test_fp8_encoder_tiny_and_special(pkg, gpu):
    from fagq_mi355x import _lib
    rng = np.random.default_rng(0)
    u = rng.integers(0, (127 - 12) << 23, size=1 << 20, dtype=np.uint32)
    f = np.concatenate([u.view(np.float32), -u.view(np.float32),
                        np.float32([0.0, -0.0, 448.0, -448.0, 1e30, -1e30, 464.0, 470.0])])
    f = f[: f.size // 8 * 8]
    got = device_encode(pkg, gpu, f, _lib.Q_FP8_E4M3FN, _lib.ROUND_RNE)
    assert np.array_equal(got, oracle.encode(f, oracle.Q_FP8, oracle.R_RNE))


@pytest.mark.parametrize("rounding", ["rne", "trunc"])
def test_int8_encoder_exhaustive(pkg, gpu, rounding):
    from fagq_mi355x import _lib
    r_lib = _lib.ROUND_RNE if rounding == "rne" else _lib.ROUND_TRUNC
    r_orc = oracle.R_RNE if rounding == "rne" else oracle.R_TRUNC
    for e in range(-3, 8):
        f = binade(e)
        note(f"case int8 {rounding} encoder binade 2^{e}")
        got = device_encode(pkg, gpu, f, _lib.Q_INT8, r_lib)
        ref = oracle.encode(f, oracle.Q_INT8, r_orc)
        bad = got != ref
        assert not bad.any(), (e, f[bad][:4], got[bad][:4], ref[bad][:4])


def span(lo: float, hi: float) -> np.ndarray:
    """Every fp32 in [lo, hi) (same sign, lo > 0), both signs, padded to a multiple of 8."""
    a = np.float32(lo).view(np.uint32)
    b = np.float32(hi).view(np.uint32)
    u = np.arange(a, b, dtype=np.uint32)
    f = np.concatenate([u, u | np.uint32(0x80000000)]).view(np.float32)
    pad = (-f.size) % 8
    return np.concatenate([f, np.repeat(f[:1], pad)]) if pad else f


def test_fp8_encoder_unclamped_above_qmax(pkg, gpu):
    """The operator's kernels skip the clamp to +-448: its values stay below
    448 * (1 + 5 * 2^-24).  The device encoder on unclamped inputs must give
    the OCP round-to-nearest-even code, which for [448, 464) is +-448 (0x7e /
    0xfe), on every fp32 of that range (the raw encoder returns NaN only from
    464 up)."""
    from fagq_mi355x import _lib
    f = span(448.0, 464.0)
    note(f"case fp8 encoder unclamped [448, 464): {f.size} values")
    got = device_encode(pkg, gpu, f, _lib.Q_FP8_E4M3FN, _lib.ROUND_RNE, clamp=False)
    ref = oracle.e4m3fn_raw(f)
    assert set(np.unique(ref)) == {0x7e, 0xfe}
    bad = got != ref
    assert not bad.any(), (f[bad][:4], got[bad][:4], ref[bad][:4])


@pytest.mark.parametrize("rounding", ["rne", "trunc"])
def test_int8_encoder_unclamped_above_qmax(pkg, gpu, rounding):
    """Same for int8: every fp32 in [127, 127.5) unclamped gives +-127, as the
    clamped reference does."""
    from fagq_mi355x import _lib
    r_lib = _lib.ROUND_RNE if rounding == "rne" else _lib.ROUND_TRUNC
    r_orc = oracle.R_RNE if rounding == "rne" else oracle.R_TRUNC
    f = span(127.0, 127.5)
    note(f"case int8 {rounding} encoder unclamped [127, 127.5): {f.size} values")
    got = device_encode(pkg, gpu, f, _lib.Q_INT8, r_lib, clamp=False)
    ref = oracle.encode(f, oracle.Q_INT8, r_orc)
    assert np.array_equal(got, ref)
