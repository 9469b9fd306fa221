"""A kernel launch that fails is reported, not swallowed (failure detection).
The library is rebuilt with -DFAGQ_TEST_LAUNCH_FAILURE, a test seam in which
the library's one launch wrapper launches nothing and reports
hipErrorLaunchFailure (719), and the device check is skipped, so the whole
path runs on a machine without a GPU: every entry point must return -719
after validation passes, keep its validation errors and no-op cases
unchanged, and the Python layer must raise FagqError naming a HIP error.

The calls pass made-up device addresses.  The seam build cannot launch a
kernel, and the module is skipped wherever a GPU is visible all the same, so
these tests only ever run on a CPU-only host."""
import ctypes
import shutil

import pytest

HIP_ERROR_LAUNCH_FAILURE = 719
BASE = 0x10_0000_0000


def fake(i):
    return ctypes.c_void_p(BASE + i * 0x1_0000_0000)


@pytest.fixture(scope="module")
def seam(pkg):
    import torch
    if torch.cuda.is_available():
        pytest.skip("made-up device addresses: CPU-only hosts run this module")
    if not shutil.which("hipcc") and not __import__("os").path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    import __graft_entry__ as ge
    from fagq_mi355x import _lib
    build = ge._load_module("fagq_mi355x_build", ge.PKG_DIR / "build.py")
    lib = build.build_variant("launch_failure", defines=("FAGQ_TEST_LAUNCH_FAILURE",))
    seam_lib = _lib.load(lib)
    seam_lib.probe = _lib.load_probe(lib.parent / "libfagq_probe.so")
    return seam_lib


def test_operator_launch_failure_is_returned(seam):
    args = [fake(0), fake(1), fake(2), fake(3), None, fake(4), fake(5), 8, 4096, 128, 1e-6, 1, 0, 0,
            0, None]
    assert seam.fagq_launch(*args) == -HIP_ERROR_LAUNCH_FAILURE
    args[7] = 0                                   # M = 0: nothing launched
    assert seam.fagq_launch(*args) == 0
    args[7], args[0] = 8, None                    # validation still comes first
    assert seam.fagq_launch(*args) == 1


def test_every_launching_entry_point_reports_it(seam):
    st = seam.fagq_launch_mapped(fake(0), fake(1), fake(2), fake(3), None, fake(4), fake(5), 8, 7168,
                                 128, 1e-6, 1, 0, 1, 0, 4, 2, 2, 8, 0, None)
    assert st == -HIP_ERROR_LAUNCH_FAILURE
    parts = (ctypes.c_void_p * 2)(BASE + 6 * 0x1_0000_0000, BASE + 7 * 0x1_0000_0000)
    st = seam.fagq_launch_parts(ctypes.cast(parts, ctypes.c_void_p), 2, fake(1), fake(2), fake(3),
                                fake(4), fake(5), 8, 4096, 128, 1e-6, 1, 0, 0, 0, None)
    assert st == -HIP_ERROR_LAUNCH_FAILURE
    for act, res in ((1, 1), (0, 2), (1, 2), (2, 2)):      # the typed form's type pairs
        st = seam.fagq_launch_typed(fake(0), fake(1), fake(2), fake(3), fake(6), fake(4), fake(5),
                                    8, 4096, 128, 1e-6, 1, 0, 0, 0, act, res, None)
        assert st == -HIP_ERROR_LAUNCH_FAILURE, (act, res)
    assert seam.probe.fagq_diag_stream(fake(0), fake(1), 4096, 0, None) == -HIP_ERROR_LAUNCH_FAILURE
    assert seam.probe.fagq_diag_mfma_rate(fake(0), 1, 1, 0, None) == -HIP_ERROR_LAUNCH_FAILURE
    assert seam.probe.fagq_diag_lds_read(fake(0), 1, 1, 0, None) == -HIP_ERROR_LAUNCH_FAILURE
    assert seam.fagq_diag_encode(fake(0), fake(1), 64, 1, 0, 0, None) == -HIP_ERROR_LAUNCH_FAILURE
    st = seam.fagq_dsa_topk_launch(fake(0), 0, fake(1), fake(2), fake(3), 0, fake(4), fake(5), 1, 2,
                                   4, 1024, 64, 32, None)
    assert st == -HIP_ERROR_LAUNCH_FAILURE
    st = seam.fagq_gemm_launch(fake(0), fake(1), fake(2), fake(3), fake(4), 256, 256, 1024, 0, 1, 0,
                               None)
    assert st == -HIP_ERROR_LAUNCH_FAILURE
    # MLA backward: the first of its three launches fails and the call stops there.
    B, H, S, D = 1, 4, 256, 512
    need = seam.fagq_mla_bwd_workspace_bytes(B, S, D)
    assert need > 0
    st = seam.fagq_mla_bwd_launch(fake(0), fake(1), fake(2), fake(3), fake(4), fake(5), fake(6),
                                  fake(7), need, B, H, S, D, 0.05, 1, 1, None)
    assert st == -HIP_ERROR_LAUNCH_FAILURE
    # The allocation-free form looks up its array's device address first; on
    # a host without a GPU that runtime call's error is what comes back.
    st = seam.fagq_mla_bwd_launch_noalloc(fake(0), fake(1), fake(2), fake(3), fake(4), fake(5),
                                          fake(6), B, H, S, D, 0.05, 1, 1, None)
    assert st < 0


def test_noalloc_refuses_calls_beyond_its_array(seam):
    # The allocation-free MLA entry point refuses a call whose workspace would
    # not fit its 32 MiB per-GPU array, before any device work.
    B, S, D = 8, 4096, 512
    assert seam.fagq_mla_bwd_workspace_bytes(B, S, D) > 32 << 20
    st = seam.fagq_mla_bwd_launch_noalloc(fake(0), fake(1), fake(2), fake(3), fake(4), fake(5),
                                          fake(6), B, 4, S, D, 0.05, 0, 0, None)
    assert st == 7    # FAGQ_E_TOO_LARGE


def test_python_layer_raises_on_it(seam):
    from fagq_mi355x import _lib
    st = seam.fagq_launch(fake(0), fake(1), fake(2), fake(3), None, fake(4), fake(5), 8, 4096, 128,
                          1e-6, 1, 0, 0, 0, None)
    with pytest.raises(_lib.FagqError) as e:
        _lib.check(st)
    assert e.value.status == -HIP_ERROR_LAUNCH_FAILURE and "HIP error" in str(e.value)
