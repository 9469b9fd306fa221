"""The benchmark workloads: seeded, deterministic, and with the byte model
the roofline is computed from."""
import torch


def test_algorithmic_bytes_match_the_byte_model(pkg):
    from fagq_mi355x.workloads import CONFIGS
    # B = 4N + 2D + 2N + N + sb * N / G
    expect = {
        "cpu_ref_128x4096": 3_694_592,
        "prefill_4096x4096": 117_972_992,
        "dsv3_16384x7168": 825_767_936,
        "decode_1x8192": 73_984,
        "decode_4x8192": 246_784,
        "decode_16x8192": 937_984,
        "decode_32x8192": 1_859_584,
        "ue8m0_8192x5120": 293_939_200,
    }
    for name, b in expect.items():
        assert CONFIGS[name].algorithmic_bytes() == b, name
    w = CONFIGS["dsv3_16384x7168"]
    assert w.algorithmic_bytes(with_norm=True) == 825_767_936 + 2 * w.M * w.D


def test_reference_mode_workloads(pkg):
    """The 4-output workloads count norm_out (2 B per element) by default."""
    from fagq_mi355x.workloads import REFERENCE_MODE_CONFIGS
    w = REFERENCE_MODE_CONFIGS["ref4_16384x7168"]
    N = w.M * w.D
    assert w.norm and w.out_dtype == torch.int8 and w.rounding == "trunc"
    assert not w.scale_col_major and not w.scale_ue8m0
    assert w.algorithmic_bytes() == 9 * N + 2 * w.D + 4 * N // 128
    assert w.algorithmic_bytes(with_norm=False) == 7 * N + 2 * w.D + 4 * N // 128


def test_inputs_are_deterministic_and_shaped(pkg):
    from fagq_mi355x.workloads import CONFIGS, make_inputs
    w = CONFIGS["cpu_ref_128x4096"]
    a = make_inputs(w)
    b = make_inputs(w)
    for t, u in zip(a, b):
        assert t.dtype == torch.bfloat16 and torch.equal(t, u)
    assert a[0].shape == (128, 4096) and a[2].shape == (4096,)
    small = make_inputs(w, M=16)
    assert small[0].shape == (16, 4096) and torch.equal(small[0], make_inputs(w, M=16)[0])


def test_outlier_channels(pkg):
    from fagq_mi355x.workloads import CONFIGS, make_inputs, outlier_channels
    w = CONFIGS["dsv3_16384x7168"]
    ch = outlier_channels(w.D, w.seed)
    assert ch.numel() == 72 and ch.unique().numel() == 72
    x, res, _ = make_inputs(w, M=64)
    col_rms = x.float().pow(2).mean(0).sqrt()
    mask = torch.zeros(w.D, dtype=torch.bool)
    mask[ch] = True
    assert col_rms[mask].min() > 20 and col_rms[~mask].max() < 2


def test_student_t_inputs_have_heavy_tails(pkg):
    from fagq_mi355x.workloads import CONFIGS, make_inputs
    x, _, _ = make_inputs(CONFIGS["ue8m0_8192x5120"], M=256)
    xf = x.float()
    kurt = ((xf - xf.mean()) ** 4).mean() / xf.var() ** 2
    assert kurt > 6      # a normal distribution has 3
