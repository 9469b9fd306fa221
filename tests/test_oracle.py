"""Pins the CPU oracle (oracle/fagq_oracle.c) before it is trusted as the
checker: number-format encoders against PyTorch's own casts (exhaustively
over the ranges that matter), closed-form known answers, mathematical
invariants of the operator, and agreement of the two independent
restatements (C and eager PyTorch).  CPU only."""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle.torch_eager import fagq_torch


def bits_to_f32(u):
    return np.asarray(u, dtype=np.uint32).view(np.float32)


def binade(e: int) -> np.ndarray:
    """Every fp32 in [2^e, 2^(e+1)) and its negation."""
    base = np.uint32((e + 127) << 23)
    u = base | np.arange(1 << 23, dtype=np.uint32)
    return np.concatenate([u, u | np.uint32(0x80000000)]).view(np.float32)


# ----------------------------------------------------------------- encoders

def test_e4m3fn_matches_torch_cast_exhaustively():
    """All fp32 in the binades 2^-12 .. 2^9 (subnormals, every normal binade,
    the 448..464 round-down and >= 464 overflow) against torch's cast."""
    for e in range(-12, 10):
        f = binade(e)
        ours = oracle.e4m3fn_raw(f)
        ref = torch.from_numpy(f).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        both_nan = ((ours & 0x7F) == 0x7F) & ((ref & 0x7F) == 0x7F)
        bad = (ours != ref) & ~both_nan
        assert not bad.any(), (e, f[bad][:4], ours[bad][:4], ref[bad][:4])


def test_e4m3fn_tiny_values_round_to_zero():
    rng = np.random.default_rng(1)
    u = rng.integers(0, (127 - 12) << 23, size=1 << 20, dtype=np.uint32)   # |v| < 2^-12
    f = np.concatenate([bits_to_f32(u), -bits_to_f32(u), np.float32([0.0, -0.0])])
    ours = oracle.e4m3fn_raw(f)
    ref = torch.from_numpy(f).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    assert set(np.unique(ours & 0x7F).tolist()) == {0}


@pytest.mark.parametrize("v,code", [
    (448.0, 0x7E), (-448.0, 0xFE), (1.0, 0x38), (2.0 ** -6, 0x08), (2.0 ** -9, 0x01),
    (2.0 ** -10, 0x00),            # tie between 0 and 2^-9 -> even (0)
    (1.5 * 2.0 ** -10, 0x01), (1.0625, 0x38),   # tie between 1.0 and 1.125 -> 1.0
    (1.1875, 0x3A),                # tie between 1.125 and 1.25 -> 1.25 (even mantissa)
    (464.0, 0x7E), (500.0, 0x7E),  # the operator clamps to 448 first
])
def test_e4m3fn_known_answers_after_clamp(v, code):
    assert int(oracle.encode(np.float32([v]), oracle.Q_FP8)[0]) == code


def test_int8_rne_and_trunc_match_torch():
    parts = [binade(e) for e in range(-2, 7)]                # |v| in [0.25, 128)
    rng = np.random.default_rng(2)
    parts.append(rng.uniform(-130, 130, size=1 << 20).astype(np.float32))
    halves = np.arange(-127, 128, dtype=np.float64) + 0.5
    parts.append(np.concatenate([halves, np.nextafter(halves, 0), np.nextafter(halves, 200)]).astype(np.float32))
    f = np.concatenate(parts)
    t = torch.from_numpy(f).clamp(-127.0, 127.0)
    rne = oracle.encode(f, oracle.Q_INT8, oracle.R_RNE).view(np.int8)
    assert np.array_equal(rne, torch.round(t).to(torch.int8).numpy())
    tr = oracle.encode(f, oracle.Q_INT8, oracle.R_TRUNC).view(np.int8)
    assert np.array_equal(tr, t.to(torch.int8).numpy())
    assert np.array_equal(tr, torch.trunc(t).to(torch.int8).numpy())


@pytest.mark.parametrize("v,rne,trunc", [
    (0.5, 0, 0), (1.5, 2, 1), (2.5, 2, 2), (-0.5, 0, 0), (-1.5, -2, -1), (126.5, 126, 126),
    (127.4, 127, 127), (130.0, 127, 127), (-1e30, -127, -127), (1.9, 2, 1), (-1.9, -2, -1),
])
def test_int8_known_answers(v, rne, trunc):
    f = np.float32([v])
    assert int(oracle.encode(f, oracle.Q_INT8, oracle.R_RNE).view(np.int8)[0]) == rne
    assert int(oracle.encode(f, oracle.Q_INT8, oracle.R_TRUNC).view(np.int8)[0]) == trunc


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(3)
    u = rng.integers(0, 1 << 32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 1 << 16, size=1 << 20, dtype=np.uint32) << 16) | np.uint32(0x8000)
    f = np.concatenate([bits_to_f32(u), bits_to_f32(ties)])
    f = f[np.isfinite(f)]
    ours = oracle.bf16_from_f32(f)
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.uint16).numpy()
    assert np.array_equal(ours, ref)
    nan = oracle.bf16_from_f32(np.float32([np.nan]))
    assert (int(nan[0]) & 0x7F80) == 0x7F80 and (int(nan[0]) & 0x7F) != 0


def test_ceil_log2_brute_force():
    rng = np.random.default_rng(4)
    u = rng.integers(1 << 23, 255 << 23, size=1 << 20, dtype=np.uint32)     # positive normals
    s = bits_to_f32(u)
    e = oracle.ceil_log2(s).astype(np.int64)
    sd = s.astype(np.float64)
    assert np.all(np.ldexp(1.0, e - 1) < sd) and np.all(sd <= np.ldexp(1.0, e))


@pytest.mark.parametrize("k", [-40, -1, 0, 1, 7, 100])
def test_ceil_log2_known_answers(k):
    p = np.float32(2.0 ** k)
    above = np.nextafter(p, np.float32(np.inf))
    assert int(oracle.ceil_log2(np.float32([p]))[0]) == k
    assert int(oracle.ceil_log2(np.float32([above]))[0]) == k + 1
    assert int(oracle.ceil_log2(np.float32([1e-12]))[0]) == -39   # 2^-40 < 1e-12 < 2^-39


# ----------------------------------------------------------------- operator

FMT = {
    "fp8": (oracle.Q_FP8, oracle.R_RNE, 448.0),
    "int8_rne": (oracle.Q_INT8, oracle.R_RNE, 127.0),
    "int8_trunc": (oracle.Q_INT8, oracle.R_TRUNC, 127.0),
}


def bf16(a) -> np.ndarray:
    return oracle.bf16_from_f32(np.asarray(a, dtype=np.float32))


def run(x, r, g, G=128, fmt="fp8", ue8m0=False, col=False, eps=1e-6, with_norm=False):
    qf, rnd, _ = FMT[fmt]
    return oracle.fagq(x, r, g, eps, G, qf, oracle.S_UE8M0 if ue8m0 else oracle.S_F32,
                       oracle.L_COL if col else oracle.L_ROW, rnd, with_norm)


def decode_codes(q, fmt):
    if fmt == "fp8":
        return torch.from_numpy(q.copy()).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    return q.view(np.int8).astype(np.float64)


def math_norm(x, r, g, eps):
    """n = (x + r) * g / sqrt(mean((x + r)^2) + eps) in float64 (the spec, not the op order)."""
    rr = oracle.f32_from_bf16(x).astype(np.float64) + oracle.f32_from_bf16(r).astype(np.float64)
    inv = 1.0 / np.sqrt((rr * rr).mean(axis=1, keepdims=True) + eps)
    return rr * oracle.f32_from_bf16(g).astype(np.float64) * inv


def random_inputs(M, D, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    x = bf16(scale * rng.standard_normal((M, D)))
    r = bf16(scale * rng.standard_normal((M, D)))
    g = bf16(1.0 + 0.1 * rng.standard_normal(D))
    return x, r, g


@pytest.mark.parametrize("fmt", list(FMT))
@pytest.mark.parametrize("ue8m0", [False, True])
def test_one_hot_row(fmt, ue8m0):
    M, D, G = 3, 1024, 128
    x = np.zeros((M, D), np.uint16)
    r = np.zeros((M, D), np.uint16)
    cols = [5, 300, 1023]
    vals = [3.0, -0.25, 1000.0]
    for m, (c, v) in enumerate(zip(cols, vals)):
        x[m, c] = bf16([v])[0]
    g = bf16(np.ones(D))
    out = run(x, r, g, G, fmt, ue8m0)
    qmax = FMT[fmt][2]
    codes = decode_codes(out["q"], fmt)
    floor_byte = 127 + int(oracle.ceil_log2(np.float32([1e-12]))[0])
    for m, (c, v) in enumerate(zip(cols, vals)):
        assert out["residual_out"][m, c] == x[m, c]
        expect = np.zeros(D)
        expect[c] = math.copysign(qmax, v)
        if ue8m0:   # scale is the next power of two >= |v| inv / 448 -> |code| <= qmax
            assert qmax / 2 - 1 <= abs(codes[m, c]) <= qmax
            codes[m, c] = expect[c]
        assert np.array_equal(codes[m], expect), (m, codes[m][codes[m] != 0])
        others = [gg for gg in range(D // G) if gg != c // G]
        if ue8m0:
            assert np.all(out["scale"][m, others] == floor_byte)
        else:
            assert np.all(out["scale"][m, others] == np.float32(1e-12))


@pytest.mark.parametrize("fmt", list(FMT))
def test_zero_rows(fmt):
    x = np.zeros((2, 512), np.uint16)
    out = run(x, x, bf16(np.ones(512)), 128, fmt)
    assert not out["residual_out"].any()
    assert np.all(decode_codes(out["q"], fmt) == 0)
    assert np.all(out["scale"] == np.float32(1e-12))


@pytest.mark.parametrize("c", [0.001, 0.5, 3.0, 250.0])
@pytest.mark.parametrize("D", [512, 4096, 7168])
def test_constant_row_closed_form(c, D):
    """x = c, residual = 0, gamma = 1: inv = 1/sqrt(c^2 + eps), so every scale is
    |c| / sqrt(c^2 + eps) / 448 and every code is +-448."""
    eps = 1e-6
    cb = float(oracle.f32_from_bf16(bf16([c]))[0])
    x = np.full((2, D), bf16([c])[0], np.uint16)
    x[1] = bf16([-c])[0]
    out = run(x, np.zeros_like(x), bf16(np.ones(D)), 128, "fp8", eps=eps)
    expect = cb / math.sqrt(cb * cb + eps) / 448.0
    rel = np.abs(out["scale"].astype(np.float64) - expect) / expect
    assert rel.max() < 1e-6
    codes = decode_codes(out["q"], "fp8")
    assert np.all(codes[0] == 448.0) and np.all(codes[1] == -448.0)


def test_gamma_is_applied_before_the_group_max():
    """Scaling gamma by 2 (exact) doubles every scale and leaves every code."""
    x, r, g = random_inputs(8, 2048, 5)
    g2 = bf16(oracle.f32_from_bf16(g) * 2.0)
    a, b = run(x, r, g), run(x, r, g2)
    assert np.array_equal(a["q"], b["q"])
    assert np.array_equal(b["scale"], a["scale"] * np.float32(2.0))


def test_rms_normalisation_is_scale_invariant():
    """With eps = 0, scaling x and residual by 2^k changes residual_out by 2^k
    and leaves codes and scales unchanged."""
    x, r, g = random_inputs(8, 2048, 6)
    k = 8.0
    x2 = bf16(oracle.f32_from_bf16(x) * k)
    r2 = bf16(oracle.f32_from_bf16(r) * k)
    a, b = run(x, r, g, eps=0.0), run(x2, r2, g, eps=0.0)
    assert np.array_equal(a["q"], b["q"])
    assert np.array_equal(a["scale"], b["scale"])
    assert np.array_equal(oracle.f32_from_bf16(b["residual_out"]), oracle.f32_from_bf16(a["residual_out"]) * k)


@pytest.mark.parametrize("G", [64, 128, 256])
@pytest.mark.parametrize("fmt", ["fp8", "int8_rne"])
def test_dequantisation_error_bounds(G, fmt):
    """Against the float64 mathematics: every group's largest element maps to
    +-QMAX, and |q * s - n| is within half a code step."""
    M, D, eps = 16, 2048, 1e-6
    x, r, g = random_inputs(M, D, 7)
    out = run(x, r, g, G, fmt, eps=eps, with_norm=True)
    n = math_norm(x, r, g, eps)
    s = out["scale"].astype(np.float64)                      # [M, groups]
    q = decode_codes(out["q"], fmt)
    qmax = FMT[fmt][2]
    ng = n.reshape(M, D // G, G)
    qg = q.reshape(M, D // G, G)
    assert np.allclose(s, np.abs(ng).max(axis=2) / qmax, rtol=2e-6)
    assert np.all(np.abs(qg).max(axis=2) == qmax)
    deq = qg * s[..., None]
    if fmt == "int8_rne":
        bound = 0.5 * s[..., None] * (1 + 1e-5)
    else:   # 3 mantissa bits: half a step is 2^-4 relative; subnormal step 2^-9
        bound = np.maximum(np.abs(ng) * 2.0 ** -4, 2.0 ** -10 * s[..., None]) * (1 + 1e-5)
    assert np.all(np.abs(deq - ng) <= bound + 1e-12)
    norm = oracle.f32_from_bf16(out["norm_out"]).astype(np.float64)
    assert np.all(np.abs(norm - n) <= np.abs(n) * 2.0 ** -8 + 1e-30)


def test_ue8m0_scale_is_the_next_power_of_two():
    M, D, eps = 16, 2048, 1e-6
    x, r, g = random_inputs(M, D, 8, scale=3.0)
    a = run(x, r, g, 128, "fp8", ue8m0=False, eps=eps)
    u = run(x, r, g, 128, "fp8", ue8m0=True, eps=eps)
    e = u["scale"].astype(np.int64) - 127
    s = a["scale"].astype(np.float64)
    assert np.all(np.ldexp(1.0, e - 1) < s) and np.all(s <= np.ldexp(1.0, e))
    n = math_norm(x, r, g, eps).reshape(M, D // 128, 128)
    q = decode_codes(u["q"], "fp8").reshape(M, D // 128, 128)
    deq = q * np.ldexp(1.0, e)[..., None]
    bound = np.maximum(np.abs(n) * 2.0 ** -4, 2.0 ** -10 * np.ldexp(1.0, e)[..., None]) * (1 + 1e-5)
    assert np.all(np.abs(deq - n) <= bound)


def test_column_major_is_the_transpose():
    x, r, g = random_inputs(12, 1024, 9)
    for ue in (False, True):
        a, b = run(x, r, g, ue8m0=ue, col=False), run(x, r, g, ue8m0=ue, col=True)
        assert np.array_equal(a["scale"].T, b["scale"])
        assert np.array_equal(a["q"], b["q"])


def test_trunc_rounds_toward_zero_of_rne():
    x, r, g = random_inputs(8, 2048, 10)
    a = run(x, r, g, fmt="int8_rne")["q"].view(np.int8).astype(np.int32)
    b = run(x, r, g, fmt="int8_trunc")["q"].view(np.int8).astype(np.int32)
    assert np.all(np.abs(b) <= np.abs(a)) and np.all(np.abs(a - b) <= 1)
    assert np.count_nonzero(a != b) > 0.3 * a.size     # about half the codes differ


@pytest.mark.parametrize("case", [
    (64, 4096, 128, torch.float8_e4m3fn, False, False, "rne", False),
    (33, 7168, 128, torch.float8_e4m3fn, False, True, "rne", True),
    (17, 8192, 128, torch.int8, False, False, "rne", True),
    (9, 5120, 128, torch.float8_e4m3fn, True, True, "rne", False),
    (20, 4096, 256, torch.int8, False, False, "trunc", True),
    (5, 1024, 64, torch.int8, True, False, "trunc", False),
])
def test_c_and_eager_restatements_agree(case):
    M, D, G, qd, ue, col, rnd, wn = case
    gen = torch.Generator().manual_seed(M * D)
    x = (3 * torch.randn(M, D, generator=gen)).bfloat16()
    r = torch.randn(M, D, generator=gen).bfloat16()
    w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    outs = fagq_torch(x, r, w, 1e-6, G, qd, ue, col, rnd, wn)
    o = oracle.fagq(x.view(torch.uint16).numpy(), r.view(torch.uint16).numpy(),
                    w.view(torch.uint16).numpy(), 1e-6, G,
                    oracle.Q_FP8 if qd == torch.float8_e4m3fn else oracle.Q_INT8,
                    oracle.S_UE8M0 if ue else oracle.S_F32, oracle.L_COL if col else oracle.L_ROW,
                    oracle.R_RNE if rnd == "rne" else oracle.R_TRUNC, wn)
    assert np.array_equal(outs[0].view(torch.uint16).numpy(), o["residual_out"])
    assert np.array_equal(outs[1].view(torch.uint8).numpy(), o["q"])
    assert np.array_equal(outs[2].numpy(), o["scale"])
    if wn:
        assert np.array_equal(outs[3].view(torch.uint16).numpy(), o["norm_out"])


def test_thread_count_does_not_change_results():
    x, r, g = random_inputs(37, 1536, 11)
    a = oracle.fagq(x, r, g, 1e-6, 128, nthreads=1)
    b = oracle.fagq(x, r, g, 1e-6, 128, nthreads=8)
    for k in a:
        assert np.array_equal(a[k], b[k])


# ----------------------------------------------------------------- typed form

def test_f16_decoder_matches_torch_exhaustively():
    """All 65536 fp16 bit patterns (subnormals, infinities, NaNs) against torch."""
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f32_from_f16(h)
    ref = torch.from_numpy(h.view(np.int16)).view(torch.float16).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours.view(np.uint32)[~nan], ref.view(np.uint32)[~nan])


def test_f16_encoder_matches_torch_cast():
    """fp32 -> fp16 round to nearest even against torch's cast: every fp32 in
    the binades around the subnormal range, the subnormal/normal boundary and
    the overflow edge (65504 .. 65520 .. inf), every tie between fp16
    neighbours in [1, 2), and 4 M random bit patterns."""
    parts = [binade(e) for e in (-26, -25, -24, -15, -14, 15, 16)]
    ties = (np.arange(1 << 10, dtype=np.uint32) << 13 | np.uint32(0x1000)) | np.uint32(127 << 23)
    rng = np.random.default_rng(8)
    u = rng.integers(0, 1 << 32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    parts += [bits_to_f32(ties), -bits_to_f32(ties), bits_to_f32(u),
              np.float32([65504.0, 65519.996, 65520.0, 70000.0, np.inf, -np.inf, 0.0, -0.0])]
    f = np.concatenate(parts)
    f = f[~np.isnan(f)]
    ours = oracle.f16_from_f32(f)
    ref = torch.from_numpy(f).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    bad = ours != ref
    assert not bad.any(), (f[bad][:4], ours[bad][:4], ref[bad][:4])
    nan = oracle.f16_from_f32(np.float32([np.nan]))
    assert (int(nan[0]) & 0x7C00) == 0x7C00 and (int(nan[0]) & 0x3FF) != 0


def run_typed(x, r, g, act, res, G=128, fmt="fp8", ue8m0=False, col=False, eps=1e-6,
              with_norm=False):
    qf, rnd, _ = FMT[fmt]
    return oracle.fagq_typed(x, r, g, eps, G, act, res, qf,
                             oracle.S_UE8M0 if ue8m0 else oracle.S_F32,
                             oracle.L_COL if col else oracle.L_ROW, rnd, with_norm)


@pytest.mark.parametrize("fmt", list(FMT))
@pytest.mark.parametrize("ue8m0,col", [(False, False), (True, True)])
def test_typed_bf16_pair_is_the_bf16_oracle(fmt, ue8m0, col):
    x, r, g = random_inputs(9, 3072, 11, scale=3.0)
    a = run(x, r, g, 128, fmt, ue8m0, col, with_norm=True)
    b = run_typed(x, r, g, oracle.DT_BF16, oracle.DT_BF16, 128, fmt, ue8m0, col, with_norm=True)
    for k in a:
        assert np.array_equal(a[k], b[k]), k


@pytest.mark.parametrize("act", [oracle.DT_BF16, oracle.DT_F16])
def test_f32_residual_stream_widens_exactly(act):
    """An fp32 residual stream holding exactly the widened 16-bit residual gives
    the same r, so the same codes, scales and norm_out as the 16-bit stream;
    residual_out is then r itself, which rounds to the 16-bit residual_out.
    Catches a residual loaded or stored with the wrong width or type."""
    rng = np.random.default_rng(12)
    M, D = 6, 2048
    enc = oracle.bf16_from_f32 if act == oracle.DT_BF16 else oracle.f16_from_f32
    dec = oracle.f32_from_bf16 if act == oracle.DT_BF16 else oracle.f32_from_f16
    x = enc(rng.standard_normal((M, D)).astype(np.float32))
    r16 = enc(rng.standard_normal((M, D)).astype(np.float32))
    g = enc((1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    a = run_typed(x, r16, g, act, act, with_norm=True)
    b = run_typed(x, dec(r16), g, act, oracle.DT_F32, with_norm=True)
    assert np.array_equal(a["q"], b["q"]) and np.array_equal(a["scale"], b["scale"])
    assert np.array_equal(a["norm_out"], b["norm_out"])
    r = dec(x) + dec(r16)
    assert np.array_equal(b["residual_out"].view(np.uint32), r.view(np.uint32))
    assert np.array_equal(enc(b["residual_out"]), a["residual_out"])


def test_f32_activations_match_f64_mathematics():
    """All-fp32 tensors: dequantized codes against the float64 mathematics of
    (x + r) * g / rms, within half a code step (catches a dropped /D, a wrong
    eps or a gamma applied after the maximum, without any 16-bit rounding)."""
    rng = np.random.default_rng(13)
    M, D, G, eps = 8, 1024, 128, 1e-6
    x = rng.standard_normal((M, D)).astype(np.float32)
    r = rng.standard_normal((M, D)).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    out = run_typed(x, r, g, oracle.DT_F32, oracle.DT_F32, G, "int8_rne", eps=eps, with_norm=True)
    rr = x.astype(np.float64) + r.astype(np.float64)
    n = rr * g.astype(np.float64) / np.sqrt((rr * rr).mean(axis=1, keepdims=True) + eps)
    s = out["scale"].astype(np.float64)
    assert np.allclose(s, np.abs(n.reshape(M, D // G, G)).max(axis=2) / 127.0, rtol=2e-6)
    deq = decode_codes(out["q"], "int8_rne").reshape(M, D // G, G) * s[..., None]
    assert np.all(np.abs(deq - n.reshape(M, D // G, G)) <= 0.5 * s[..., None] * (1 + 1e-5))
    assert np.allclose(out["norm_out"].astype(np.float64), n, rtol=1e-6, atol=1e-30)
    assert np.array_equal(out["residual_out"], (x + r).astype(np.float32))


def test_f16_constant_row_closed_form():
    """fp16 x = c, residual = 0, gamma = 1: every scale |c| / sqrt(c^2 + eps) / 448."""
    eps, D = 1e-6, 4096
    for c in (0.001, 0.5, 3.0, 250.0):
        cf = float(oracle.f32_from_f16(oracle.f16_from_f32(np.float32([c])))[0])
        x = np.full((1, D), oracle.f16_from_f32(np.float32([c]))[0], np.uint16)
        out = run_typed(x, np.zeros_like(x), oracle.f16_from_f32(np.ones(D, np.float32)),
                        oracle.DT_F16, oracle.DT_F16, eps=eps)
        expect = cf / math.sqrt(cf * cf + eps) / 448.0
        assert np.abs(out["scale"].astype(np.float64) - expect).max() / expect < 1e-6
