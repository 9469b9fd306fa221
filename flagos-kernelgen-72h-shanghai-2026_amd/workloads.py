"""Seeded synthetic inputs for the operator's benchmark configurations.

All values are drawn in fp32 from a CPU ``torch.Generator`` in the order
x, residual, weight (then any extra draws), and cast to bf16, so the same
seed gives the same bytes on every machine.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    M: int
    D: int
    group_size: int = 128
    out_dtype: torch.dtype = torch.float8_e4m3fn
    scale_col_major: bool = False
    scale_ue8m0: bool = False
    rounding: str = "rne"            # int8 only
    dist: str = "normal"             # "normal" | "outliers" | "student_t"
    eps: float = 1e-6
    seed: int = 0
    act: torch.dtype = torch.bfloat16     # x and weight (the typed form: fp16 or fp32 too)
    res: torch.dtype = torch.bfloat16     # residual and residual_out
    norm: bool = False                    # norm_out written too (the 4-output form)

    @property
    def groups(self) -> int:
        return self.D // self.group_size

    @property
    def scale_bytes(self) -> int:
        return 1 if self.scale_ue8m0 else 4

    def algorithmic_bytes(self, with_norm: bool | None = None) -> int:
        """HBM bytes one call must move: read x, residual (2 B each per bf16
        element) and gamma once; write residual_out, codes (1 B) and scales,
        and norm_out in the 4-output form (with_norm, default: the workload's)."""
        with_norm = self.norm if with_norm is None else with_norm
        N = self.M * self.D
        ba, br = self.act.itemsize, self.res.itemsize
        b = (ba + br) * N + ba * self.D + br * N + N + self.scale_bytes * self.M * self.groups
        return b + (ba * N if with_norm else 0)


# The benchmark configurations (BASELINE.json "configs", in order).
CONFIGS = {
    "cpu_ref_128x4096": Workload("cpu_ref_128x4096", 128, 4096),
    "prefill_4096x4096": Workload("prefill_4096x4096", 4096, 4096),
    "dsv3_16384x7168": Workload("dsv3_16384x7168", 16384, 7168, scale_col_major=True,
                                dist="outliers"),
    "decode_1x8192": Workload("decode_1x8192", 1, 8192, out_dtype=torch.int8),
    "decode_4x8192": Workload("decode_4x8192", 4, 8192, out_dtype=torch.int8),
    "decode_16x8192": Workload("decode_16x8192", 16, 8192, out_dtype=torch.int8),
    "decode_32x8192": Workload("decode_32x8192", 32, 8192, out_dtype=torch.int8),
    "ue8m0_8192x5120": Workload("ue8m0_8192x5120", 8192, 5120, scale_col_major=True,
                                scale_ue8m0=True, dist="student_t"),
}

HEADLINE = "dsv3_16384x7168"

# The headline shape through the typed form (fagq_launch_typed): fp16 tensors,
# and bf16 activations with an fp32 residual stream.  Not BASELINE configs.
TYPED_CONFIGS = {
    "f16_16384x7168": Workload("f16_16384x7168", 16384, 7168, scale_col_major=True,
                               dist="outliers", act=torch.float16, res=torch.float16),
    "bf16_r32_16384x7168": Workload("bf16_r32_16384x7168", 16384, 7168, scale_col_major=True,
                                    dist="outliers", res=torch.float32),
}

# The reference operator's own output mode (task01.py:1731-1741, :112-116):
# norm_out written (4 outputs), int8 codes by truncation toward zero, fp32
# row-major scales.  Not BASELINE configs.
REFERENCE_MODE_CONFIGS = {
    "ref4_16384x7168": Workload("ref4_16384x7168", 16384, 7168, out_dtype=torch.int8,
                                rounding="trunc", dist="outliers", norm=True),
    "ref4_4096x4096": Workload("ref4_4096x4096", 4096, 4096, out_dtype=torch.int8,
                               rounding="trunc", norm=True),
}


def outlier_channels(D: int, seed: int) -> torch.Tensor:
    """The fixed 1 % of hidden channels (round(0.01 * D)) scaled by 50."""
    g = torch.Generator(device="cpu").manual_seed(seed + 7919)
    k = max(1, round(0.01 * D))
    return torch.randperm(D, generator=g)[:k].sort().values


def make_inputs(w: Workload, M: int | None = None):
    """(x, residual, weight) CPU tensors for workload ``w`` (bf16, or the
    workload's typed-form element types).  ``M``
    overrides the row count: same distributions and seed, but a different
    draw (weight is drawn after x and residual)."""
    M = w.M if M is None else M
    g = torch.Generator(device="cpu").manual_seed(w.seed)
    if w.dist == "student_t":
        def draw(shape):
            z = torch.randn(shape, generator=g)
            chi2 = sum(torch.randn(shape, generator=g) ** 2 for _ in range(3))
            return 0.5 * z / torch.sqrt(chi2 / 3.0)
    else:
        def draw(shape):
            return torch.randn(shape, generator=g)
    x = draw((M, w.D))
    res = draw((M, w.D))
    weight = 1.0 + 0.1 * torch.randn(w.D, generator=g)
    if w.dist == "outliers":
        ch = outlier_channels(w.D, w.seed)
        x[:, ch] *= 50.0
        res[:, ch] *= 50.0
    return x.to(w.act), res.to(w.res), weight.to(w.act)


# ------------------------------------------------------------- GEMM consumer

@dataclass(frozen=True)
class GemmWorkload:
    """The fp8 block-scaled GEMM fed by the quantizer: A [M, K] fp8 codes with 1 x 128
    scales (column-major [K/128, M] physical), B [N, K] fp8 with 128 x 128 block scales."""
    name: str
    M: int
    N: int
    K: int
    a_scale: str = "f32"       # "f32" | "ue8m0"
    b_scale: str = "f32"
    seed: int = 0

    def flops(self) -> int:
        return 2 * self.M * self.N * self.K

    def min_bytes(self) -> int:
        """Bytes that must cross HBM at least once: A, B, their scales, C (bf16)."""
        sa = 4 if self.a_scale == "f32" else 1
        sb = 4 if self.b_scale == "f32" else 1
        kb = self.K // 128
        return (self.M * self.K + self.N * self.K + sa * self.M * kb
                + sb * ((self.N + 127) // 128) * kb + 2 * self.M * self.N)


# DeepSeek-V3 shapes whose input is the headline quantizer's output (16384 tokens, hidden
# 7168): an expert / shared-expert gate+up projection (N = 2 x 2048) with fp32 or UE8M0
# scales, and the fused q_a + kv_a projection (N = 1536 + 576).
GEMM_CONFIGS = {
    "gemm_dsv3_16384x4096x7168": GemmWorkload("gemm_dsv3_16384x4096x7168", 16384, 4096, 7168),
    "gemm_dsv3_ue8m0_16384x4096x7168": GemmWorkload("gemm_dsv3_ue8m0_16384x4096x7168", 16384,
                                                    4096, 7168, "ue8m0", "ue8m0"),
    "gemm_qkva_16384x2112x7168": GemmWorkload("gemm_qkva_16384x2112x7168", 16384, 2112, 7168),
}


def make_gemm_inputs(w: GemmWorkload, M: int | None = None):
    """(a_q, a_scale, b_q, b_scale) CPU tensors: fp8 codes spread over the e4m3fn range
    (normal, sigma 56, clamped to +-448), scales exp(U(-12, 2)) (fp32) or biased
    exponents in [100, 140) (UE8M0).  a_scale is the physical [K/128, M] array."""
    M = w.M if M is None else M
    g = torch.Generator(device="cpu").manual_seed(w.seed)
    kb, nb = w.K // 128, (w.N + 127) // 128

    def codes(shape):
        return (torch.randn(shape, generator=g) * 56.0).clamp_(-448.0, 448.0).to(torch.float8_e4m3fn)

    def scales(shape, fmt):
        if fmt == "f32":
            return torch.exp(torch.empty(shape).uniform_(-12.0, 2.0, generator=g))
        return torch.randint(100, 140, shape, generator=g, dtype=torch.uint8)

    a_q = codes((M, w.K))
    b_q = codes((w.N, w.K))
    a_s = scales((kb, M), w.a_scale)
    b_s = scales((nb, kb), w.b_scale)
    return a_q, a_s, b_q, b_s


# --------------------------------------------- multi-input form (TP epilogue)

@dataclass(frozen=True)
class PartsWorkload:
    """The multi-input form at one rank's shard of a tensor-parallel layer: nparts
    partial tensors [M, D] (one per rank) summed before the residual."""
    name: str
    M: int
    D: int
    nparts: int
    group_size: int = 128
    seed: int = 0

    def algorithmic_bytes(self) -> int:
        """Read nparts partials, residual (bf16) and gamma; write residual_out
        (bf16), fp8 codes and fp32 scales."""
        N = self.M * self.D
        return (2 * self.nparts * N + 2 * N + 2 * self.D + 2 * N + N
                + 4 * self.M * (self.D // self.group_size))


# DeepSeek-V3 width at the headline batch, sharded over 8 ranks: each rank
# reduces and normalizes 16384 / 8 = 2048 rows from 8 partial sums.
PARTS_CONFIGS = {
    "tp8_shard_2048x7168": PartsWorkload("tp8_shard_2048x7168", 2048, 7168, 8),
    "tp4_shard_4096x7168": PartsWorkload("tp4_shard_4096x7168", 4096, 7168, 4),
}


def make_parts_inputs(w: PartsWorkload):
    """(parts, residual, weight) bf16 CPU tensors: partial sums N(0, 1/nparts)
    (so their sum is ~N(0, 1)), residual N(0, 1), weight 1 + 0.1 N(0, 1)."""
    g = torch.Generator(device="cpu").manual_seed(w.seed)
    sd = 1.0 / w.nparts ** 0.5
    parts = [(sd * torch.randn(w.M, w.D, generator=g)).to(torch.bfloat16)
             for _ in range(w.nparts)]
    res = torch.randn(w.M, w.D, generator=g).to(torch.bfloat16)
    weight = (1.0 + 0.1 * torch.randn(w.D, generator=g)).to(torch.bfloat16)
    return parts, res, weight


# ------------------------------------------ Task 02: DSA top-k page table

@dataclass(frozen=True)
class DsaWorkload:
    """scores[B, H, Q, NB] -> top_k block ids and pages per query row."""
    name: str
    B: int
    H: int
    Q: int
    NB: int
    top_k: int
    block_size: int
    dtype: torch.dtype = torch.float32
    seed: int = 0
    full_rows: bool = False        # every query sees all NB blocks (decode-like)

    @property
    def rows(self) -> int:
        return self.B * self.H * self.Q

    def algorithmic_bytes(self, valid_blocks_total: int) -> int:
        """Scores of the valid prefixes (read once), two int32 outputs per
        rank, one int32 page-table read per written page, q_pos/kv_lens."""
        esz = 2 if self.dtype == torch.bfloat16 else 4
        return (esz * valid_blocks_total + 12 * self.rows * self.top_k
                + 4 * self.B * self.Q + 4 * self.B)


def _dsa(B, H, Q, NB, K, BS, dtype=torch.float32, full_rows=False):
    tag = "bf16" if dtype == torch.bfloat16 else "f32"
    name = f"dsa_{tag}_b{B}h{H}q{Q}_nb{NB}_k{K}_bs{BS}" + ("_full" if full_rows else "")
    return name, DsaWorkload(name, B, H, Q, NB, K, BS, dtype, full_rows=full_rows)


# The (B, H, Q, NB, top_k, block_size) shapes the reference routes
# (src/task02_dsa_topk_page_table_transform.py:1668-1672), fp32 scores.
DSA_CONFIGS = dict(_dsa(*c) for c in [
    (2, 32, 512, 4096, 128, 64), (1, 32, 1024, 4096, 128, 64), (4, 16, 512, 4096, 128, 64),
    (1, 32, 512, 2048, 64, 128), (2, 16, 512, 2048, 64, 128), (1, 32, 1024, 2048, 64, 64),
    (1, 8, 128, 512, 32, 128), (2, 8, 128, 512, 32, 128), (1, 16, 256, 1024, 32, 128),
    (2, 16, 256, 1024, 64, 128),
])
DSA_CONFIGS.update(dict([_dsa(2, 32, 512, 4096, 128, 64, torch.bfloat16),
                         # all rows valid: the worst-case traffic R (4 NB + 12 K) bytes
                         # (reports/task02_dsa_topk_page_table_transform.md:33-36)
                         _dsa(2, 32, 512, 4096, 128, 64, full_rows=True),
                         # top_k past 256: the reference's power-of-two top_k up to its
                         # 1024-block chunk (task02.py:913-945, :1712-1725)
                         _dsa(2, 32, 512, 4096, 512, 64), _dsa(2, 32, 512, 4096, 1024, 64)]))
DSA_HEADLINE = "dsa_f32_b2h32q512_nb4096_k128_bs64"


def make_dsa_inputs(w: DsaWorkload):
    """(scores, page_table, q_pos, kv_lens) CPU tensors.  Scores N(0, 1) in the
    workload's dtype; kv_len[b] = NB * block_size - 3 b block_size (at least 1);
    query q of batch b at position (q + 1) kv_len / Q - 1, so the causal prefixes
    of a batch's rows spread evenly from ~kv_len/Q to kv_len tokens;
    page_table[b] a random permutation of physical pages b * NB ...  int32.
    With full_rows every kv_len is NB * block_size and every query sits at
    the last position, so each row selects from all NB blocks."""
    g = torch.Generator(device="cpu").manual_seed(w.seed)
    scores = torch.randn(w.B, w.H, w.Q, w.NB, generator=g).to(w.dtype)
    if w.full_rows:
        kv = torch.full((w.B,), w.NB * w.block_size, dtype=torch.int32)
        q_pos = (kv[:, None] - 1).expand(w.B, w.Q).contiguous()
    else:
        kv = torch.tensor([max(1, w.NB * w.block_size - 3 * b * w.block_size)
                           for b in range(w.B)], dtype=torch.int32)
        q = torch.arange(w.Q, dtype=torch.int64)
        q_pos = torch.stack([((q + 1) * int(kv[b]) // w.Q - 1) for b in range(w.B)]).to(torch.int32)
    page_table = torch.stack([b * w.NB + torch.randperm(w.NB, generator=g)
                              for b in range(w.B)]).to(torch.int32)
    return scores, page_table, q_pos, kv


def dsa_valid_blocks(w: DsaWorkload, q_pos: torch.Tensor, kv_lens: torch.Tensor) -> int:
    """Total selectable-prefix length over all rows (the blocks a kernel must read)."""
    kv = kv_lens.to(torch.int64)
    vb = torch.clamp((kv + w.block_size - 1) // w.block_size, max=w.NB)          # [B]
    pos = q_pos.to(torch.int64)
    last = torch.minimum(torch.where(pos >= 0, pos // w.block_size, torch.full_like(pos, -1)),
                         (vb - 1)[:, None])
    per_row = torch.clamp(last + 1, min=0)                                         # [B, Q]
    return int(per_row.sum()) * w.H


# ---------------------------------------------------------------- Task 03 MLA backward

@dataclass(frozen=True)
class MlaWorkload:
    """q, out, do [B, H, S, D], c_kv [B, S, D] bf16 -> dq, dc_kv."""
    name: str
    B: int
    H: int
    S: int
    D: int
    grad_dtype: torch.dtype = torch.bfloat16     # dq and dc_kv
    seed: int = 0

    @property
    def sm_scale(self) -> float:
        return self.D ** -0.5

    @property
    def exact_rows(self) -> int:
        return min(16, self.S)

    def algorithmic_bytes(self) -> int:
        """do read once, dq and dc written once, plus the exact rows' q, out, c
        and lse reads."""
        g = 2 if self.grad_dtype == torch.bfloat16 else 4
        n = self.B * self.H * self.S * self.D
        e = self.exact_rows
        return (2 * n + g * n + g * self.B * self.S * self.D
                + 4 * self.B * self.H * e * self.D + 2 * self.B * e * self.D
                + 4 * self.B * self.H * e)


def _mla(B, H, S, D, grad=torch.bfloat16):
    tag = "" if grad == torch.bfloat16 else "_f32grad"
    name = f"mla_b{B}h{H}s{S}d{D}{tag}"
    return name, MlaWorkload(name, B, H, S, D, grad)


# The reference's workloads: H = 64, D = 512, S in {256, ..., 4096}, up to B = 2
# (reports/task03_mla_bwd_nope_dkdv.md:27-33, :57).
MLA_CONFIGS = dict(_mla(2, 64, S, 512) for S in (256, 512, 1024, 2048, 4096))
MLA_CONFIGS.update(dict([_mla(2, 64, 4096, 512, torch.float32)]))
MLA_HEADLINE = "mla_b2h64s4096d512"


def make_mla_inputs(w: MlaWorkload, device="cpu"):
    """(q, c_kv, out, do, lse) on `device`: q, c_kv, do N(0, 1) in bf16.  The
    first exact_rows query rows of out and lse come from the causal forward
    with K = V = C (the only rows of out and lse the operator reads); the
    other rows of out are N(0, 0.05) and of lse log(i + 1)."""
    g = torch.Generator(device=device).manual_seed(w.seed)
    B, H, S, D, E = w.B, w.H, w.S, w.D, w.exact_rows
    q = torch.randn(B, H, S, D, generator=g, device=device).to(torch.bfloat16)
    c = torch.randn(B, S, D, generator=g, device=device).to(torch.bfloat16)
    do = torch.randn(B, H, S, D, generator=g, device=device).to(torch.bfloat16)
    out = (torch.randn(B, H, S, D, generator=g, device=device) * 0.05).to(torch.bfloat16)
    lse = torch.log(torch.arange(1, S + 1, device=device, dtype=torch.float32)).expand(B, H, S)
    lse = lse.contiguous()
    qe, ce = q[:, :, :E].double(), c[:, :E].double()
    logits = torch.einsum("bhsd,btd->bhst", qe, ce) * w.sm_scale
    logits = logits.masked_fill(~torch.ones(E, E, dtype=torch.bool, device=device).tril(),
                                float("-inf"))
    lse[:, :, :E] = torch.logsumexp(logits, -1).float()
    out[:, :, :E] = torch.einsum("bhst,btd->bhsd", torch.softmax(logits, -1), ce).to(torch.bfloat16)
    return q, c, out, do, lse
