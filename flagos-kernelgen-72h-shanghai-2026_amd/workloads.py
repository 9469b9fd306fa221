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

    @property
    def groups(self) -> int:
        return self.D // self.group_size

    @property
    def scale_bytes(self) -> int:
        return 1 if self.scale_ue8m0 else 4

    def algorithmic_bytes(self, with_norm: bool = False) -> int:
        """HBM bytes one call must move: read x, residual (2 B each per element)
        and gamma once; write residual_out (2 B), codes (1 B) and scales."""
        N = self.M * self.D
        b = 4 * N + 2 * self.D + 2 * N + N + self.scale_bytes * self.M * self.groups
        return b + (2 * N if with_norm else 0)


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


def outlier_channels(D: int, seed: int) -> torch.Tensor:
    """The fixed 1 % of hidden channels (round(0.01 * D)) scaled by 50."""
    g = torch.Generator(device="cpu").manual_seed(seed + 7919)
    k = max(1, round(0.01 * D))
    return torch.randperm(D, generator=g)[:k].sort().values


def make_inputs(w: Workload, M: int | None = None):
    """(x, residual, weight) bf16 CPU tensors for workload ``w``.  ``M``
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
    return x.to(torch.bfloat16), res.to(torch.bfloat16), weight.to(torch.bfloat16)
