"""Parity comparator: GPU outputs vs the oracle (TEST INFRASTRUCTURE ONLY).

Tolerance (from the build's north star):
* residual_out (and norm_out): bit-exact bf16;
* fp32 scales: |gpu - ref| <= 1e-6 * |ref|;
* UE8M0 scale bytes: equal, except a +-1 exponent on at most 0.01 % of the
  groups (an fp32 scale within an ulp of a power of two); codes of such
  groups are then not compared;
* codes: equal, except differences of exactly one code step on at most
  0.01 % of the elements (rounding ties moved by a last-ulp difference).
Everything is also reported as exact-match counts, so a test can demand
bit-exactness where the two sides compute the same roundings.
"""
from __future__ import annotations

import numpy as np

CODE_TOL_FRAC = 1e-4
SCALE_RTOL = 1e-6


def fp8_ordinal(b: np.ndarray) -> np.ndarray:
    """Maps e4m3fn bytes to integers that are adjacent for adjacent values."""
    b = b.astype(np.int32)
    mag = b & 0x7F
    return np.where(b & 0x80, -mag, mag)


def int8_ordinal(b: np.ndarray) -> np.ndarray:
    return b.astype(np.uint8).view(np.int8).astype(np.int32)


class ParityError(AssertionError):
    pass


def compare(gpu: dict, ref: dict, *, fp8: bool, ue8m0: bool, code_tol_frac: float = CODE_TOL_FRAC,
            label: str = "") -> dict:
    """gpu/ref: dicts of numpy arrays with keys residual_out (uint16), q (uint8),
    scale (float32 or uint8, same physical layout on both sides) and
    optionally norm_out (uint16).  Raises ParityError outside the tolerance;
    returns statistics."""
    stats: dict = {"label": label}
    ro_g, ro_r = gpu["residual_out"], ref["residual_out"]
    if ro_g.shape != ro_r.shape:
        raise ParityError(f"{label}: residual_out shape {ro_g.shape} != {ro_r.shape}")
    bad = int(np.count_nonzero(ro_g != ro_r))
    stats["residual_out_mismatch"] = bad
    if bad:
        i = np.argwhere(ro_g != ro_r)[:5].tolist()
        raise ParityError(f"{label}: residual_out differs at {bad} elements, e.g. {i}")
    if "norm_out" in ref:
        bad = int(np.count_nonzero(gpu["norm_out"] != ref["norm_out"]))
        stats["norm_out_mismatch"] = bad
        if bad:
            i = np.argwhere(gpu["norm_out"] != ref["norm_out"])[:5].tolist()
            raise ParityError(f"{label}: norm_out differs at {bad} elements, e.g. {i}")

    sg, sr = gpu["scale"], ref["scale"]
    if sg.shape != sr.shape:
        raise ParityError(f"{label}: scale shape {sg.shape} != {sr.shape}")
    skip_groups = None
    if ue8m0:
        d = sg.astype(np.int32) - sr.astype(np.int32)
        nd = int(np.count_nonzero(d))
        stats["scale_mismatch"] = nd
        if np.any(np.abs(d) > 1) or nd > code_tol_frac * max(1, d.size):
            raise ParityError(f"{label}: ue8m0 scales differ at {nd} groups (max |d| "
                              f"{int(np.abs(d).max())})")
        skip_groups = d != 0
    else:
        rel = np.abs(sg.astype(np.float64) - sr.astype(np.float64)) / np.maximum(
            np.abs(sr.astype(np.float64)), np.finfo(np.float64).tiny)
        stats["scale_mismatch"] = int(np.count_nonzero(sg != sr))
        stats["scale_max_rel"] = float(rel.max()) if rel.size else 0.0
        if rel.size and rel.max() > SCALE_RTOL:
            i = np.unravel_index(int(rel.argmax()), rel.shape)
            raise ParityError(f"{label}: scale rel error {rel.max():.3e} at {i} "
                              f"(gpu {sg[i]!r}, ref {sr[i]!r})")

    qg, qr = gpu["q"], ref["q"]
    if qg.shape != qr.shape:
        raise ParityError(f"{label}: q shape {qg.shape} != {qr.shape}")
    ordf = fp8_ordinal if fp8 else int8_ordinal
    dq = np.abs(ordf(qg) - ordf(qr))
    if skip_groups is not None and skip_groups.any():
        M, D = qg.shape
        sgm = skip_groups if skip_groups.shape[0] == M else skip_groups.T   # -> [M, groups]
        G = D // sgm.shape[1]
        dq = np.where(np.repeat(sgm, G, axis=1), 0, dq)
    nbad = int(np.count_nonzero(dq))
    stats["q_mismatch"] = nbad
    stats["q_max_step"] = int(dq.max()) if dq.size else 0
    if dq.size and dq.max() > 1:
        i = np.unravel_index(int(dq.argmax()), dq.shape)
        raise ParityError(f"{label}: code differs by {int(dq.max())} steps at {i} "
                          f"(gpu {qg[i]:#04x}, ref {qr[i]:#04x}); {nbad} codes differ")
    if nbad > code_tol_frac * max(1, dq.size):
        raise ParityError(f"{label}: {nbad} of {dq.size} codes differ by one step "
                          f"(> {code_tol_frac:.2%})")
    stats["exact"] = (stats["residual_out_mismatch"] == 0 and stats["scale_mismatch"] == 0
                      and nbad == 0 and stats.get("norm_out_mismatch", 0) == 0)
    return stats
