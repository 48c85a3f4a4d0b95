"""The reference's comparators (src/Lrm.Tensor/Compare.fs:52-235) and kernel bounds (src/Lrm.Tensor/KernelBounds.fs),
restated in numpy float64. Test infrastructure only.
"""
from __future__ import annotations

import numpy as np

# KernelBounds.fs: Factor 2, Floor 1e-6, SmallestNormalF32 2^-126.
FACTOR = 2.0
FLOOR = 1e-6
SMALLEST_NORMAL_F32 = 1.1754943508222875e-38


def rel_l2(candidate, reference) -> float:
    """Metrics.relL2 (Compare.fs:59-71): ||c - r||2 / ||r||2, sums sequential in float64; 0 when both are zero,
    +inf when only the reference is; NaN when either holds a NaN."""
    c = np.asarray(candidate, np.float64).ravel()
    r = np.asarray(reference, np.float64).ravel()
    if c.size != r.size:
        raise ValueError(f"lengths differ: {c.size} and {r.size}")
    d = c - r
    num = float(np.dot(d, d))
    den = float(np.dot(r, r))
    if np.isnan(num) or np.isnan(den):
        return float("nan")
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return float(np.sqrt(num) / np.sqrt(den))


def max_abs(candidate, reference) -> float:
    """Metrics.maxAbs (Compare.fs:74-88)."""
    d = np.abs(np.asarray(candidate, np.float64) - np.asarray(reference, np.float64))
    if d.size == 0:
        return 0.0
    if np.isnan(d).any():
        return float("nan")
    return float(d.max())


def _log_softmax(row: np.ndarray) -> np.ndarray:
    m = row.max()
    return row - (m + np.log(np.exp(row - m).sum()))


def kl_max(candidate, reference) -> float:
    """Compare.kl (Compare.fs:370-385) with Metrics.klRow: the largest per-row KL(P_reference || P_candidate)."""
    a = np.asarray(candidate, np.float64)
    b = np.asarray(reference, np.float64)
    worst = 0.0
    for i in range(a.shape[0]):
        lq = _log_softmax(a[i])
        lp = _log_softmax(b[i])
        if np.isnan(lq).any() or np.isnan(lp).any():
            return float("nan")
        p = np.exp(lp)
        m = p > 0
        worst = max(worst, float(np.sum(p[m] * (lp[m] - lq[m]))))
    return worst


def relative_bound(reference_error: float) -> float:
    """KernelBounds.relativeBound: max(Floor, Factor * referenceError); NaN stays NaN."""
    if np.isnan(reference_error):
        return float("nan")
    return max(FLOOR, FACTOR * reference_error)


def flush_allowance(ref64) -> float:
    """KernelBounds.flushAllowance: 2^-126 * sqrt(d) / ||ref64||2 over the d results in (0, 2^-126)."""
    r = np.asarray(ref64, np.float64).ravel()
    a = np.abs(r)
    d = int(np.count_nonzero((a > 0) & (a < SMALLEST_NORMAL_F32)))
    if d == 0:
        return 0.0
    return SMALLEST_NORMAL_F32 * np.sqrt(d) / np.sqrt(float(np.dot(r, r)))


def check_relative(gpu, ref32, ref64) -> dict:
    """KernelBounds.checkRelative: relL2(gpu, ref64) <= max(1e-6, 2 * relL2(ref32, ref64)) + allowance."""
    ref_err = rel_l2(ref32, ref64)
    bound = relative_bound(ref_err) + flush_allowance(ref64)
    measured = rel_l2(gpu, ref64)
    ok = not np.isnan(measured) and not np.isnan(bound) and measured <= bound
    return {"measured": measured, "bound": bound, "ref_error": ref_err, "passed": bool(ok)}


def top1_agreement(candidate, reference) -> float:
    """Fraction of rows whose argmax agrees (lowest index of the maximum on both sides)."""
    a = np.asarray(candidate)
    b = np.asarray(reference)
    return float(np.mean(np.argmax(a, axis=-1) == np.argmax(b, axis=-1)))


def top1_flip_gaps(candidate, reference) -> np.ndarray:
    """For the rows whose argmax disagrees, how far the candidate's choice sits below the reference's maximum in the
    reference's own logits (0 for an exact tie). A disagreement inside the logit error bound is a near-tie that the
    bound allows; one beyond it is a wrong answer."""
    a = np.asarray(candidate)
    b = np.asarray(reference)
    ia, ib = np.argmax(a, axis=-1), np.argmax(b, axis=-1)
    rows = np.flatnonzero(ia != ib)
    return b[rows, ib[rows]] - b[rows, ia[rows]]
