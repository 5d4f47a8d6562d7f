"""Numeric helpers shared by CPU and GPU tests (no GPU or library imports)."""
import numpy as np


def half_ulp(x) -> np.ndarray:
    """Half the fp16 spacing at |x| (the largest correct-rounding error)."""
    a = np.abs(np.asarray(x, np.float64)).astype(np.float16)
    up = np.nextafter(a, np.float16(np.inf)).astype(np.float64) - a.astype(np.float64)
    return 0.5 * np.maximum(up, 2.0 ** -24)


def tight_bound(ref) -> np.ndarray:
    """Per-element bound of a correctly rounded fp16 output of an fp32 result:
    half an fp16 ulp plus 2e-6 relative fp32 accumulation error."""
    r = np.asarray(ref, np.float64)
    return half_ulp(r) + 2e-6 * np.abs(r) + 1e-7


def cond_bound(ref, mag) -> np.ndarray:
    """tight_bound widened by the rounding of the fp32 arithmetic itself where an
    output cancels: the terms a kernel accumulates have magnitude
    mag = sum_j p_j |v_jd| (oracle.batch.magnitude_gqa), and scores, weights and
    sums are each rounded at that scale, so |error| may reach a few fp32 ulps of
    mag even when |ref| is 1000x smaller. Adds 8 fp32 ulps (2^-21) of mag; for
    an output that does not cancel (mag ~ |ref|) that is under 5e-7 |ref|."""
    return tight_bound(ref) + 2.0 ** -21 * np.asarray(mag, np.float64)
