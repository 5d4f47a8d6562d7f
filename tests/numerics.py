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
