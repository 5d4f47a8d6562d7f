"""Host side of the read-probe digest (va_probe_digest): a buffer pattern in
which every 16-byte word is distinct, and the XOR of the words a probe form
must read.

The probe is the MBU denominator (the reference's read_kernel +
probe_ceiling, src/voltattn.cu:64-78, 935-957): GB/s = bytes credited / time.
A form that read fewer bytes than it is credited with (a skipped tile, a
dropped load, a wrong chunk size) would overstate the ceiling. Its digest
(XOR of every word loaded, number of 16-byte loads) is compared with the
host's XOR and count over exactly the credited bytes.
"""
from __future__ import annotations

import numpy as np


def pattern(nbytes: int, salt: int = 0x9E3779B9) -> np.ndarray:
    """`nbytes` (a multiple of 16) of 16-byte words w_i = four 32-bit lanes of
    splitmix64-style mixes of (i, lane): distinct words, no structure a
    plausible coverage mistake could cancel."""
    n = nbytes // 16
    i = np.arange(n, dtype=np.uint64)
    out = np.empty((n, 4), dtype=np.uint32)
    for lane in range(4):
        z = (i * np.uint64(4) + np.uint64(lane) + np.uint64(salt)) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
        out[:, lane] = (z & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    return out.reshape(-1).view(np.uint8)


def xor16(buf: np.ndarray) -> bytes:
    """XOR of the 16-byte words of `buf` (length a multiple of 16), as 16 bytes."""
    w = np.ascontiguousarray(buf).view(np.uint32).reshape(-1, 4)
    return np.bitwise_xor.reduce(w, axis=0).astype("<u4").tobytes()
