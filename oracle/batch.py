"""Test infrastructure: CPU oracle of the grouped-query, batched and paged forms.

The reference (kamilch1k/voltattn) decodes one sequence with one query head
per K/V head from a contiguous cache; its per-head attention is
``reference()`` (src/voltattn.cu:769-794), restated by :func:`oracle.reference`.
The forms below are definitions layered on that restatement, not new
arithmetic:

* grouped-query attention: query head h of a sequence uses KV head
  h // (Hq // Hkv), i.e. the reference over K/V heads repeated Hq/Hkv times
  (:func:`reference_gqa`);
* paged cache: position j of sequence b is row j % page_rows of page
  block_table[b][j // page_rows], each page holding [Hkv][page_rows][...]
  (:func:`scatter_rows` writes a contiguous cache into pages,
  :func:`gather_rows` reads it back);
* the magnitude of each output, sum_j p_j |v_jd| with the same softmax
  weights (:func:`magnitude_gqa`): the scale of the summands an fp32 kernel
  accumulates, which sets its rounding error where the output itself cancels
  far below it. Not part of the reference; the randomized tests use it to
  size their error bound.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline import this
package; the product never does.
"""
from __future__ import annotations

import numpy as np

from . import reference as _reference


def reference_gqa(kd: np.ndarray, vd: np.ndarray, q: np.ndarray, Hq: int, Hkv: int, L: int,
                  D: int, threads: int = 1) -> np.ndarray:
    """Double-precision attention of Hq query heads over Hkv KV heads.

    kd, vd: float32 [Hkv][L][D] (dequantized values); q: fp16 bits [Hq][D].
    Returns float32 [Hq*D]."""
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    g = Hq // Hkv
    kr = np.repeat(np.asarray(kd, np.float32).reshape(Hkv, L, D), g, axis=0)
    vr = np.repeat(np.asarray(vd, np.float32).reshape(Hkv, L, D), g, axis=0)
    return _reference(np.ascontiguousarray(kr).ravel(), np.ascontiguousarray(vr).ravel(),
                      np.ascontiguousarray(q).ravel(), Hq, L, D, threads=threads)


def magnitude_gqa(kd: np.ndarray, vd: np.ndarray, q: np.ndarray, Hq: int, Hkv: int, L: int,
                  D: int) -> np.ndarray:
    """sum_j p_hj |v_jd| in double, p_h the softmax of q_h . k_j / sqrt(D) over the
    KV head of query head h (the weights of reference(), src/voltattn.cu:776-791).

    kd, vd: float32 [Hkv][L][D]; q: fp16 bits [Hq][D]. Returns float64 [Hq*D].
    It equals |reference| when every v_jd >= 0 and bounds it from above."""
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    g = Hq // Hkv
    k = np.asarray(kd, np.float32).reshape(Hkv, L, D).astype(np.float64)
    v = np.abs(np.asarray(vd, np.float32).reshape(Hkv, L, D).astype(np.float64))
    qf = np.asarray(q).view(np.float16).reshape(Hq, D).astype(np.float64)
    out = np.empty((Hq, D), np.float64)
    for h in range(Hq):
        s = k[h // g] @ qf[h] / np.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p @ v[h // g]) / p.sum()
    return out.ravel()


def scatter_rows(pool: np.ndarray, rows: np.ndarray, table: np.ndarray, page_rows: int) -> None:
    """Write rows [Hkv][L][W] of one sequence into pool [num_pages][Hkv][page_rows][W]
    through its block-table row `table` (positions 0..L-1)."""
    Hkv, L = rows.shape[0], rows.shape[1]
    for j0 in range(0, L, page_rows):
        n = min(page_rows, L - j0)
        pool[table[j0 // page_rows], :, :n] = rows[:, j0:j0 + n]


def gather_rows(pool: np.ndarray, table: np.ndarray, L: int, page_rows: int) -> np.ndarray:
    """Rows [Hkv][L][W] of one sequence from pool [num_pages][Hkv][page_rows][W]."""
    Hkv, W = pool.shape[1], pool.shape[3]
    out = np.empty((Hkv, L, W), pool.dtype)
    for j0 in range(0, L, page_rows):
        n = min(page_rows, L - j0)
        out[:, j0:j0 + n] = pool[table[j0 // page_rows], :, :n]
    return out
