"""fp64 NumPy model of split-KV partials and their LSE merge (test infrastructure only).

Restates the two-stage algorithm of csrc_native/m1_kernel.cpp: the split
partial (paged_decode_v3 with grid.z = splits, :553-859, covering positions
[s * chunk_len, (s + 1) * chunk_len)) and split_combine (:861-888: max of the
split maxima, rescale, sum, skip empty splits, 0 when nothing was summed).
Partials are kept here as (normalised output, log-sum-exp) pairs, which is the
form the HIP kernels store; the merge is the same algebra.
"""

from __future__ import annotations

import numpy as np


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """Single query: q [D], k/v [L, D] -> [D]; zeros when L == 0."""
    if k.shape[0] == 0:
        return np.zeros(q.shape[-1], dtype=np.float64)
    s = (k.astype(np.float64) @ q.astype(np.float64)) * scale
    w = np.exp(s - s.max())
    return (w / w.sum()) @ v.astype(np.float64)


def split_partials(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
                   chunk_len: int, num_splits: int) -> tuple[np.ndarray, np.ndarray]:
    """Per split: normalised output [NS, D] and natural-log LSE [NS] (-inf when empty)."""
    d = q.shape[-1]
    outs = np.zeros((num_splits, d), dtype=np.float64)
    lse = np.full(num_splits, -np.inf, dtype=np.float64)
    for sidx in range(num_splits):
        lo, hi = sidx * chunk_len, min((sidx + 1) * chunk_len, k.shape[0])
        if hi <= lo:
            continue
        s = (k[lo:hi].astype(np.float64) @ q.astype(np.float64)) * scale
        m = s.max()
        w = np.exp(s - m)
        outs[sidx] = (w / w.sum()) @ v[lo:hi].astype(np.float64)
        lse[sidx] = m + np.log(w.sum())
    return outs, lse


def lse_combine(outs: np.ndarray, lse: np.ndarray) -> np.ndarray:
    """Merge split partials; splits with LSE = -inf contribute nothing."""
    valid = np.isfinite(lse)
    if not valid.any():
        return np.zeros(outs.shape[-1], dtype=np.float64)
    m = lse[valid].max()
    w = np.where(valid, np.exp(np.where(valid, lse, m) - m), 0.0)
    return (w[:, None] * outs).sum(axis=0) / w.sum()
