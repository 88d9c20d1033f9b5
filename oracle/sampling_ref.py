"""numpy restatement of the reference's sampling step — TEST INFRASTRUCTURE ONLY.

Used by tests/ as the checker of the fused sampling kernel
(pkv_sample_rows); never by the product. float64 throughout. Paths are
relative to the reference repository.

The reference draws with torch.multinomial, whose random stream cannot be
reproduced; the restatement draws by inverse CDF from a given uniform u,
in ascending vocabulary order (the kernel's definition), so kernel and
oracle agree for every u that is not within rounding of a bucket edge.
"""
from __future__ import annotations

import numpy as np


def top_k_keep(y: np.ndarray, top_k: int) -> np.ndarray:
    """sampling.py:75-92 (apply_top_k): keep y >= the k-th largest value
    (k = min(top_k, vocab); ties at the threshold are kept); top_k <= 0
    keeps everything. y: [vocab]; returns a boolean mask."""
    if top_k <= 0:
        return np.ones(y.shape, dtype=bool)
    k = min(top_k, y.shape[-1])
    kth = np.sort(y)[::-1][k - 1]
    return y >= kth


def top_p_keep(y: np.ndarray, keep: np.ndarray, top_p: float) -> np.ndarray:
    """sampling.py:27-72 (apply_top_p) on the values kept so far: sort
    descending (ties by ascending index), softmax, and drop a token when the
    cumulative mass of the tokens before it exceeds top_p (:50-55: the
    removal mask shifted right by one, the first token always kept)."""
    if top_p >= 1.0:
        return keep.copy()
    idx = np.nonzero(keep)[0]
    order = idx[np.lexsort((idx, -y[idx]))]
    e = np.exp(y[order] - y[order[0]])
    p = e / e.sum()
    before = np.concatenate([[0.0], np.cumsum(p)[:-1]])
    out = np.zeros_like(keep)
    out[order[before <= top_p]] = True
    out[order[0]] = True
    return out


def sample_probs(logits: np.ndarray, temperature: float, top_k: int, top_p: float):
    """sampling.py:94-130 (sample, up to the softmax): y = logits /
    temperature, top-k then top-p masks, softmax over what is kept.
    Returns (mask, probs) over the vocabulary."""
    y = np.asarray(logits, dtype=np.float64) / temperature
    keep = top_p_keep(y, top_k_keep(y, top_k), top_p)
    e = np.where(keep, np.exp(y - y[keep].max()), 0.0)
    return keep, e / e.sum()


def pick(probs: np.ndarray, u: float):
    """The draw (sampling.py:132-135 draws with torch.multinomial): the
    first index, ascending, whose cumulative probability exceeds u * total.
    Returns (index, distance of u * total to the nearest bucket edge)."""
    c = np.cumsum(probs)
    t = u * c[-1]
    i = int(np.searchsorted(c, t, side="right"))
    i = min(i, len(probs) - 1)
    while probs[i] == 0 and i > 0:
        i -= 1
    edges = c[probs > 0]
    margin = float(np.min(np.abs(edges - t))) if len(edges) else 1.0
    return i, margin
