"""Semantic index query oracles (test infrastructure only), numpy float64.

Three call sites normalise slightly differently; each is restated as written:
  mode 0  _kessie_index_query_kernel (kessie_hip_kernels.py:350-359):
          q / sqrt(sum(q*q) + 1e-8), row / sqrt(sum(row*row) + 1e-8), dot
  mode 1  the conversation-index searches (kessie_exp3.py:1866-1869, 2423-2426):
          q / (|q| + 1e-8), rows / (|row| + 1e-8), rows @ q
  mode 2  VectorIndex.rebuild / search (kessie_exp3.py:74-76, 89-105):
          norms below 1e-8 replaced by 1, rows / norm; q / |q| (|q| < 1e-8: no result)
Top-k order: similarity descending, ties by ascending row index.
"""
from __future__ import annotations

import numpy as np


def cosine_ref(query, mat, mode: int = 0) -> np.ndarray:
    q = np.asarray(query, dtype=np.float64).reshape(-1)
    m = np.asarray(mat, dtype=np.float64).reshape(-1, q.shape[0])
    if mode == 0:
        qn = q / np.sqrt(np.sum(q * q) + 1e-8)
        rn = m / np.sqrt(np.sum(m * m, axis=1, keepdims=True) + 1e-8)
        return rn @ qn
    if mode == 1:
        qn = q / (np.linalg.norm(q) + 1e-8)
        rn = m / (np.linalg.norm(m, axis=1, keepdims=True) + 1e-8)
        return rn @ qn
    if mode == 2:
        norms = np.linalg.norm(m, axis=1, keepdims=True)
        norms[norms < 1e-8] = 1.0
        qn = np.linalg.norm(q)
        return (m / norms) @ (q / (qn if qn >= 1e-8 else 1.0))
    raise ValueError(f"mode {mode}")


def topk_ref(sims, k: int):
    """(ids, scores) of the k best rows: similarity descending, ties by index."""
    s = np.asarray(sims)
    order = np.lexsort((np.arange(len(s)), -s))[:k]
    return order.astype(np.int64), s[order]


def vector_search_ref(vectors, ids, query, top_k: int = 5):
    """VectorIndex.rebuild + search (kessie_exp3.py:69-105, numpy path) in
    float32 as the reference computes it; ties resolved by row index."""
    if not len(vectors):
        return []
    mat = np.stack([np.asarray(v, dtype=np.float32) for v in vectors])
    norms = np.linalg.norm(mat, axis=1, keepdims=True)
    norms[norms < 1e-8] = 1.0
    mat_normed = mat / norms
    q = np.asarray(query, dtype=np.float32).reshape(1, -1)
    qn = np.linalg.norm(q)
    if qn < 1e-8:
        return []
    q = q / qn
    k = min(top_k, len(ids))
    sims = (mat_normed @ q.T).flatten()
    order, _ = topk_ref(sims, k)
    return [(ids[i], float(sims[i])) for i in order]


def numpy_search_step(mat_normed: np.ndarray, q_normed: np.ndarray, top_k: int = 5):
    """The search step of VectorIndex.search's numpy path (kessie_exp3.py:101-103)
    on an already normalised float32 matrix: matrix-vector product + argsort."""
    sims = (mat_normed @ q_normed.reshape(-1, 1)).flatten()
    top_idx = np.argsort(sims)[-top_k:][::-1]
    return top_idx, sims[top_idx]
