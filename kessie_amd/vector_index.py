"""Conversation vector index on the GPU (the reference's VectorIndex,
kessie_exp3.py:58-110: FAISS IndexFlatIP or a numpy matrix product on the
CPU).  Same methods and results -- rows normalised with norms below 1e-8
taken as 1, a query with norm below 1e-8 finds nothing, [(id, score)] best
first -- with the scan and the top-k in one kessie_index_query call over a
matrix kept in HBM, and one small device-to-host copy per search.  Ties are
resolved by insertion order (lower row first)."""
from __future__ import annotations

import threading
from typing import List, Tuple

import numpy as np
import torch

from . import ops


class VectorIndex:
    """Cosine-similarity index over fixed-size embeddings, searched on the GPU."""

    def __init__(self, dim: int = 256, device=None, dtype=torch.float32):
        self.dim = dim
        self.device = torch.device(device or "cuda")
        self.dtype = dtype
        self._lock = threading.RLock()
        self._ids: List[int] = []
        self._mat = None

    def rebuild(self, vectors: List[np.ndarray], ids: List[int]):
        if not len(vectors):
            with self._lock:
                self._ids, self._mat = [], None
            return
        mat = torch.from_numpy(np.stack([np.asarray(v, dtype=np.float32) for v in vectors]))
        dev = mat.to(self.device, dtype=self.dtype)
        with self._lock:
            self._ids = list(ids)
            self._mat = dev

    def search(self, query: np.ndarray, top_k: int = 5) -> List[Tuple[int, float]]:
        q = np.asarray(query, dtype=np.float32).reshape(-1)
        if np.linalg.norm(q) < 1e-8:
            return []
        with self._lock:
            if not self._ids or self._mat is None:
                return []
            k = min(top_k, len(self._ids))
            qd = torch.from_numpy(q).to(self.device)
            _, idx, sc = ops.index_query(self._mat, qd, top_k=k, norm_mode=2)
            host = torch.cat([idx.view(torch.float32), sc]).cpu()  # one copy: id bits + scores
            ids = host[:k].view(torch.int32).tolist()
            scores = host[k:].tolist()
            return [(self._ids[i], float(s)) for i, s in zip(ids, scores) if 0 <= i < len(self._ids)]

    @property
    def count(self):
        with self._lock:
            return len(self._ids)
