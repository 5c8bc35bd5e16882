"""Paged-KV management oracles (test infrastructure only), numpy.

Reference semantics restated here:
  * threshold evict predicate  valid==1 && pos < thr           (kessie_kernels_v2.hip:393-407)
  * insert addressing           page = target[t//P], slot t%P   (kessie_kernels_v2.hip:414-456)
  * free-list order             LIFO pop from the end; evict appends every
                                not-free invalid page in ascending id order
                                (kessie_hip_kernels.py:501,520-540)
  * gather order (get_layer_kv) valid pages, ascending physical id
                                (kessie_hip_kernels.py:558-564)
Score eviction (the lowest fraction of valid pages by score) is not in the
reference; it is the threshold predicate applied at the exact k-th order
statistic of the total order (score asc, page id asc), followed by per-table
compaction that keeps survivors in logical order.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np


def threshold_evict(valid: np.ndarray, positions: np.ndarray, thr: int):
    """kessie_page_evict (kessie_kernels_v2.hip:393-407).  Returns (valid', count)."""
    valid = valid.copy()
    hit = (valid == 1) & (positions < thr)
    valid[hit] = 0
    return valid, int(hit.sum())


def evict_list(valid: np.ndarray, positions: np.ndarray, allocated: Optional[np.ndarray], thr: int):
    """Pages freed by KeSSiePagedKVCache.evict_before (kessie_hip_kernels.py:526-540).

    After the threshold predicate, every page that is invalid and not on the
    free list is appended in ascending id order.  ``allocated`` marks pages
    not on the free list (None = exactly the valid pages).
    Returns (valid', allocated', freed ids ascending).
    """
    allocated = (valid == 1).astype(np.int8) if allocated is None else allocated.copy()
    valid, _ = threshold_evict(valid, positions, thr)
    freed = np.nonzero((valid == 0) & (allocated != 0))[0].astype(np.int32)
    allocated[freed] = 0
    return valid, allocated, freed


def page_insert(pool: np.ndarray, new_k: np.ndarray, new_v: np.ndarray, target_pages: np.ndarray,
                valid: np.ndarray, positions: np.ndarray, conv_pos: int):
    """kessie_page_insert (kessie_kernels_v2.hip:414-456) on a native pool
    [pages, P, 2, H, D]; in place.  Ids outside [0, pages) are skipped."""
    num_pages, p = pool.shape[0], pool.shape[1]
    t = new_k.shape[0]
    for tok in range(t):
        phys = int(target_pages[tok // p])
        if phys < 0 or phys >= num_pages:
            continue
        pool[phys, tok % p, 0] = new_k[tok]
        pool[phys, tok % p, 1] = new_v[tok]
        if tok % p == 0:
            valid[phys] = 1
            positions[phys] = conv_pos + tok
    return pool, valid, positions


def score_keys(scores: np.ndarray) -> np.ndarray:
    """uint64 keys ordering (score asc, id asc); -0 and +0 compare equal."""
    s = scores.astype(np.float32).copy()
    s[s == 0] = 0.0  # fold -0 into +0
    bits = s.view(np.uint32).astype(np.uint64)
    neg = (bits >> np.uint64(31)) == 1
    ordered = np.where(neg, (~bits) & np.uint64(0xFFFFFFFF), bits | np.uint64(0x80000000))
    ids = np.arange(len(scores), dtype=np.uint64)
    return (ordered << np.uint64(32)) | ids


def evict_k(n_valid: int, k_evict: int, evict_fraction: float) -> int:
    if k_evict >= 0:
        return min(k_evict, n_valid)
    return int(math.floor(float(evict_fraction) * n_valid))


def select_evict(scores: np.ndarray, valid: np.ndarray, k_evict: int = -1, evict_fraction: float = 0.25):
    """Evict the k lowest (score, id) among valid pages.

    Brute-force statement: a stable sort of the valid ids by score (ties keep
    ascending id) and take the first k.  Returns (valid', evicted ids ascending).
    """
    valid = valid.copy()
    ids = np.nonzero(valid == 1)[0]
    k = evict_k(len(ids), k_evict, evict_fraction)
    s = scores[ids].astype(np.float32).copy()
    s[s == 0] = 0.0
    order = np.argsort(s, kind="stable")
    chosen = np.sort(ids[order[:k]]).astype(np.int32)
    valid[chosen] = 0
    return valid, chosen


def compact(tables: np.ndarray, lens: np.ndarray, valid: np.ndarray):
    """Per-table survivors in logical order; gather list in (seq, logical) order.

    Returns (new_tables (-1 padded), new_lens, gather_idx)."""
    s, width = tables.shape
    num_pages = valid.shape[0]
    new_tables = np.full_like(tables, -1)
    new_lens = np.zeros(s, dtype=np.int32)
    gather = []
    for i in range(s):
        row = tables[i, : min(max(int(lens[i]), 0), width)]  # a length outside [0, width] is clamped
        ok = (row >= 0) & (row < num_pages)
        ok[ok] = valid[row[ok]] == 1
        keep = row[ok]
        new_tables[i, : len(keep)] = keep
        new_lens[i] = len(keep)
        gather.append(keep)
    gidx = np.concatenate(gather).astype(np.int32) if gather else np.zeros(0, np.int32)
    return new_tables, new_lens, gidx


def valid_list(valid: np.ndarray) -> np.ndarray:
    """get_layer_kv order (kessie_hip_kernels.py:558-564): valid ids ascending."""
    return np.nonzero(valid == 1)[0].astype(np.int32)


def gather_pages(pool_bytes: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """Byte copy of whole pages: pool_bytes [pages, page_bytes] -> [len(idx), page_bytes]."""
    return pool_bytes[idx]


class PagedKVCacheModel:
    """Host model of KeSSiePagedKVCache's page bookkeeping (kessie_hip_kernels.py:484-570):
    free list, LIFO allocation, evict_before's ascending append, get_layer_kv order."""

    def __init__(self, num_pages: int):
        self.num_pages = num_pages
        self.page_valid = np.zeros(num_pages, np.int8)
        self.page_positions = np.zeros(num_pages, np.int32)
        self.free_pages = list(range(num_pages))
        self.total_evictions = 0

    def allocate_pages(self, n: int):
        if len(self.free_pages) < n:
            return None
        return [self.free_pages.pop() for _ in range(n)]

    def insert(self, page_ids, num_tokens: int, page_size: int, conv_position: int):
        for p, pid in enumerate(page_ids):
            self.page_valid[pid] = 1
            self.page_positions[pid] = conv_position + p * page_size

    def evict_before(self, position: int) -> int:
        self.page_valid, _ = threshold_evict(self.page_valid, self.page_positions, position)
        free = set(self.free_pages)
        evicted = 0
        for i in range(self.num_pages):
            if self.page_valid[i] == 0 and i not in free:
                self.free_pages.append(i)
                evicted += 1
        self.total_evictions += evicted
        return evicted

    def layer_order(self):
        return valid_list(self.page_valid)
