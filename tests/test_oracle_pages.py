"""CPU: pin the page-management oracle (oracle/pages.py) with the reference's
known answer and brute-force statements of each rule."""
import numpy as np
import pytest

from oracle import pages as P


def test_threshold_evict_known_answer():
    """kessie_kernels_v2.hip:1008-1023: 128 valid pages at i*128, thr 8192 -> 64."""
    valid = np.zeros(256, np.int8)
    valid[:128] = 1
    pos = np.zeros(256, np.int32)
    pos[:128] = np.arange(128) * 128
    v2, n = P.threshold_evict(valid, pos, 8192)
    assert n == 64
    assert v2[:64].sum() == 0 and v2[64:128].sum() == 64 and v2[128:].sum() == 0


def test_paged_cache_model_free_list_order():
    """LIFO pop, ascending append on eviction (kessie_hip_kernels.py:520-540)."""
    m = P.PagedKVCacheModel(8)
    a = m.allocate_pages(3)
    assert a == [7, 6, 5]
    m.insert(a, 48, 16, 0)          # positions 0, 16, 32
    b = m.allocate_pages(2)
    assert b == [4, 3]
    m.insert(b, 32, 16, 1000)       # positions 1000, 1016
    assert m.evict_before(20) == 2  # pages 7 (pos 0) and 6 (pos 16)
    assert m.free_pages == [0, 1, 2, 6, 7]
    assert m.allocate_pages(1) == [7]
    assert list(m.layer_order()) == [3, 4, 5]
    assert m.allocate_pages(10) is None


def test_evict_list_matches_model():
    rng = np.random.default_rng(0)
    for _ in range(20):
        n = 50
        m = P.PagedKVCacheModel(n)
        ids = m.allocate_pages(30)
        m.insert(ids[:25], 25 * 4, 4, 0)            # 5 allocated pages stay invalid
        m.page_positions[:] = rng.integers(0, 100, n).astype(np.int32)
        allocated = np.zeros(n, np.int8)
        allocated[ids] = 1
        valid_before = m.page_valid.copy()
        free_before = list(m.free_pages)
        m.evict_before(40)
        _, _, freed = P.evict_list(valid_before, m.page_positions, allocated, 40)
        assert m.free_pages == free_before + list(freed)


def _brute_select(scores, valid, k_evict, frac):
    ids = [i for i in range(len(scores)) if valid[i] == 1]
    k = P.evict_k(len(ids), k_evict, frac)
    key = lambda i: (0.0 if scores[i] == 0 else float(scores[i]), i)  # -0 == +0
    return sorted(sorted(ids, key=key)[:k])


@pytest.mark.parametrize("seed", range(6))
def test_select_evict_brute_force(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 300))
    scores = rng.choice(np.array([0.5, -0.0, 0.0, 0.25, -1.0, 0.125], np.float32), n)
    scores = np.where(rng.random(n) < 0.5, rng.random(n).astype(np.float32), scores).astype(np.float32)
    valid = (rng.random(n) < 0.8).astype(np.int8)
    for k_evict, frac in ((-1, 0.25), (-1, 0.5), (3, 0.0), (10 ** 6, 0.0), (0, 0.9)):
        v2, got = P.select_evict(scores, valid, k_evict, frac)
        want = _brute_select(scores, valid, k_evict, frac)
        assert list(got) == want
        assert v2.sum() == valid.sum() - len(want)


def test_score_keys_total_order():
    s = np.array([0.5, -0.0, 0.0, -2.0, 0.5, 1e-30, -1e-30], np.float32)
    keys = P.score_keys(s)
    order = list(np.argsort(keys, kind="stable"))
    want = sorted(range(len(s)), key=lambda i: (0.0 if s[i] == 0 else float(s[i]), i))
    assert order == want


def test_compact_brute_force():
    rng = np.random.default_rng(3)
    tables = rng.permutation(400).astype(np.int32).reshape(8, 50)
    tables[1, 3] = -5
    tables[2, 0] = 999
    lens = np.array([50, 0, 10, 49, 1, 50, 25, 3], np.int32)
    valid = (rng.random(400) < 0.6).astype(np.int8)
    nt, nl, g = P.compact(tables, lens, valid)
    flat = []
    for s in range(8):
        keep = [int(x) for x in tables[s, : lens[s]] if 0 <= x < 400 and valid[x] == 1]
        assert list(nt[s, : len(keep)]) == keep and all(nt[s, len(keep):] == -1)
        assert nl[s] == len(keep)
        flat += keep
    assert list(g) == flat


def test_insert_addressing_brute_force():
    pool = np.zeros((5, 4, 2, 2, 3), np.float32)
    t = 10
    nk = np.arange(t * 2 * 3, dtype=np.float32).reshape(t, 2, 3)
    nv = -nk
    target = np.array([2, 7, 0], np.int32)   # id 7 is out of range: skipped
    valid = np.zeros(5, np.int8)
    pos = np.zeros(5, np.int32)
    P.page_insert(pool, nk, nv, target, valid, pos, 100)
    for tok in range(t):
        page = target[tok // 4]
        if page >= 5:
            continue
        assert (pool[page, tok % 4, 0] == nk[tok]).all() and (pool[page, tok % 4, 1] == nv[tok]).all()
    assert list(valid) == [1, 0, 1, 0, 0] and pos[2] == 100 and pos[0] == 108
