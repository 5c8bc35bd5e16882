"""CPU: pin the index-query oracles (oracle/index.py) with closed forms and a
library routine (scikit-learn's cosine_similarity)."""
import numpy as np
import pytest

from oracle.index import cosine_ref, topk_ref, vector_search_ref


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_cosine_closed_forms(mode):
    rng = np.random.default_rng(0)
    q = rng.standard_normal(256)
    o = rng.standard_normal(256)
    o -= (o @ q) / (q @ q) * q          # orthogonal to q
    mat = np.stack([q, 3.5 * q, -q, o, np.zeros(256)])
    s = cosine_ref(q, mat, mode)
    # mode 1's (|x| + 1e-8) denominators leave 1 - 2e-8/|q| for parallel rows
    assert s[0] == pytest.approx(1.0, abs=1e-8) and s[1] == pytest.approx(1.0, abs=1e-8)
    assert s[2] == pytest.approx(-1.0, abs=1e-8)
    assert abs(s[3]) < 1e-12
    assert s[4] == 0.0                   # a zero row scores 0 in every mode


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_cosine_matches_sklearn(mode):
    from sklearn.metrics.pairwise import cosine_similarity

    rng = np.random.default_rng(1)
    mat = rng.standard_normal((500, 64)) * rng.uniform(0.1, 10, (500, 1))
    q = rng.standard_normal(64)
    want = cosine_similarity(mat, q[None])[:, 0]
    assert np.allclose(cosine_ref(q, mat, mode), want, atol=1e-8)


def test_modes_differ_only_near_zero_norms():
    tiny = np.full((1, 4), 1e-6)
    q = np.ones(4)
    s0, s1, s2 = (cosine_ref(q, tiny, m)[0] for m in (0, 1, 2))
    assert s2 == pytest.approx(1.0) and s1 == pytest.approx(1.0, rel=1e-2)
    assert s0 < 0.5                      # 1e-8 inside the square root dominates |row|^2 = 4e-12


def test_topk_order_and_ties():
    sims = np.array([0.5, 0.9, 0.5, -1.0, 0.9, 0.7])
    ids, scores = topk_ref(sims, 4)
    assert ids.tolist() == [1, 4, 5, 0] and scores.tolist() == [0.9, 0.9, 0.7, 0.5]
    rng = np.random.default_rng(2)
    s = rng.integers(0, 20, 1000).astype(np.float64)
    ids, _ = topk_ref(s, 50)
    brute = sorted(range(1000), key=lambda i: (-s[i], i))[:50]
    assert ids.tolist() == brute


def test_vector_search_reference_semantics():
    rng = np.random.default_rng(3)
    vecs = [rng.standard_normal(16).astype(np.float32) for _ in range(40)]
    vecs[7] = np.zeros(16, np.float32)
    ids = list(range(100, 140))
    q = vecs[12] * 2
    res = vector_search_ref(vecs, ids, q, top_k=3)
    assert res[0][0] == 112 and res[0][1] == pytest.approx(1.0, abs=1e-6)
    assert len(res) == 3 and res[0][1] >= res[1][1] >= res[2][1]
    assert vector_search_ref(vecs, ids, np.zeros(16), 3) == []
    assert len(vector_search_ref(vecs[:2], ids[:2], q, top_k=5)) == 2
