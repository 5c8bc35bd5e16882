"""GPU parity: semantic index query (cosine scan + exact top-k) against
oracle/index.py.  Similarities: |gpu - ref| <= 2e-6 (fp32 rows) / 1e-5 (bf16
rows, oracle on the same bf16 values); top-k: bit-exact against a sort of the
kernel's own similarities (score desc, row asc) and equal to the oracle's
ranking wherever the oracle's scores are separated by more than the
similarity tolerance."""
import numpy as np
import pytest
import torch

from oracle.index import cosine_ref, topk_ref, vector_search_ref
from tests.inputs import randn

pytestmark = pytest.mark.gpu


def _check_topk(sims, ids, scores, ref_sims, k, tol):
    s = sims.cpu().numpy().astype(np.float64)
    own_ids, own_scores = topk_ref(s, min(k, len(s)))
    got_ids = ids.cpu().numpy()
    got_scores = scores.cpu().numpy()
    kk = len(own_ids)
    assert np.array_equal(got_ids[:kk], own_ids)
    assert np.array_equal(got_scores[:kk], own_scores.astype(np.float32))
    assert np.all(got_ids[kk:] == -1) and np.all(np.isneginf(got_scores[kk:]))
    ref_ids, ref_scores = topk_ref(ref_sims, min(k + 1, len(ref_sims)))
    for j in range(kk):
        gap_prev = ref_scores[j - 1] - ref_scores[j] if j > 0 else np.inf
        gap_next = ref_scores[j] - ref_scores[j + 1] if j + 1 < len(ref_scores) else np.inf
        if min(gap_prev, gap_next) > 4 * tol:
            assert got_ids[j] == ref_ids[j], f"rank {j}"


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-6), (torch.bfloat16, 1e-5)])
def test_index_query_78k(dev, mode, dtype, tol):
    from kessie_amd import ops

    n, d = 78125, 256
    mat = randn((n, d), torch.float32, dev, 0)
    mat[17] = 0.0                                  # a zero row
    mat[1000] = mat[5] * 3.0                       # same direction as row 5
    mat = mat.to(dtype)
    q = randn((d,), torch.float32, dev, 1)
    sims, ids, scores = ops.index_query(mat, q, top_k=5, norm_mode=mode)
    torch.cuda.synchronize()
    ref = cosine_ref(q.cpu().numpy(), mat.float().cpu().numpy(), mode)
    assert np.abs(sims.cpu().numpy() - ref).max() <= tol
    assert sims[17].item() == 0.0
    _check_topk(sims, ids, scores, ref, 5, tol)


@pytest.mark.parametrize("n,k", [(78125, 1024), (3000, 64), (2048, 2048 // 2), (5, 8), (1, 1), (0, 3)])
def test_index_topk_shapes(dev, n, k):
    from kessie_amd import ops

    d = 128
    mat = randn((max(n, 1), d), torch.float32, dev, 2)[:n]
    q = randn((d,), torch.float32, dev, 3)
    sims, ids, scores = ops.index_query(mat, q, top_k=k)
    torch.cuda.synchronize()
    ref = cosine_ref(q.cpu().numpy(), mat.cpu().numpy(), 0) if n else np.zeros(0)
    _check_topk(sims, ids, scores, ref, k, 2e-6)


def test_index_ties_go_to_lower_rows(dev):
    from kessie_amd import ops

    d = 64
    base = randn((50, d), torch.float32, dev, 4)
    mat = torch.cat([base, base[[3, 3, 9]], base]).contiguous()   # exact duplicates
    q = base[3].clone()
    sims, ids, scores = ops.index_query(mat, q, top_k=6)
    torch.cuda.synchronize()
    got = ids.cpu().tolist()
    assert got[:4] == [3, 50, 51, 56]             # the four copies of base[3], ascending rows
    assert len(set(scores.cpu().tolist()[:4])) == 1


def test_vector_index_class(dev):
    from kessie_amd.vector_index import VectorIndex

    rng = np.random.default_rng(5)
    vecs = [rng.standard_normal(256).astype(np.float32) for _ in range(3000)]
    vecs[10] = np.zeros(256, np.float32)
    ids = [1000 + i for i in range(3000)]
    idx = VectorIndex(256, device=dev)
    assert idx.search(vecs[0]) == []
    idx.rebuild(vecs, ids)
    assert idx.count == 3000
    q = vecs[42] + 0.05 * rng.standard_normal(256).astype(np.float32)
    got = idx.search(q, top_k=5)
    want = vector_search_ref(vecs, ids, q, top_k=5)
    assert [g[0] for g in got] == [w[0] for w in want]
    assert np.allclose([g[1] for g in got], [w[1] for w in want], atol=2e-6)
    assert idx.search(np.zeros(256, np.float32)) == []
    idx.rebuild([], [])
    assert idx.count == 0 and idx.search(q) == []


@pytest.mark.parametrize("n,k,dtype", [(200000, 16, torch.float32), (129, 16, torch.float32), (130, 1, torch.float32),
                                       (78125, 2, torch.bfloat16), (257, 7, torch.float16)])
def test_index_fused_scan_topk(dev, n, k, dtype):
    """k <= 16 runs the scan with each wave's top-k kept in registers and one
    merge launch: bit-exact against a sort of the kernel's own similarities,
    with rows spread over many waves (the last one partial) and exact
    duplicates of the best rows placed in far-apart waves (ties go to the lower
    row)."""
    from kessie_amd import ops

    d = 256
    mat = randn((n, d), torch.float32, dev, 6)
    q = randn((d,), torch.float32, dev, 7)
    mat[n // 2] = q * 2.0           # the best row, and copies of it further on
    mat[n - 1] = q * 0.5
    if n > 3:
        mat[1] = q
    mat = mat.to(dtype)
    sims, ids, scores = ops.index_query(mat, q, top_k=k)
    torch.cuda.synchronize()
    ref = cosine_ref(q.cpu().numpy(), mat.float().cpu().numpy(), 0)
    tol = 2e-6 if dtype == torch.float32 else 1e-5
    assert np.abs(sims.cpu().numpy() - ref).max() <= tol
    _check_topk(sims, ids, scores, ref, k, tol)
    top = ids.cpu().tolist()
    best = sorted({n // 2, n - 1} | ({1} if n > 3 else set()))
    assert top[:len(best)] == best if k >= len(best) else top[:k] == best[:k]


@pytest.mark.parametrize("n,k", [(78125, 5), (78125, 6), (78125, 8), (78125, 9), (40000, 8)])
@pytest.mark.parametrize("clustered", [False, True])
def test_index_merge_threshold_and_fallback(dev, n, k, clustered):
    """One merge workgroup over the scan workgroups' lists (489 of them for
    78,125 rows, 250 for 40,000): with k <= 8 and at most 3,072 keys (78,125
    rows with k = 5, 6; 40,000 rows with k = 8) it ranks the keys at or below
    the largest of its waves' smallest keys; more keys (78,125 with k = 8),
    k = 9, or the best rows clustered in one merge wave's share (rows 0..2047
    close to the query: more candidates than the threshold pass holds) take
    the selection rounds.  Bit-exact against a sort of the kernel's own
    similarities either way."""
    from kessie_amd import ops

    d = 256
    mat = randn((n, d), torch.float32, dev, 8)
    q = randn((d,), torch.float32, dev, 9)
    if clustered:
        mat[:2048] = q + 0.05 * randn((2048, d), torch.float32, dev, 10)
    sims, ids, scores = ops.index_query(mat, q, top_k=k)
    torch.cuda.synchronize()
    ref = cosine_ref(q.cpu().numpy(), mat.cpu().numpy(), 0)
    assert np.abs(sims.cpu().numpy() - ref).max() <= 2e-6
    _check_topk(sims, ids, scores, ref, k, 2e-6)
    if clustered:
        assert ids.cpu().max().item() < 2048
