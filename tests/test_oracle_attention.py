"""CPU: pin the attention oracles (oracle/attention.py) with brute force on tiny
inputs and special cases the mathematics fixes."""
import math

import numpy as np
import pytest
import torch

from oracle.attention import (fused_fog_attention_ref, paged_decode_blockwise, paged_decode_ref,
                              paged_prefill_ref, windowed_attention_ref)
from oracle.fog import build_fog_weights


def brute(q, k, v, w, bias, window, causal, scale):
    """float64 loops: q [Nq,D] at positions qpos, keys 0..N-1."""
    nq, n = q.shape[0], k.shape[0]
    out = np.zeros((nq, v.shape[1]))
    for i in range(nq):
        qp = n - nq + i
        s = []
        for j in range(n):
            dist = qp - j
            ok = (not causal or dist >= 0) and (window == 0 or 0 <= dist < window)
            s.append(q[i] @ k[j] * scale + (bias[j] if bias is not None else 0.0) if ok else -np.inf)
        s = np.array(s)
        m = s.max()
        p = np.exp(s - m)
        p /= p.sum()
        out[i] = sum(p[j] * (w[j] if w is not None else 1.0) * v[j] for j in range(n))
    return out


def rnd(*shape, seed=0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


@pytest.mark.parametrize("window,causal", [(0, True), (5, True), (13, True), (0, False), (4, False)])
def test_windowed_matches_brute_force(window, causal):
    q, k, v = rnd(1, 2, 13, 8, seed=1), rnd(1, 2, 13, 8, seed=2), rnd(1, 2, 13, 8, seed=3)
    got = windowed_attention_ref(q, k, v, window, causal)
    for h in range(2):
        want = brute(q[0, h].numpy(), k[0, h].numpy(), v[0, h].numpy(), None, None, window, causal, 1 / math.sqrt(8))
        assert np.allclose(got[0, h].numpy(), want, atol=1e-12)


def test_fused_fog_matches_brute_force_and_special_cases():
    n, d = 11, 8
    q, k, v = rnd(1, 1, n, d, seed=4), rnd(1, 1, n, d, seed=5), rnd(1, 1, n, d, seed=6)
    w = build_fog_weights(n, 0.5, 0.5).double()
    got = fused_fog_attention_ref(q, k, v, w)
    want = brute(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), w.numpy(), None, 0, True, 1 / math.sqrt(d))
    assert np.allclose(got[0, 0].numpy(), want, atol=1e-12)
    # w == 1 is plain attention.
    assert torch.allclose(fused_fog_attention_ref(q, k, v, torch.ones(n, dtype=torch.float64)),
                          windowed_attention_ref(q, k, v), atol=0)
    # Window >= N equals full attention.
    assert torch.allclose(windowed_attention_ref(q, k, v, n + 3), windowed_attention_ref(q, k, v), atol=1e-15)
    # Row 0 (single visible key) is w0 * v0; constant V rows c give c * sum(p w).
    assert torch.allclose(got[0, 0, 0], w[0] * v[0, 0, 0])
    vc = torch.full_like(v, 2.5)
    row = fused_fog_attention_ref(q, k, vc, w)[0, 0, -1]
    s = (q[0, 0, -1] @ k[0, 0].T) / math.sqrt(d)
    p = torch.softmax(s, -1)
    assert torch.allclose(row, torch.full_like(row, 2.5 * float((p * w).sum())))


def _paged(seed, n_pages, p, hkv, d):
    pool = torch.randn(n_pages, p, 2, hkv, d, generator=torch.Generator().manual_seed(seed))
    return pool


def test_paged_decode_is_last_row_of_dense_with_gqa():
    hq, hkv, d, p, ctx = 8, 2, 16, 4, 23
    g = hq // hkv
    pool = _paged(7, 10, p, hkv, d)
    table = torch.tensor([[3, 9, 0, 5, 7, 1]], dtype=torch.int32)
    q = torch.randn(1, hq, d, generator=torch.Generator().manual_seed(8))
    w = build_fog_weights(ctx)
    got = paged_decode_ref(q, pool, table, torch.tensor([ctx]), w)
    kv = pool[table[0].long()].reshape(-1, 2, hkv, d)[:ctx]
    for h in range(hq):
        kk, vv = kv[:, 0, h // g].double().numpy(), kv[:, 1, h // g].double().numpy()
        want = brute(q[0, h:h + 1].double().numpy(), kk, vv, w.double().numpy(), None, 0, True, 1 / math.sqrt(d))
        assert np.allclose(got[0, h].numpy(), want[0], atol=1e-5)


def test_paged_decode_bias_window_and_empty():
    hq, hkv, d, p = 4, 4, 8, 4
    pool = _paged(9, 12, p, hkv, d)
    table = torch.arange(12, dtype=torch.int32).view(2, 6)
    q = torch.randn(2, hq, d, generator=torch.Generator().manual_seed(10))
    bias = torch.randn(2, 24, generator=torch.Generator().manual_seed(11))
    got = paged_decode_ref(q, pool, table, torch.tensor([0, 19]), None, bias, window=7)
    assert torch.count_nonzero(got[0]) == 0
    kv = pool[table[1].long()].reshape(-1, 2, hkv, d)[:19]
    for h in range(hq):
        want = brute(q[1, h:h + 1].double().numpy(), kv[:, 0, h].double().numpy(), kv[:, 1, h].double().numpy(),
                     None, bias[1].double().numpy(), 7, True, 1 / math.sqrt(d))
        assert np.allclose(got[1, h].numpy(), want[0], atol=1e-5)


def test_paged_prefill_is_last_rows_of_dense():
    hq, hkv, d, p, ctx, c = 4, 2, 8, 4, 18, 5
    pool = _paged(12, 8, p, hkv, d)
    table = torch.tensor([[6, 2, 7, 0, 4]], dtype=torch.int32)
    q = torch.randn(1, c, hq, d, generator=torch.Generator().manual_seed(13))
    w = build_fog_weights(ctx)
    got = paged_prefill_ref(q, pool, table, torch.tensor([ctx]), w, window=6)
    kv = pool[table[0].long()].reshape(-1, 2, hkv, d)[:ctx]
    for h in range(hq):
        want = brute(q[0, :, h].double().numpy(), kv[:, 0, h // 2].double().numpy(),
                     kv[:, 1, h // 2].double().numpy(), w.double().numpy(), None, 6, True, 1 / math.sqrt(d))
        assert np.allclose(got[0, :, h].numpy(), want, atol=1e-5)
    sub = paged_prefill_ref(q, pool, table, torch.tensor([ctx]), w, window=6, rows=torch.tensor([1, 4]))
    assert torch.allclose(sub[0], got[0, [1, 4]], atol=1e-6)
    # Decode == prefill with one row.
    dec = paged_decode_ref(q[:, -1], pool, table, torch.tensor([ctx]), w, window=6)
    assert torch.allclose(dec[0], got[0, -1], atol=1e-6)


def test_blockwise_decode_equals_direct():
    hq, hkv, d, p, ctx = 8, 2, 16, 4, 150
    pool = _paged(14, 40, p, hkv, d)
    table = torch.randperm(40, generator=torch.Generator().manual_seed(15)).to(torch.int32).view(1, 40)
    q = torch.randn(1, hq, d, generator=torch.Generator().manual_seed(16))
    w = build_fog_weights(ctx)
    a = paged_decode_ref(q, pool, table, torch.tensor([ctx]), w, window=61)
    b = paged_decode_blockwise(q, pool, table, torch.tensor([ctx]), w, window=61, block_pages=3)
    assert torch.allclose(a, b, atol=1e-5)


def test_blockwise_prefill_equals_direct():
    from oracle.attention import paged_prefill_blockwise

    hq, hkv, d, p, ctx, c = 8, 2, 16, 4, 150, 40
    pool = _paged(17, 40, p, hkv, d)
    table = torch.randperm(40, generator=torch.Generator().manual_seed(18)).to(torch.int32).view(1, 40)
    q = torch.randn(1, c, hq, d, generator=torch.Generator().manual_seed(19))
    w = build_fog_weights(ctx)
    rows = torch.tensor([0, 7, 39])
    for window in (0, 23):
        a = paged_prefill_ref(q, pool, table, torch.tensor([ctx]), w, window=window, rows=rows)
        b = paged_prefill_blockwise(q, pool, table, torch.tensor([ctx]), rows, w, window=window, block_pages=3)
        assert torch.allclose(a, b, atol=1e-5)
        # One kv head's query heads (all, or a subset): those heads equal the
        # direct result, every other head stays zero.
        for kvh, sub in ((1, None), (0, [3, 1])):
            hs = [kvh * 4 + x for x in (sub if sub is not None else range(4))]
            c_ = paged_prefill_blockwise(q, pool, table, torch.tensor([ctx]), rows, w, window=window,
                                         block_pages=3, kv_head=kvh, q_heads=sub)
            assert torch.allclose(a[:, :, hs], c_[:, :, hs], atol=1e-5)
            rest = [h for h in range(hq) if h not in hs]
            assert bool((c_[:, :, rest] == 0).all())
