"""CPU: pin the HF tiered-cache oracle (oracle/hf_cache.py) with closed forms
of its fog mask and invariants of its update / evict / recall bookkeeping."""
import pytest
import torch

from oracle.hf_cache import HFCacheModel, hf_fog_mask, hf_fogged_v


@pytest.mark.parametrize("n,alpha,fs", [(100, 0.5, 0.5), (4097, 0.5, 0.5), (10, 2.0, 0.3), (3, 0.5, 0.5)])
def test_hf_fog_mask_closed_form(n, alpha, fs):
    w = hf_fog_mask(n, alpha, fs).view(-1)
    cc = max(1, int(n * fs))
    fc = n - cc
    assert w.shape == (n,)
    assert torch.all(w[fc:] == 1.0)
    assert w[0].item() == pytest.approx(0.01)            # 0^alpha clamped to 0.01
    if fc > 1:
        assert w[fc - 1].item() == pytest.approx(1.0)
    assert torch.all(w[1:] >= w[:-1])
    p = torch.arange(fc, dtype=torch.float64) / max(fc - 1, 1)
    assert torch.allclose(w[:fc].double(), (p ** alpha).clamp(min=0.01), atol=1e-6)


def test_hf_fog_mask_degenerate():
    assert hf_fog_mask(100, 0.0, 0.5) is None
    assert hf_fog_mask(0, 0.5, 0.5) is None
    assert hf_fog_mask(1, 0.5, 0.5) is None                # cc = 1 -> fc = 0
    assert hf_fog_mask(10, 0.5, 1.0) is None
    v = torch.randn(1, 2, 5, 4, dtype=torch.bfloat16)
    assert hf_fogged_v(v, 0.0, 0.5) is v


def test_model_history_is_lossless():
    """After evictions and a recall, stored chunks + window cover the history,
    and a recall prepends exactly the stored chunk."""
    g = torch.Generator().manual_seed(0)
    m = HFCacheModel(window_size=8, fog_alpha=0.5, fog_start=0.5)
    hist = []
    for step in range(60):
        t = 20 if step == 0 else 1
        k = torch.randn(1, 2, t, 4, generator=g)
        hist.append(k)
        m.update(k, k * 2, 0)
        m.evict_if_needed()
    full = torch.cat(hist, dim=2)
    stored = torch.cat([c[2][0][0] for c in m.cpu_kv_store], dim=2)
    assert torch.equal(torch.cat([stored, m.key_cache[0]], dim=2), full)
    assert m.window_start == stored.shape[2] and m.seen_tokens == full.shape[2]
    first = m.cpu_kv_store[0]
    assert m.recall_from_cpu(first[0])
    assert torch.equal(m.key_cache[0][:, :, : first[1] - first[0]], first[2][0][0])
    assert m.window_start == first[0] and m.total_recalls == 1
    assert not m.recall_from_cpu(10 ** 9)
