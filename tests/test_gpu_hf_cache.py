"""GPU parity: the HF tiered cache (kessie_amd.hf_cache.KeSSieCache) and its
fog kernels against oracle/hf_cache.py run on the same device -- the
reference's torch.cat / fog op sequence -- bit-exact for K, the fog-weighted V,
the evicted chunks and the bookkeeping."""
import pytest
import torch

from oracle.hf_cache import HFCacheModel, hf_fog_mask, hf_fogged_v
from tests.inputs import randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,alpha,fs", [(100, 0.5, 0.5), (8193, 0.5, 0.5), (1000, 2.0, 0.3), (777, 0.8, 0.4),
                                        (1, 0.5, 0.5), (50, 0.0, 0.5)])
def test_hf_fog_weights(dev, n, alpha, fs):
    from kessie_amd import ops

    got = ops.hf_fog_weights(n, alpha, fs, device=dev)
    torch.cuda.synchronize()
    want = hf_fog_mask(n, alpha, fs, device=dev)
    if want is None:
        assert torch.all(got == 1.0)
        return
    want = want.view(-1)
    if alpha in (0.5, 1.0, 2.0, 3.0):
        assert torch.equal(got, want)
    else:
        assert torch.allclose(got, want, rtol=2.5e-7, atol=0)
    assert (got.cpu() - hf_fog_mask(n, alpha, fs).view(-1)).abs().max().item() <= 1e-6


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_hf_fog_apply(dev, dtype):
    from kessie_amd import ops

    arena = randn((2, 4, 300, 64), dtype, dev, 1)
    v = arena[:, :, 17:17 + 250]                       # strided window view
    out = ops.hf_fog_apply(v, 0.5, 0.5)
    torch.cuda.synchronize()
    assert torch.equal(out, hf_fogged_v(v, 0.5, 0.5))


def _check_layer(cache, model, li):
    k, v = cache[li]
    assert torch.equal(k, model.key_cache[li]) and torch.equal(v, model.value_cache[li])


def test_hf_cache_sequence(dev):
    from kessie_amd.hf_cache import KeSSieCache

    L, H, D, W = 3, 4, 64, 32
    cache = KeSSieCache(window_size=W, fog_alpha=0.5, fog_start=0.5)
    model = HFCacheModel(window_size=W, fog_alpha=0.5, fog_start=0.5)
    seed = [10]

    def step(t):
        for li in range(L):
            seed[0] += 1
            k = randn((1, H, t, D), torch.bfloat16, dev, seed[0])
            v = randn((1, H, t, D), torch.bfloat16, dev, seed[0] + 1000)
            gk, gv = cache.update(k, v, li)
            mk, mv = model.update(k, v, li)
            assert torch.equal(gk, mk) and torch.equal(gv, mv), f"layer {li}"

    step(50)
    for _ in range(40):            # decode with eviction after every step
        step(1)
        cache.evict_if_needed()
        model.evict_if_needed()
    torch.cuda.synchronize()
    assert cache.total_evictions == model.total_evictions > 0
    assert (cache.window_start, cache.seen_tokens) == (model.window_start, model.seen_tokens)
    assert len(cache.cpu_kv_store) == len(model.cpu_kv_store)
    for (s0, e0, lay0), (s1, e1, lay1) in zip(cache.cpu_kv_store, model.cpu_kv_store):
        assert (s0, e0) == (s1, e1)
        for (kc, vc), (km, vm) in zip(lay0, lay1):
            assert kc.is_pinned() and torch.equal(kc, km.cpu()) and torch.equal(vc, vm.cpu())
    assert cache.cpu_kv_bytes == model.cpu_kv_bytes
    for li in range(L):
        _check_layer(cache, model, li)

    # Recall the first chunk (in front of the window), then keep decoding and
    # evicting: exercises the front reserve and the arena moves.
    pos = cache.cpu_kv_store[0][0] + 3
    assert cache.recall_from_cpu(pos, dev) and model.recall_from_cpu(pos)
    assert not cache.recall_from_cpu(10 ** 9, dev)
    for li in range(L):
        _check_layer(cache, model, li)
    for _ in range(70):
        step(1)
        cache.evict_if_needed()
        model.evict_if_needed()
    pos = cache.cpu_kv_store[-1][0]
    assert cache.recall_from_cpu(pos, dev) and model.recall_from_cpu(pos)
    step(3)
    torch.cuda.synchronize()
    for li in range(L):
        _check_layer(cache, model, li)
    assert (cache.window_start, cache.seen_tokens, cache.total_recalls, cache.cpu_kv_bytes) == \
        (model.window_start, model.seen_tokens, model.total_recalls, model.cpu_kv_bytes)
    st = cache.get_stats()
    assert st["kv_seq_len"] == model.key_cache[0].shape[2] and st["kv_layers"] == L
    assert st["kv_cpu_chunks"] == len(model.cpu_kv_store)
    cache.full_reset()
    assert len(cache) == 0 and cache.get_seq_length() == 0
