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


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n_old,t_new", [(250, 1), (250, 37), (0, 40), (5000, 1)])
def test_hf_append_fog(dev, dtype, n_old, t_new):
    """The fused append + fog launch: arena rows after the append equal the
    new states, untouched rows keep their bytes, and the fogged window equals
    the oracle's fog over the concatenated V."""
    from kessie_amd import ops

    b, h, d, off, cap = 2, 4, 64, 9, n_old + t_new + 40
    k_ar = randn((b, h, cap, d), dtype, dev, 1)
    v_ar = randn((b, h, cap, d), dtype, dev, 2)
    k0, v0 = k_ar.clone(), v_ar.clone()
    big = randn((b, h, t_new, d + 8), dtype, dev, 3)
    new_k = big[..., :d]                                # token stride d+8: still 16-byte rows
    new_v = randn((b, h, t_new, d), dtype, dev, 4)
    n = n_old + t_new
    vfog = torch.empty(b, h, n + 3, d, dtype=dtype, device=dev)[:, :, :n]
    assert ops.hf_append_fog(k_ar, v_ar, off, n_old, new_k, new_v, vfog, 0.5, 0.5)
    torch.cuda.synchronize()
    s = slice(off + n_old, off + n)
    assert torch.equal(k_ar[:, :, s], new_k) and torch.equal(v_ar[:, :, s], new_v)
    keep = torch.ones(cap, dtype=torch.bool)
    keep[s] = False
    assert torch.equal(k_ar[:, :, keep], k0[:, :, keep]) and torch.equal(v_ar[:, :, keep], v0[:, :, keep])
    want = hf_fogged_v(torch.cat([v0[:, :, off:off + n_old], new_v], dim=2), 0.5, 0.5)
    assert torch.equal(vfog, want)


def test_hf_append_only_and_unaligned_fallback(dev):
    """vfog=None appends without a fog pass; rows that are not 16-byte multiples
    are refused without writing (the cache then takes its copy path)."""
    from kessie_amd import ops
    from kessie_amd.hf_cache import KeSSieCache

    k_ar = torch.zeros(1, 2, 64, 32, dtype=torch.bfloat16, device=dev)
    v_ar = torch.zeros_like(k_ar)
    nk, nv = randn((1, 2, 3, 32), torch.bfloat16, dev, 5), randn((1, 2, 3, 32), torch.bfloat16, dev, 6)
    assert ops.hf_append_fog(k_ar, v_ar, 4, 10, nk, nv, None, 0.5, 0.5)
    torch.cuda.synchronize()
    assert torch.equal(k_ar[:, :, 14:17], nk) and torch.equal(v_ar[:, :, 14:17], nv)
    assert torch.count_nonzero(k_ar[:, :, :14]) == 0 and torch.count_nonzero(k_ar[:, :, 17:]) == 0
    odd = randn((1, 2, 3, 33), torch.bfloat16, dev, 7)[..., :32]   # token stride 33 elements
    before = k_ar.clone()
    assert not ops.hf_append_fog(k_ar, v_ar, 0, 0, odd, nv, None, 0.5, 0.5)
    torch.cuda.synchronize()
    assert torch.equal(k_ar, before)
    # The cache falls back to copies + the fog kernel and stays exact.
    cache, model = KeSSieCache(window_size=16), HFCacheModel(window_size=16)
    for step in range(3):
        big_k = randn((1, 2, 5, 33), torch.bfloat16, dev, 20 + step)[..., :32]
        big_v = randn((1, 2, 5, 33), torch.bfloat16, dev, 40 + step)[..., :32]
        k, v = cache.update(big_k, big_v, 0)
        mk, mv = model.update(big_k, big_v, 0)
        torch.cuda.synchronize()
        assert torch.equal(k, mk) and torch.equal(v, mv)


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


def test_hf_recall_right_after_eviction_keeps_host_copies(dev):
    """Evict, then at once (no synchronisation) recall an OLDER chunk: the
    recall prepends into the arena slots in front of the window, which are the
    source of the eviction's asynchronous copy to pinned host memory.  The
    recall must wait for that copy; every chunk still on the host must equal
    the reference algorithm's."""
    from kessie_amd.hf_cache import KeSSieCache

    L, H, D, W = 2, 8, 128, 1024
    cache = KeSSieCache(window_size=W, fog_alpha=0.5, fog_start=0.5)
    model = HFCacheModel(window_size=W, fog_alpha=0.5, fog_start=0.5)
    seed = [500]

    def step(t):
        for li in range(L):
            seed[0] += 1
            k = randn((1, H, t, D), torch.bfloat16, dev, seed[0])
            v = randn((1, H, t, D), torch.bfloat16, dev, seed[0] + 1000)
            cache.update(k, v, li)
            model.update(k, v, li)

    step(2100)
    cache.evict_if_needed()
    model.evict_if_needed()
    step(1100)
    cache.evict_if_needed()  # the newest chunk's device-to-host copy is now in flight
    model.evict_if_needed()
    assert len(cache.cpu_kv_store) == len(model.cpu_kv_store) == 2
    pos = cache.cpu_kv_store[0][0] + 1
    assert cache.recall_from_cpu(pos, dev) and model.recall_from_cpu(pos)
    torch.cuda.synchronize()
    assert len(cache.cpu_kv_store) == len(model.cpu_kv_store) == 1
    for (s0, e0, lay0), (s1, e1, lay1) in zip(cache.cpu_kv_store, model.cpu_kv_store):
        assert (s0, e0) == (s1, e1)
        for (kc, vc), (km, vm) in zip(lay0, lay1):
            assert torch.equal(kc, km.cpu()) and torch.equal(vc, vm.cpu())
    for li in range(L):
        _check_layer(cache, model, li)
