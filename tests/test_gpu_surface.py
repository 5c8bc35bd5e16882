"""GPU: producers around the attention call (fog bias / fog weights / slot-mapped
K/V write) and the mirrored Python surface (fog cache, attention impl,
paged KV cache, KV connector) against the oracles.

Fog vectors: bit-exact against the reference's torch op sequence executed on
the same device (oracle.fog with device=cuda), and within one unit in the last
place of the dtype against the same ops on the CPU (torch's CPU kernel divides
where its device kernel multiplies by a reciprocal).  Copies: bit-exact.
Attention: bf16 |gpu - ref| <= 2e-2 + 1e-2 |ref|.
"""
import math

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_ref, paged_prefill_ref
from oracle.fog import build_fog_weights, fog_bias
from oracle.pages import PagedKVCacheModel
from oracle.rope import rope_remap_ref
from tests.inputs import gen, randn, randperm

pytestmark = pytest.mark.gpu

ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -23}


def _close_attn(got, ref):
    g = got.float().cpu()
    diff = (g - ref).abs()
    bad = diff > 2e-2 + 1e-2 * ref.abs()
    assert not bad.any(), f"{int(bad.sum())}/{bad.numel()} outside tol, max diff {diff.max().item():.3e}"


@pytest.mark.parametrize("dtype,kv_len,alpha,start,recall", [
    (torch.bfloat16, 131072, 0.5, 0.5, [7, 1000, 65535, 131071, 200000, -3, 7]),
    (torch.float32, 4096, 0.8, 0.3, [5]),
    (torch.float32, 128, 0.5, 0.5, [10, 50, 100]),
    (torch.float16, 70000, 0.5, 0.0, [69999, 3]),   # fp16 positions overflow to inf
    (torch.bfloat16, 1000, 0.0, 0.5, []),
    (torch.float32, 3, 0.5, 1.5, [1]),               # negative boundary: no fog
    (torch.float32, 0, 0.5, 0.5, []),
    # thousands of recalled positions (every workgroup scans the whole list):
    # workgroup edges, duplicates, out-of-range values
    (torch.bfloat16, 131072, 0.5, 0.5, list(range(0, 131072, 37)) + [255, 256, 511, 512, 512, 131071, 131072, -1]),
])
def test_fog_bias_fill(dev, dtype, kv_len, alpha, start, recall):
    from kessie_amd import ops

    buf = torch.full((kv_len + 5,), 7.0, dtype=dtype, device=dev)
    rec = torch.tensor(recall, dtype=torch.int32, device=dev) if recall else None
    got = ops.fog_bias_fill(buf, kv_len, alpha, start, rec, 0.1)
    torch.cuda.synchronize()
    want_dev = fog_bias(kv_len, alpha, start, recall, 0.1, dtype=dtype, device=dev)
    assert torch.equal(got, want_dev)
    assert torch.all(buf[kv_len:] == 7.0)  # nothing written past kv_len
    want_cpu = fog_bias(kv_len, alpha, start, recall, 0.1, dtype=dtype)
    g, w = got.float().cpu(), want_cpu.float()
    # torch's CPU fp16 arange overflows to inf at 65532 where the device (and
    # round-to-nearest-even) overflows at 65520: compare where both are finite.
    fin = torch.isfinite(w) & torch.isfinite(g)
    if kv_len:
        assert (g[fin] - w[fin]).abs().max().item() <= ULP[dtype] * max(1.0, alpha)


@pytest.mark.parametrize("n,alpha,start", [(4096, 0.5, 0.5), (131072, 0.5, 0.5), (1000, 1.0, 0.3),
                                           (1000, 2.0, 0.5), (2049, 0.8, 0.25), (7, 0.5, 0.5), (2, 0.5, 0.5)])
def test_fog_weights(dev, n, alpha, start):
    from kessie_amd import ops

    got = ops.fog_weights(n, alpha, start, device=dev)
    torch.cuda.synchronize()
    want_dev = build_fog_weights(n, alpha, start, device=dev)
    if alpha in (0.5, 1.0, 2.0, 3.0):
        assert torch.equal(got, want_dev)
    else:  # powf: same math library call, allow one ulp across builds
        assert torch.allclose(got, want_dev, rtol=2.5e-7, atol=0)
    assert (got.cpu() - build_fog_weights(n, alpha, start)).abs().max().item() <= 1e-6


@pytest.mark.parametrize("layout,dtype,d", [("kv_first", torch.bfloat16, 128), ("block_kv", torch.bfloat16, 128),
                                            ("native", torch.float32, 128), ("kv_first", torch.float16, 100)])
def test_kv_cache_write(dev, layout, dtype, d):
    from kessie_amd import ops

    nb, p, hkv, hq, t = 20, 16, 8, 32, 45
    shape = {"kv_first": (2, nb, p, hkv, d), "block_kv": (nb, 2, p, hkv, d), "native": (nb, p, 2, hkv, d)}[layout]
    pool = randn(shape, dtype, dev, 1)
    before = pool.clone()
    qkv = randn((t, (hq + 2 * hkv) * d), dtype, dev, 2)
    key = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)          # strided views, as vLLM hands them over
    value = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    slots = randperm(nb * p, dev, 3)[:t].to(torch.int64)
    slots[[4, 17]] = -1
    ops.kv_cache_write(pool, key, value, slots, layout=layout)
    torch.cuda.synchronize()
    ref = before.cpu()
    s = slots.cpu()
    ok = s >= 0
    blk, off = (s[ok] // p), (s[ok] % p)
    kk, vv = key.cpu()[ok], value.cpu()[ok]
    if layout == "kv_first":
        ref[0, blk, off], ref[1, blk, off] = kk, vv
    elif layout == "block_kv":
        ref[blk, 0, off], ref[blk, 1, off] = kk, vv
    else:
        ref[blk, off, 0], ref[blk, off, 1] = kk, vv
    assert torch.equal(pool.cpu(), ref)


def _state(**kw):
    st = {"fog_alpha": 0.5, "fog_start": 0.5, "prompt_len": 100, "recall_positions": {10, 50, 100},
          "recall_boost": 0.1, "enabled": True, "generation": 1}
    st.update(kw)
    return st


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fog_cache_generations(dev, dtype):
    from kessie_amd.kessie_attention import _FogCache

    cache = _FogCache()
    s1 = _state()
    b1 = cache.get_fog_bias(128, dev, dtype, s1)
    assert b1.shape == (1, 1, 1, 128)
    want = fog_bias(128, 0.5, 0.5, {10, 50, 100}, 0.1, dtype=dtype, device=dev)
    assert torch.equal(b1.view(-1), want)
    assert cache.get_fog_bias(128, dev, dtype, s1).data_ptr() == b1.data_ptr()
    # Next generation, same parameters: the side stream's buffer, same values.
    b2 = cache.get_fog_bias(128, dev, dtype, _state(generation=2))
    assert b2.data_ptr() != b1.data_ptr()
    assert torch.equal(b2.view(-1), want)
    # Next generation with new parameters (state.update bumps by one): the
    # precomputed buffer is stale and must not be used.
    s3 = _state(generation=3, fog_alpha=0.8, fog_start=0.3, recall_positions={5})
    b3 = cache.get_fog_bias(256, dev, dtype, s3)
    assert torch.equal(b3.view(-1), fog_bias(256, 0.8, 0.3, {5}, 0.1, dtype=dtype, device=dev))
    # Same generation, context grew by one (decode): recomputed for the new kv_len.
    b4 = cache.get_fog_bias(257, dev, dtype, s3)
    assert torch.equal(b4.view(-1), fog_bias(257, 0.8, 0.3, {5}, 0.1, dtype=dtype, device=dev))
    f32 = cache.get_fog_bias_f32(257, dev, dtype, s3)
    assert f32.dtype == torch.float32 and torch.equal(f32, b4.view(-1).float())


def _mixed_batch(dev, order, seed=0, p=16):
    """Sequences (query_len, ctx) in ``order``; blocks of ``p`` tokens drawn at random."""
    hq, hkv, d, nb = 32, 8, 128, 96
    spec = {"d0": (1, 300), "pf": (37, 500), "d1": (1, 77)}
    seqs = [spec[k] for k in order]
    width = 32
    perm = randperm(nb, dev, seed + 1).cpu()
    table = torch.zeros(len(seqs), width, dtype=torch.int32)
    at = 0
    for i, (_, ctx) in enumerate(seqs):
        n = -(-ctx // p)
        table[i, :n] = perm[at:at + n]
        at += n
    qsl = [0]
    for ql, _ in seqs:
        qsl.append(qsl[-1] + ql)
    n_tok = qsl[-1]
    slots = []
    for i, (ql, ctx) in enumerate(seqs):
        for pos in range(ctx - ql, ctx):
            slots.append(int(table[i, pos // p]) * p + pos % p)
    kv_cache = randn((2, nb, p, hkv, d), torch.bfloat16, dev, seed + 2)
    query = randn((n_tok, hq * d), torch.bfloat16, dev, seed + 3)
    key = randn((n_tok, hkv, d), torch.bfloat16, dev, seed + 4)
    value = randn((n_tok, hkv, d), torch.bfloat16, dev, seed + 5)
    from kessie_amd.kessie_attention import KeSSieAttentionMetadata

    meta = KeSSieAttentionMetadata(
        num_actual_tokens=n_tok, max_query_len=max(q for q, _ in seqs),
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=dev),
        max_seq_len=max(c for _, c in seqs), seq_lens=torch.tensor([c for _, c in seqs], dtype=torch.int32, device=dev),
        block_table=table.to(dev), slot_mapping=torch.tensor(slots, dtype=torch.int64, device=dev))
    return seqs, qsl, kv_cache, query, key, value, meta


@pytest.mark.parametrize("order,fog,p", [(("d0", "pf", "d1"), True, 16), (("d0", "d1", "pf"), True, 16),
                                         (("pf", "d0"), False, 16), (("d0", "pf", "d1"), True, 32)])
def test_attention_impl_forward(dev, monkeypatch, order, fog, p):
    """A mixed batch through KeSSieAttentionImpl.forward: slot-mapped cache
    write, decode rows and one varlen prefill launch, against the oracle
    (16- and 32-token blocks)."""
    from kessie_amd import kessie_attention as ka

    hq, hkv, d = 32, 8, 128
    seqs, qsl, kv_cache, query, key, value, meta = _mixed_batch(dev, order, p=p)
    state = ka.KeSSieAttentionState()
    state.update(prompt_len=100 if fog else 0, recall_positions={5, 250})
    monkeypatch.setattr(ka, "KESSIE_STATE", state)
    monkeypatch.setattr(ka, "_FOG_CACHE", ka._FogCache())
    before = kv_cache.clone()
    impl = ka.KeSSieAttentionImpl(hq, d, d ** -0.5, hkv)
    out = impl.forward(None, query, key, value, kv_cache, meta)
    torch.cuda.synchronize()
    assert out.shape == (qsl[-1], hq * d)

    # The new rows landed in their slots and nothing else changed.
    ref_cache = before.cpu()
    sl = meta.slot_mapping.cpu()
    ref_cache[0, sl // p, sl % p] = key.cpu()
    ref_cache[1, sl // p, sl % p] = value.cpu()
    assert torch.equal(kv_cache.cpu(), ref_cache)

    pool = ref_cache.permute(1, 2, 0, 3, 4).contiguous()  # native [pages, P, 2, H, D]
    table, lens = meta.block_table.cpu(), meta.seq_lens.cpu()
    q = query.cpu().view(-1, hq, d)
    o = out.view(-1, hq, d)
    for i, (ql, ctx) in enumerate(seqs):
        # Each sequence's bias is the reference's vector for its own length.
        bias = fog_bias(ctx, 0.5, 0.5, {5, 250}, 0.1, dtype=torch.bfloat16).float() if fog else None
        s, e = qsl[i], qsl[i + 1]
        if ql == 1:
            ref = paged_decode_ref(q[s:e], pool, table[i:i + 1], lens[i:i + 1], None, bias)
            _close_attn(o[s:e], ref)
        else:
            ref = paged_prefill_ref(q[s:e].unsqueeze(0), pool, table[i:i + 1], lens[i:i + 1], None, bias)
            _close_attn(o[s:e].unsqueeze(0), ref)


def test_paged_kv_cache_matches_model(dev):
    from kessie_amd.paged_kv_cache import KeSSiePagedKVCache

    P, H, D, L, N = 16, 8, 128, 2, 64
    cache = KeSSiePagedKVCache(N, P, L, H, D, dev, dtype=torch.bfloat16)
    model = PagedKVCacheModel(N)
    content = {}  # (layer, page) -> (k [P,H,D], v) on the CPU

    def insert(layer, t, conv, seed):
        k = randn((t, H, D), torch.bfloat16, dev, seed)
        v = randn((t, H, D), torch.bfloat16, dev, seed + 1)
        assert cache.insert_probe_kv(layer, k, v, conv)
        ids = model.allocate_pages(-(-t // P))
        model.insert(ids, t, P, conv)
        zeros = torch.zeros(P, H, D, dtype=torch.bfloat16)
        for j, pid in enumerate(ids):
            # A reused page keeps its old rows past the inserted ones.
            kk, vv = (x.clone() for x in content.get((layer, pid), (zeros, zeros)))
            n = min(P, t - j * P)
            kk[:n], vv[:n] = k.cpu()[j * P:j * P + n], v.cpu()[j * P:j * P + n]
            content[(layer, pid)] = (kk, vv)

    insert(0, 40, 0, 10)
    insert(1, 100, 1000, 20)
    got = cache.allocate_pages(2)
    assert got.tolist() == model.allocate_pages(2)   # allocated, never inserted
    insert(0, 16, 5000, 30)
    assert cache.evict_before(1016) == model.evict_before(1016)
    assert cache.free_pages == model.free_pages
    insert(0, 33, 7000, 40)  # reuses freed pages (LIFO)
    assert cache.evict_before(0) == model.evict_before(0) == 0
    assert cache.free_pages == model.free_pages
    st = cache.get_stats()
    assert st["active_pages"] == N - len(model.free_pages) and st["total_insertions"] == 40 + 100 + 16 + 33
    assert np.array_equal(cache.page_valid.cpu().numpy().astype(np.int8), model.page_valid)
    assert np.array_equal(cache.page_positions.cpu().numpy()[model.page_valid == 1],
                          model.page_positions[model.page_valid == 1])
    for layer in range(L):
        k, v = cache.get_layer_kv(layer)
        order = model.layer_order()
        assert k.shape == (len(order) * P, H, D)
        # Each layer's page holds what that layer last wrote there (zeros if never).
        zeros = torch.zeros(P, H, D, dtype=torch.bfloat16)
        want_k = torch.cat([content.get((layer, int(pid)), (zeros, zeros))[0] for pid in order])
        want_v = torch.cat([content.get((layer, int(pid)), (zeros, zeros))[1] for pid in order])
        assert torch.equal(k.cpu(), want_k) and torch.equal(v.cpu(), want_v)


class _Meta:
    def __init__(self, table, lens, slots):
        self.block_table, self.seq_lens, self.slot_mapping = table, lens, slots


@pytest.mark.parametrize("remap", [False, True])
def test_connector_save_and_recall(dev, monkeypatch, remap):
    from kessie_amd import kessie_kv_connector as kc

    monkeypatch.setattr(kc, "_KESSIE_STORE", None)
    monkeypatch.setattr(kc, "_RECALL_STATES", {})
    theta = 10000.0
    extra = {"max_cpu_gb": 1}
    if remap:
        extra["rope_theta"] = theta
    conn = kc.KeSSieKVConnector(kv_connector_extra_config=extra)
    kv = {"L0": randn((2, 32, 16, 8, 128), torch.bfloat16, dev, 1),
          "L1": randn((32, 2, 16, 8, 128), torch.bfloat16, dev, 2)}
    conn.register_kv_caches(kv)
    table = torch.tensor([[3, 7, 1]], dtype=torch.int32, device=dev)
    meta = _Meta(table, torch.tensor([40], dtype=torch.int32, device=dev),
                 torch.tensor([table[0, t // 16].item() * 16 + t % 16 for t in range(40)], device=dev))
    for name, cache in kv.items():
        conn.save_kv_layer(name, cache, meta)
    conn.wait_for_save()
    for name, cache in kv.items():
        kf = cache if name == "L0" else cache.transpose(0, 1)
        for bid, pos, tok in [(3, 0, 16), (7, 16, 16), (1, 32, 8)]:
            blk = conn.store.get_blocks_for_positions(pos, pos + tok, name)
            assert blk is not None and blk.block_id == bid
            assert torch.equal(blk.kv_data, kf[:, bid, :tok].cpu())
    saved = {name: [conn.store.get_blocks_for_positions(pos, 0, name).kv_data.clone() for pos in (0, 32)]
             for name in kv}

    # Recall positions 0..15 and 32..39 into freshly allocated blocks 20, 21.
    kc._RECALL_STATES["r"] = kc.RecallState(request_id="r", recalled_positions=[(0, 16), (32, 48)],
                                            num_recalled_tokens=24, load_pending=True, target_block_ids=[20, 21])
    before = {n: c.clone() for n, c in kv.items()}
    conn.start_load_kv()
    for name in kv:
        conn.wait_for_layer_load(name)
    torch.cuda.synchronize()
    assert not kc._RECALL_STATES["r"].load_pending
    for name, cache in kv.items():
        kf = cache if name == "L0" else cache.transpose(0, 1)
        bf = before[name] if name == "L0" else before[name].transpose(0, 1)
        want = torch.cat(saved[name], dim=1)  # [2, 24, H, D]
        got = torch.cat([kf[:, 20, :16], kf[:, 21, :8]], dim=1).cpu()
        assert torch.equal(got[1], want[1])  # V is copied unchanged
        if not remap:
            assert torch.equal(got[0], want[0])
        else:
            k_ref = want[0].clone()
            orig = torch.tensor(list(range(16)) + list(range(32, 40)), dtype=torch.int32)
            rope_remap_ref(k_ref, orig, torch.arange(24, dtype=torch.int32), theta)
            assert torch.equal(got[0][:16], want[0][:16])  # delta 0 is the identity
            assert (got[0].float() - k_ref.float()).abs().max().item() <= 2e-2
        # Untouched blocks stay as they were.
        mask = torch.ones(32, dtype=torch.bool)
        mask[[20, 21]] = False
        assert torch.equal(kf[:, mask].cpu(), bf[:, mask].cpu())


@pytest.mark.parametrize("remap", [False, True])
def test_connector_save_and_recall_32_token_blocks(dev, monkeypatch, remap):
    """The save and recall-inject path with 32-token blocks (both vLLM cache
    layouts): a 72-token sequence saved block by block, positions 32..71 recalled
    into two fresh blocks at positions 0..39 (K re-rotated by -32 when remapping)."""
    from kessie_amd import kessie_kv_connector as kc

    monkeypatch.setattr(kc, "_KESSIE_STORE", None)
    monkeypatch.setattr(kc, "_RECALL_STATES", {})
    theta, p = 10000.0, 32
    extra = {"max_cpu_gb": 1}
    if remap:
        extra["rope_theta"] = theta
    conn = kc.KeSSieKVConnector(kv_connector_extra_config=extra)
    kv = {"L0": randn((2, 16, p, 8, 128), torch.bfloat16, dev, 11),
          "L1": randn((16, 2, p, 8, 128), torch.bfloat16, dev, 12)}
    conn.register_kv_caches(kv)
    table = torch.tensor([[3, 7, 1]], dtype=torch.int32, device=dev)
    meta = _Meta(table, torch.tensor([72], dtype=torch.int32, device=dev),
                 torch.tensor([table[0, t // p].item() * p + t % p for t in range(72)], device=dev))
    for name, cache in kv.items():
        conn.save_kv_layer(name, cache, meta)
    conn.wait_for_save()
    for name, cache in kv.items():
        kf = cache if name == "L0" else cache.transpose(0, 1)
        for bid, pos, tok in [(3, 0, 32), (7, 32, 32), (1, 64, 8)]:
            blk = conn.store.get_blocks_for_positions(pos, pos + tok, name)
            assert blk is not None and blk.block_id == bid
            assert torch.equal(blk.kv_data, kf[:, bid, :tok].cpu())
    saved = {name: [conn.store.get_blocks_for_positions(pos, 0, name).kv_data.clone() for pos in (32, 64)]
             for name in kv}

    kc._RECALL_STATES["r"] = kc.RecallState(request_id="r", recalled_positions=[(32, 64), (64, 96)],
                                            num_recalled_tokens=40, load_pending=True, target_block_ids=[10, 11])
    before = {n: c.clone() for n, c in kv.items()}
    conn.start_load_kv()
    for name in kv:
        conn.wait_for_layer_load(name)
    torch.cuda.synchronize()
    assert not kc._RECALL_STATES["r"].load_pending
    for name, cache in kv.items():
        kf = cache if name == "L0" else cache.transpose(0, 1)
        bf = before[name] if name == "L0" else before[name].transpose(0, 1)
        want = torch.cat(saved[name], dim=1)  # [2, 40, H, D]
        got = torch.cat([kf[:, 10, :32], kf[:, 11, :8]], dim=1).cpu()
        assert torch.equal(got[1], want[1])  # V is copied unchanged
        if not remap:
            assert torch.equal(got[0], want[0])
        else:
            k_ref = want[0].clone()
            rope_remap_ref(k_ref, torch.arange(32, 72, dtype=torch.int32), torch.arange(40, dtype=torch.int32), theta)
            assert (got[0].float() - k_ref.float()).abs().max().item() <= 2e-2
        mask = torch.ones(16, dtype=torch.bool)
        mask[[10, 11]] = False
        assert torch.equal(kf[:, mask].cpu(), bf[:, mask].cpu())


@pytest.mark.parametrize("mode", ["written", "all"])
def test_connector_save_blocks_modes(dev, monkeypatch, mode):
    """A step that wrote only the last block: the default mode saves that
    block, save_blocks="all" every block of the sequence (the reference's
    plan), each with the cache's bytes."""
    from kessie_amd import kessie_kv_connector as kc

    monkeypatch.setattr(kc, "_KESSIE_STORE", None)
    conn = kc.KeSSieKVConnector(kv_connector_extra_config={"max_cpu_gb": 1, "save_blocks": mode})
    cache = randn((2, 32, 16, 8, 128), torch.bfloat16, dev, 5)
    conn.register_kv_caches({"L0": cache})
    table = torch.tensor([[3, 7, 1]], dtype=torch.int32, device=dev)
    meta = _Meta(table, torch.tensor([40], dtype=torch.int32, device=dev),
                 torch.tensor([1 * 16 + 7], device=dev))
    conn.save_kv_layer("L0", cache, meta)
    conn.wait_for_save()
    want = [(1, 32, 8)] if mode == "written" else [(3, 0, 16), (7, 16, 16), (1, 32, 8)]
    assert sorted(k[1] for k in conn.store._blocks) == sorted(b for b, _, _ in want)
    for bid, pos, tok in want:
        blk = conn.store.get_blocks_for_positions(pos, pos + tok, "L0")
        assert blk is not None and blk.block_id == bid
        assert torch.equal(blk.kv_data, cache[:, bid, :tok].cpu())


@pytest.mark.parametrize("dtype,rec", [(torch.bfloat16, [5, 250, 4000, 131071]), (torch.float16, [5, 250, 4000, 131071]),
                                       (torch.float32, [5, 250, 4000, 131071]),
                                       (torch.bfloat16, list(range(3, 131072, 41)) + [255, 256, 298, 299, 300, 300, -7])])
def test_fog_bias_rows_match_the_reference_vector_per_sequence(dev, dtype, rec):
    """Row b of the batched producer equals, bit for bit, the reference's op
    sequence run by torch on the same device for kv_len = seq_lens[b] (widened
    to fp32), zero past the row's length; recalled positions past a row's
    length leave it untouched."""
    from kessie_amd import ops

    lens = [0, 1, 7, 300, 4096, 131072, 999, 2]
    n = max(lens)
    out = torch.full((len(lens), n), float("nan"), dtype=torch.float32, device=dev)
    ops.fog_bias_rows(out, torch.tensor(lens, dtype=torch.int32, device=dev), dtype, 0.5, 0.5,
                      torch.tensor(rec, dtype=torch.int32, device=dev), 0.1)
    torch.cuda.synchronize()
    for b, ln in enumerate(lens):
        if ln:
            ref = fog_bias(ln, 0.5, 0.5, set(rec), 0.1, dtype=dtype, device=dev).reshape(-1).float()
            assert torch.equal(out[b, :ln], ref), f"row {b} (len {ln})"
        assert bool((out[b, ln:] == 0).all()), f"row {b} past its length"
