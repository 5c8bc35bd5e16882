"""CPU: the Python surface mirrored from kessie_attention.py and
kessie_kv_connector.py -- state, backend metadata, impl argument parsing,
the CPU KV store (eviction order pinned against the reference's linear-scan
restatement in oracle/store.py) and the connector's scheduler-side hooks."""
import random

import numpy as np
import pytest
import torch

from oracle.store import StoreModel


def test_attention_state_update_and_get():
    from kessie_amd.kessie_attention import KESSIE_STATE, KeSSieAttentionState

    st = KeSSieAttentionState()
    assert st.get() == {"fog_alpha": 0.5, "fog_start": 0.5, "prompt_len": 0, "recall_positions": set(),
                        "recall_boost": 0.1, "enabled": True, "generation": 0}
    st.update(fog_alpha=0.8, recall_positions=[3, 5, 3])
    g = st.get()
    assert g["fog_alpha"] == 0.8 and g["recall_positions"] == {3, 5} and g["generation"] == 1
    g["recall_positions"].add(99)  # get() returns a copy
    assert st.get()["recall_positions"] == {3, 5}
    st.update()
    assert st.get()["generation"] == 2
    assert isinstance(KESSIE_STATE, KeSSieAttentionState)


def test_backend_surface_without_vllm():
    from kessie_amd import kessie_attention as ka

    assert ka.KeSSieAttentionBackend.get_name() == "KeSSie"
    assert ka.KeSSieAttentionBackend.get_impl_cls() is ka.KeSSieAttentionImpl
    if not ka.HAS_VLLM:
        assert ka.register_kessie_attention() is False
        assert ka.KeSSieAttentionBackend.get_metadata_cls() is ka.KeSSieAttentionMetadata
        assert ka.KeSSieAttentionBackend.get_kv_cache_shape(100, 16, 8, 128) == (2, 100, 16, 8, 128)


def test_impl_arguments_follow_vllm_order():
    from kessie_amd.kessie_attention import KeSSieAttentionImpl

    a = KeSSieAttentionImpl(32, 128, 0.125, 8, None, 1024)
    assert (a.num_heads, a.head_size, a.scale, a.num_kv_heads, a.window) == (32, 128, 0.125, 8, 1024)
    b = KeSSieAttentionImpl(num_heads=8, head_size=64, scale=None, sliding_window=(127, 0))
    assert b.num_kv_heads == 8 and b.window == 128 and b.scale == pytest.approx(64 ** -0.5)
    assert not b.unsupported
    assert KeSSieAttentionImpl(8, 64, 0.1, 8, None, None, "auto", 30.0).unsupported
    with pytest.raises(AttributeError):
        _ = a.some_inner_attribute  # no inner impl without vLLM


def _block(nbytes):
    return torch.zeros(nbytes, dtype=torch.uint8)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_store_eviction_matches_reference_scan(seed):
    """Random saves (new keys, replacements, timestamp ties) under a byte
    budget: the heap-based store evicts exactly what the reference's
    min-over-dict scan evicts, and keeps the same byte count."""
    from kessie_amd.kessie_kv_connector import KeSSieCPUKVStore

    rng = random.Random(seed)
    budget = 2000
    store = KeSSieCPUKVStore(max_cpu_bytes=budget)
    model = StoreModel(max_cpu_bytes=budget)
    evicted = []
    orig = store._evict_oldest

    def spy():
        before = set(store._blocks)
        orig()
        evicted.extend(sorted(before - set(store._blocks)))
    store._evict_oldest = spy
    for step in range(400):
        key = (f"layer{rng.randrange(3)}", rng.randrange(40))
        nbytes = rng.choice([50, 100, 150, 200])
        ts = float(rng.randrange(60))  # many ties
        pos = rng.randrange(10) * 16
        store._insert(key[0], key[1], _block(nbytes), [], pos, timestamp=ts)
        model.save(key, nbytes, pos, ts)
        assert store.total_bytes == model.total_bytes
        assert set(store._blocks) == set(model.blocks)
    assert evicted == model.evicted
    assert len(evicted) > 50


def test_store_lookup_and_stats():
    from kessie_amd.kessie_kv_connector import KeSSieCPUKVStore

    s = KeSSieCPUKVStore()
    s.save_block("L0", 7, torch.ones(2, 16, 2, 4), list(range(16)), 32)
    s.save_block("L1", 7, torch.ones(2, 16, 2, 4), list(range(16)), 32)
    b = s.get_blocks_for_positions(32, 48, "L1")
    assert b is not None and b.layer_name == "L1" and b.position_end == 48
    assert s.get_blocks_for_positions(16, 32, "L1") is None
    assert set(s.get_all_blocks_for_range(0, 64)) == {"L0", "L1"}
    st = s.stats()
    assert st["total_blocks"] == 2 and st["total_bytes"] == 2 * 2 * 16 * 2 * 4 * 4


def test_semantic_search_ranks_by_cosine():
    from kessie_amd.kessie_kv_connector import KeSSieCPUKVStore

    vecs = {"a": np.array([1.0, 0.0]), "b": np.array([0.6, 0.8]), "c": np.array([0.0, 1.0]),
            "q": np.array([1.0, 0.1])}

    class Tok:
        def decode(self, ids, skip_special_tokens=True):
            return ids[0]

    s = KeSSieCPUKVStore()
    s.set_embedder(lambda text: vecs[text])
    for i, name in enumerate("abc"):
        s.save_semantic_entry([name], i * 100, tokenizer=Tok())
    res = s.semantic_search("q", top_k=2)
    assert [r[0] for r in res] == [0, 100]
    assert res[0][2] == pytest.approx(float(vecs["q"] @ vecs["a"] / np.linalg.norm(vecs["q"])))
    assert [r[0] for r in s.semantic_search("q", top_k=5, exclude_positions={0})] == [100, 200]


class _Req:
    def __init__(self, rid, toks):
        self.request_id = rid
        self.prompt_token_ids = toks


class _Blocks:
    def __init__(self, ids):
        self._ids = ids

    def get_block_ids(self):
        return [self._ids]


def test_connector_scheduler_hooks(monkeypatch):
    from kessie_amd import kessie_kv_connector as kc

    monkeypatch.setattr(kc, "_KESSIE_STORE", None)
    monkeypatch.setattr(kc, "_RECALL_STATES", {})
    conn = kc.KeSSieKVConnector(kv_connector_extra_config={"max_cpu_gb": 1})
    hits = [(0, 48, 0.9), (64, 80, 0.2), (128, 160, 0.5)]
    monkeypatch.setattr(conn.store, "semantic_search", lambda text, top_k=5, exclude_positions=None: hits)
    req = _Req("r1", list(range(200)))
    assert conn.get_num_new_matched_tokens(req) == 48 + 32
    st = kc._RECALL_STATES["r1"]
    assert st.recalled_positions == [(0, 48), (128, 160)] and st.load_pending
    assert conn.get_num_new_matched_tokens(req) == 80  # cached per request
    conn.update_state_after_alloc(req, _Blocks([9, 4, 7, 1, 3, 8, 2]), 80)
    assert st.target_block_ids == [9, 4, 7, 1, 3]
    assert conn.get_num_new_matched_tokens(_Req("r2", [])) == 0
    assert conn.build_connector_meta(None) is None
    assert conn.request_finished(req, [9, 4]) == (False, None)
    assert "r1" not in kc._RECALL_STATES


def test_connector_save_plan_uses_slot_mapping():
    from kessie_amd import kessie_kv_connector as kc

    class Meta:
        block_table = torch.tensor([[5, 2, 9, 0], [7, 1, 0, 0]], dtype=torch.int32)
        seq_lens = torch.tensor([40, 20], dtype=torch.int32)
        # Step wrote seq 0's tokens 32..39 (block 9) and seq 1's token 19 (block 1).
        slot_mapping = torch.tensor([9 * 16 + i for i in range(8)] + [1 * 16 + 3, -1], dtype=torch.int64)

    conn = kc.KeSSieKVConnector()
    meta = Meta()
    assert conn._save_plan(meta) == [(9, 32, 8), (1, 16, 4)]
    assert conn._save_plan(meta) is conn._plan  # cached per metadata object


def test_connector_save_plan_follows_metadata_refilled_in_place():
    """A runner that reuses one metadata object and refills its tensors
    between steps gets a fresh plan on the next step (start_load_kv counts
    the steps); within a step the plan is shared by the layers."""
    from kessie_amd import kessie_kv_connector as kc

    class Meta:
        block_table = torch.tensor([[5, 2, 9, 0]], dtype=torch.int32)
        seq_lens = torch.tensor([40], dtype=torch.int32)
        slot_mapping = torch.tensor([9 * 16 + 7], dtype=torch.int64)

    conn = kc.KeSSieKVConnector()
    meta = Meta()
    conn.start_load_kv(kv_caches=[], layer_names=[])
    assert conn._save_plan(meta) == [(9, 32, 8)]
    meta.seq_lens[0] = 41                      # next step, same object, refilled in place
    meta.block_table[0, 2] = 3
    meta.slot_mapping[0] = 3 * 16 + 8
    assert conn._save_plan(meta) == [(9, 32, 8)]  # same step: the shared plan
    conn.start_load_kv(kv_caches=[], layer_names=[])
    assert conn._save_plan(meta) == [(3, 32, 9)]


def test_connector_save_all_blocks_matches_the_reference_plan():
    """save_blocks="all" saves what the reference's save_kv_layer saves, in
    its order: every block of every sequence, each step."""
    from kessie_amd import kessie_kv_connector as kc
    from oracle.store import reference_save_plan

    class Meta:
        block_table = torch.tensor([[5, 2, 9, 0], [7, 1, 0, 0], [3, 4, 6, 8]], dtype=torch.int32)
        seq_lens = torch.tensor([40, 20, 64], dtype=torch.int32)
        slot_mapping = torch.tensor([9 * 16 + 7, 1 * 16 + 3, 8 * 16 + 15], dtype=torch.int64)

    conn = kc.KeSSieKVConnector(kv_connector_extra_config={"save_blocks": "all"})
    meta = Meta()
    want = reference_save_plan(Meta.block_table.tolist(), Meta.seq_lens.tolist(), 16)
    assert want == [(5, 0, 16), (2, 16, 16), (9, 32, 8), (7, 0, 16), (1, 16, 4),
                    (3, 0, 16), (4, 16, 16), (6, 32, 16), (8, 48, 16)]
    assert conn._save_plan(meta) == want
    # the default saves only the written blocks, in the same order
    assert kc.KeSSieKVConnector()._save_plan(meta) == [(9, 32, 8), (1, 16, 4), (8, 48, 16)]
    with pytest.raises(ValueError):
        kc.KeSSieKVConnector(kv_connector_extra_config={"save_blocks": "some"})


def test_connector_save_all_blocks_reproduces_the_reference_eviction_order():
    """Under a byte budget, saving the reference's plan each step (every
    block re-saved, so every timestamp refreshed) leaves the store holding
    what the reference's store holds after every step."""
    from kessie_amd import kessie_kv_connector as kc
    from oracle.store import StoreModel, reference_save_plan

    tables = [[5, 2, 9, 0], [7, 1, 0, 0]]
    lens_by_step = [[40, 20], [41, 20], [42, 21]]
    nbytes = 64
    budget = 5 * nbytes
    store = kc.KeSSieCPUKVStore(max_cpu_bytes=budget)
    model = StoreModel(max_cpu_bytes=budget)
    ts = 0.0
    for lens in lens_by_step:
        for bid, pos, tok in reference_save_plan(tables, lens, 16):
            ts += 1.0
            store._insert("layer.0", bid, torch.zeros(nbytes, dtype=torch.uint8), [], pos, timestamp=ts)
            model.save(("layer.0", bid), nbytes, pos, ts)
        assert sorted(store._blocks) == sorted(model.blocks)
        assert store.total_bytes == model.total_bytes
    assert model.evicted  # the budget was exceeded along the way


def test_recall_query_text_matches_the_reference_for_byte_token_ids(monkeypatch):
    """The semantic-search query equals the reference's for every prompt whose
    token ids fit in a byte (the only prompts the reference handles); above
    255 the reference's bytes() raises and this one takes the low byte."""
    import random

    from kessie_amd import kessie_kv_connector as kc
    from oracle.store import reference_query_text

    rng = random.Random(3)
    for n in (1, 63, 64, 65, 127, 128, 129, 500):
        ids = [rng.randrange(256) for _ in range(n)]
        for importable in (True, False):
            monkeypatch.setattr(kc, "_HASH_TOKENS", 128 if importable else 64)
            assert kc.recall_query_text(ids) == reference_query_text(ids, importable)
    big = [300, 70000, 5]
    with pytest.raises(ValueError):
        reference_query_text(big)
    monkeypatch.setattr(kc, "_HASH_TOKENS", 128)
    assert kc.recall_query_text(big) == reference_query_text([t & 0xFF for t in big])


def test_attention_split_follows_metadata_refilled_in_place():
    """The decode / prefill split is keyed by the content of
    query_start_loc_cpu, not by the metadata object."""
    from kessie_amd import kessie_attention as ka

    class Meta:
        query_start_loc_cpu = torch.tensor([0, 1, 5, 6], dtype=torch.int32)

    meta = Meta()
    qsl, dec, pre = ka.KeSSieAttentionImpl._split(meta)
    assert (qsl, dec, pre) == ([0, 1, 5, 6], [0, 2], [1])
    meta.query_start_loc_cpu[1:] = torch.tensor([3, 4, 5], dtype=torch.int32)
    qsl, dec, pre = ka.KeSSieAttentionImpl._split(meta)
    assert (qsl, dec, pre) == ([0, 3, 4, 5], [1, 2], [0])


def test_attention_split_is_consistent_under_concurrent_callers():
    """Two threads alternating metadata of different decode / prefill splits
    always get the split of their own metadata (the cached key and value are
    one attribute, never paired across calls)."""
    import threading

    from kessie_amd import kessie_attention as ka

    class Meta:
        def __init__(self, qsl):
            self.query_start_loc_cpu = torch.tensor(qsl, dtype=torch.int32)

    cases = [([0, 1, 5, 6], [0, 2], [1]), ([0, 4, 5, 6, 9], [1, 2], [0, 3]), ([0, 1, 2], [0, 1], [])]
    errors = []

    def worker(order):
        metas = [(Meta(q), (q, d, p)) for q, d, p in cases]
        for i in range(4000):
            meta, want = metas[order[i % len(order)]]
            got = ka.KeSSieAttentionImpl._split(meta)
            if got != want:
                errors.append((got, want))
                return

    threads = [threading.Thread(target=worker, args=(o,)) for o in ([0, 1, 2], [2, 1, 0], [1, 0, 2, 2])]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:3]


def test_fog_bias_rows_cache_is_consistent_under_concurrent_callers(monkeypatch):
    """get_fog_bias_rows under two threads with different length tuples (the
    device fill replaced by a CPU stand-in that writes each row's length): every
    returned view has its own caller's rows, and the cached key and view are
    replaced together."""
    import threading

    from kessie_amd import kessie_attention as ka
    from kessie_amd import ops

    def fake_rows(view, lens, dtype, alpha, start, recall, boost):
        for r in range(view.shape[0]):
            view[r].fill_(float(lens[r]))

    monkeypatch.setattr(ops, "fog_bias_rows", fake_rows)
    cache = ka._FogCache()
    state = {"generation": 3, "recall_positions": set(), "fog_alpha": 0.5, "fog_start": 0.5, "recall_boost": 0.1}
    sets = [torch.tensor([5, 7], dtype=torch.int32), torch.tensor([9, 2, 4], dtype=torch.int32)]
    errors = []

    def worker(k):
        for i in range(2000):
            lens = sets[(i + k) % 2]
            v = cache.get_fog_bias_rows(lens, 16, "cpu", torch.float32, state, seq_lens_host=lens)
            if v.shape != (lens.numel(), 16):  # a key paired with another call's view
                errors.append((k, i, tuple(v.shape)))
                return

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:3]
    # The key and the view are replaced together.
    key, view = cache._rows_cache
    assert key[-1] == tuple(int(x) for x in view[:, 0].tolist())
