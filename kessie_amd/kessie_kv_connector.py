"""KeSSie KV connector: CPU-side lossless KV history with recall into the
paged GPU cache, on the MI355X kernels.

Mirrors the surface of the reference's kessie_kv_connector.py -- KVBlock
(:52-62), KeSSieCPUKVStore (:65-226), get_kessie_store (:236-243),
RecallState (:247-253) and KeSSieKVConnector with its hooks (:280-515) --
with the same names, signatures and defaults.  The data movement is
re-designed for the device:

  * save_kv_layer gathers the blocks written this step (those its
    slot_mapping touches) with page-gather launches into a device staging
    buffer and copies them to pinned host memory in ONE asynchronous transfer
    on a copy stream; the reference re-saves every block of every sequence
    each step with one ``.item()`` device sync per block-table entry plus one
    synchronous ``.cpu().clone()`` per block (:446-479).  Blocks reach the
    store once the transfer has completed (wait_for_save, or a later save).
  * start_load_kv packs the recalled blocks of a layer into one pinned buffer,
    moves it in ONE host-to-device copy and writes it into the blocks the
    scheduler allocated with one fused insert kernel, optionally re-rotating K
    from its original positions to the new ones (RoPE remap) on the way in;
    the reference copies block by block into the block id it was saved FROM
    (:413-427), not the slot allocated for the request.
  * the store's eviction keeps a min-heap on (timestamp, first-insertion
    order), so each eviction is O(log n) instead of a scan over every block
    (:203-215) while picking the same block.

Tensors crossing the hooks use the vLLM FLASH_ATTN cache layout
[2, num_blocks, block_size, num_kv_heads, head_dim] (:309); a
[num_blocks, 2, ...] cache is recognised from its shape.
"""
from __future__ import annotations

import hashlib
import heapq
import itertools
import logging
import threading
import time
from collections import defaultdict
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Set, Tuple

import numpy as np
import torch

logger = logging.getLogger("KeSSie.KVConnector")


# --- CPU KV block store ----------------------------------------------------------

@dataclass
class KVBlock:
    """A single KV cache block stored in CPU RAM (kessie_kv_connector.py:52-62)."""
    layer_name: str
    block_id: int
    token_ids: List[int]
    kv_data: Any                  # CPU tensor [2, tokens, H, D] -- exact copy from the GPU
    position_start: int
    position_end: int
    timestamp: float = 0.0
    embedding: Optional[np.ndarray] = None


def _nbytes(t) -> int:
    return t.nelement() * t.element_size() if hasattr(t, "nelement") else 0


class KeSSieCPUKVStore:
    """CPU-side KV block store with a semantic index (kessie_kv_connector.py:65-226)."""

    def __init__(self, max_cpu_bytes: int = 0, embed_dim: int = 256):
        self._lock = threading.Lock()
        self._blocks: Dict[Tuple[str, int], KVBlock] = {}
        self._position_index: Dict[int, List[Tuple[str, int]]] = defaultdict(list)
        self._semantic_index: List[Tuple[np.ndarray, int, int, List[int]]] = []
        self.embed_dim = embed_dim
        self.max_cpu_bytes = max_cpu_bytes
        self.total_bytes = 0
        self._embedder = None
        self.conversation_tokens: List[int] = []
        # Eviction order: (timestamp, first-insertion rank, key), stale entries
        # (replaced or evicted blocks) skipped lazily.
        self._heap: List[Tuple[float, int, Tuple[str, int]]] = []
        self._rank: Dict[Tuple[str, int], int] = {}
        self._counter = itertools.count()

    def set_embedder(self, fn):
        """Set the embedding function: text -> numpy vector."""
        self._embedder = fn

    def save_block(self, layer_name: str, block_id: int, kv_data, token_ids: List[int], position_start: int):
        """Save a KV block (copied to the CPU if it is a device tensor)."""
        if hasattr(kv_data, "cpu"):
            kv_data = kv_data.detach().cpu().clone()
        self._insert(layer_name, block_id, kv_data, token_ids, position_start)

    def _insert(self, layer_name, block_id, cpu_data, token_ids, position_start, timestamp=None):
        with self._lock:
            key = (layer_name, block_id)
            block = KVBlock(layer_name=layer_name, block_id=block_id, token_ids=list(token_ids), kv_data=cpu_data,
                            position_start=position_start, position_end=position_start + len(token_ids),
                            timestamp=time.time() if timestamp is None else timestamp)
            block_bytes = _nbytes(cpu_data)
            if self.max_cpu_bytes > 0:
                while self.total_bytes + block_bytes > self.max_cpu_bytes and self._blocks:
                    self._evict_oldest()
            old = self._blocks.get(key)
            if old is not None:
                self.total_bytes -= _nbytes(old.kv_data)
            else:
                self._rank[key] = next(self._counter)
            self._blocks[key] = block
            self._position_index[position_start].append(key)
            self.total_bytes += block_bytes
            heapq.heappush(self._heap, (block.timestamp, self._rank[key], key))

    def save_semantic_entry(self, token_ids: List[int], position_start: int, tokenizer=None):
        """Add a semantic index entry for a token range."""
        if self._embedder is None or tokenizer is None:
            return
        text = tokenizer.decode(token_ids, skip_special_tokens=True)
        if not text.strip():
            return
        emb = self._embedder(text)
        if emb is not None:
            with self._lock:
                self._semantic_index.append((emb, position_start, position_start + len(token_ids),
                                             list(token_ids)))

    def semantic_search(self, query_text: str, top_k: int = 5,
                        exclude_positions: Optional[Set[int]] = None) -> List[Tuple[int, int, float]]:
        """Cosine-similarity search of the semantic index:
        [(position_start, position_end, similarity)], best first."""
        if self._embedder is None or not self._semantic_index:
            return []
        query_emb = self._embedder(query_text)
        if query_emb is None:
            return []
        exclude = exclude_positions or set()
        results = []
        with self._lock:
            for emb, pos_start, pos_end, _ in self._semantic_index:
                if pos_start in exclude:
                    continue
                dot = np.dot(query_emb, emb)
                norm = np.linalg.norm(query_emb) * np.linalg.norm(emb)
                results.append((pos_start, pos_end, float(dot / max(norm, 1e-8))))
        results.sort(key=lambda x: -x[2])
        return results[:top_k]

    def get_blocks_for_positions(self, position_start: int, position_end: int,
                                 layer_name: str) -> Optional[KVBlock]:
        """The stored block of ``layer_name`` starting at position_start."""
        with self._lock:
            for key in self._position_index.get(position_start, []):
                if key[0] == layer_name and key in self._blocks:
                    block = self._blocks[key]
                    if block.position_start == position_start:
                        return block
        return None

    def get_all_blocks_for_range(self, position_start: int, position_end: int) -> Dict[str, List[KVBlock]]:
        """All layers' blocks starting inside [position_start, position_end)."""
        result: Dict[str, List[KVBlock]] = defaultdict(list)
        with self._lock:
            for pos in range(position_start, position_end):
                for key in self._position_index.get(pos, []):
                    if key in self._blocks:
                        block = self._blocks[key]
                        result[block.layer_name].append(block)
        return dict(result)

    def _evict_oldest(self):
        """Evict the block with the smallest timestamp (ties: first inserted)."""
        while self._heap:
            ts, rank, key = heapq.heappop(self._heap)
            block = self._blocks.get(key)
            if block is None or block.timestamp != ts or self._rank.get(key) != rank:
                continue  # replaced or already evicted
            del self._blocks[key]
            del self._rank[key]
            self.total_bytes -= _nbytes(block.kv_data)
            pos_keys = self._position_index.get(block.position_start, [])
            if key in pos_keys:
                pos_keys.remove(key)
            return

    def stats(self) -> Dict[str, Any]:
        with self._lock:
            return {
                "total_blocks": len(self._blocks),
                "total_bytes": self.total_bytes,
                "total_mb": self.total_bytes / 1048576,
                "semantic_entries": len(self._semantic_index),
                "conversation_tokens": len(self.conversation_tokens),
                "position_ranges": len(self._position_index),
            }


_KESSIE_STORE: Optional[KeSSieCPUKVStore] = None
_KESSIE_STORE_LOCK = threading.Lock()


_HASH_TOKENS = None


def recall_query_text(token_ids: List[int]) -> str:
    """The semantic-search query for a prompt (kessie_kv_connector.py:335-344):
    the md5 of the bytes of its last 128 token ids when transformers is
    importable, of its last 64 otherwise.  The reference's ``bytes()`` raises
    for an id above 255 (and the scheduler call with it); here such an id
    contributes its low byte, so large vocabularies still get a query."""
    global _HASH_TOKENS
    if _HASH_TOKENS is None:
        import importlib.util

        _HASH_TOKENS = 128 if importlib.util.find_spec("transformers") is not None else 64
    tail = token_ids[-_HASH_TOKENS:]
    return f"tokens:{hashlib.md5(bytes(t & 0xFF for t in tail)).hexdigest()}"


def get_kessie_store(max_cpu_bytes: int = 0) -> KeSSieCPUKVStore:
    """The process-wide store (created on first use)."""
    global _KESSIE_STORE
    with _KESSIE_STORE_LOCK:
        if _KESSIE_STORE is None:
            _KESSIE_STORE = KeSSieCPUKVStore(max_cpu_bytes=max_cpu_bytes)
            logger.info(f"KeSSie CPU KV Store initialized (max {max_cpu_bytes / 1073741824:.1f} GB)")
        return _KESSIE_STORE


@dataclass
class RecallState:
    """Which distant KV ranges are recalled for a request (kessie_kv_connector.py:247-253).
    target_block_ids: the cache blocks the scheduler allocated for them."""
    request_id: str = ""
    recalled_positions: List[Tuple[int, int]] = field(default_factory=list)
    num_recalled_tokens: int = 0
    load_pending: bool = False
    target_block_ids: List[int] = field(default_factory=list)


_RECALL_STATES: Dict[str, RecallState] = {}
_RECALL_LOCK = threading.Lock()


# --- Connector ------------------------------------------------------------------

try:
    from vllm.distributed.kv_transfer.kv_connector.v1.base import KVConnectorBase_v1
    HAS_VLLM_CONNECTOR = True
except ImportError:
    HAS_VLLM_CONNECTOR = False

    class KVConnectorBase_v1:  # stand-in base when vLLM is absent
        def __init__(self, *args, **kwargs):
            pass


def _layout(kv: torch.Tensor) -> str:
    if kv.dim() == 5 and kv.shape[1] == 2 and kv.shape[0] != 2:
        return "block_kv"
    return "kv_first"


def _halves(kv: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """K and V page arrays [blocks, P, H, D] of a cache in either layout."""
    return (kv[0], kv[1]) if _layout(kv) == "kv_first" else (kv[:, 0], kv[:, 1])


class KeSSieKVConnector(KVConnectorBase_v1):
    """vLLM V1 KV connector: saves every computed KV block to the CPU store and
    loads semantically recalled blocks back into the request's cache blocks
    (kessie_kv_connector.py:280-515).

    kv_connector_extra_config keys: ``max_cpu_gb`` (default 64),
    ``rope_theta`` (default None: recalled K is copied unchanged; a value
    re-rotates K from its original positions to its new ones while loading)
    and ``save_blocks``: ``"written"`` (default) saves the blocks this step's
    slot_mapping touched; ``"all"`` re-saves every block of every sequence
    each step, as the reference does (kessie_kv_connector.py:459-483), which
    refreshes every block's timestamp and so reproduces its eviction order
    under ``max_cpu_gb`` at the cost of copying the whole context per step.
    """

    def __init__(self, *args, **kwargs):
        # The extra config comes as a keyword (as the reference reads it) or
        # inside vllm_config.kv_transfer_config (as vLLM hands it over); it is
        # not passed on to the base class, whose signature does not take it.
        extra = kwargs.pop("kv_connector_extra_config", None)
        if extra is None:
            vc = args[0] if args else kwargs.get("vllm_config")
            extra = getattr(getattr(vc, "kv_transfer_config", None), "kv_connector_extra_config", None)
        extra = extra or {}
        super().__init__(*args, **kwargs)
        max_gb = float(extra.get("max_cpu_gb", 64))
        self.store = get_kessie_store(max_cpu_bytes=int(max_gb * 1073741824))
        self.rope_theta = extra.get("rope_theta")
        mode = extra.get("save_blocks", "written")
        if mode not in ("written", "all"):
            raise ValueError(f"save_blocks must be 'written' or 'all', not {mode!r}")
        self._save_all = mode == "all"
        self._kv_caches = []
        self._layer_names = []
        self._block_size = 16
        self._copy_streams: Dict[int, torch.cuda.Stream] = {}
        self._pending_saves: List[Tuple[torch.cuda.Event, list]] = []
        self._step = 0  # forward steps seen by this worker (start_load_kv runs once per step)
        self._scratch: Dict[Tuple[int, int], Tuple[torch.Tensor, torch.Tensor]] = {}
        logger.info(f"KeSSieKVConnector initialized (CPU budget: {max_gb:.0f} GB)")

    # -- registration ------------------------------------------------------------
    def register_kv_caches(self, kv_caches, layer_names=None, **kwargs):
        """References to the GPU KV cache tensors (one per layer)."""
        if isinstance(kv_caches, dict):
            layer_names = list(kv_caches.keys()) if layer_names is None else layer_names
            kv_caches = [kv_caches[n] for n in layer_names]
        self._kv_caches = list(kv_caches)
        self._layer_names = list(layer_names or [])
        if self._kv_caches and hasattr(self._kv_caches[0], "shape") and self._kv_caches[0].dim() >= 4:
            self._block_size = int(_halves(self._kv_caches[0])[0].shape[1])
        logger.info(f"  KV caches registered: {len(self._layer_names)} layers, block_size={self._block_size}")

    # -- scheduler side ------------------------------------------------------------
    def get_num_new_matched_tokens(self, request, *args, **kwargs) -> int:
        """Tokens of distant context the store can supply for ``request``
        (kessie_kv_connector.py:330-386): semantic search with the hash of the
        last prompt tokens, ranges with similarity >= 0.3 among the top 3."""
        token_ids = list(request.prompt_token_ids) if hasattr(request, "prompt_token_ids") else []
        if not token_ids:
            return 0
        req_id = str(request.request_id) if hasattr(request, "request_id") else ""
        with _RECALL_LOCK:
            if req_id in _RECALL_STATES:
                return _RECALL_STATES[req_id].num_recalled_tokens
        results = self.store.semantic_search(recall_query_text(token_ids), top_k=3, exclude_positions=set())
        recalled, total = [], 0
        for pos_start, pos_end, sim in results:
            if sim < 0.3:
                continue
            recalled.append((pos_start, pos_end))
            total += pos_end - pos_start
        if total > 0:
            with _RECALL_LOCK:
                _RECALL_STATES[req_id] = RecallState(request_id=req_id, recalled_positions=recalled,
                                                     num_recalled_tokens=total, load_pending=True)
            logger.info(f"KeSSie recall: {total} tokens from {len(recalled)} distant ranges")
        return total

    def update_state_after_alloc(self, request, blocks, num_external_tokens, **kwargs):
        """Record the cache blocks the scheduler allocated for the recalled
        tokens (the request's first ceil(num_external_tokens / block_size))."""
        req_id = str(request.request_id) if hasattr(request, "request_id") else ""
        with _RECALL_LOCK:
            state = _RECALL_STATES.get(req_id)
            if state and num_external_tokens > 0:
                ids = blocks.get_block_ids() if hasattr(blocks, "get_block_ids") else blocks
                if ids and isinstance(ids[0], (list, tuple)):
                    ids = ids[0]
                n = -(-num_external_tokens // self._block_size)
                state.target_block_ids = [int(x) for x in list(ids)[:n]]
                state.load_pending = True

    def build_connector_meta(self, scheduler_output, **kwargs):
        """Metadata for this step (none: recall state is process-global)."""
        return None

    def request_finished(self, request, block_ids, **kwargs):
        """Drop the request's recall state; CPU blocks stay (conversation history)."""
        req_id = str(request.request_id) if hasattr(request, "request_id") else ""
        with _RECALL_LOCK:
            _RECALL_STATES.pop(req_id, None)
        return (False, None)

    # -- worker side: load ------------------------------------------------------------
    def start_load_kv(self, kv_caches=None, layer_names=None, **kwargs):
        """Copy the recalled blocks of every pending request into its
        allocated cache blocks: per layer one pinned H2D copy and one fused
        insert (+ optional RoPE remap) launch, on the copy stream."""
        from . import ops

        self._step += 1
        caches = kv_caches if kv_caches is not None else self._kv_caches
        names = layer_names if layer_names is not None else self._layer_names
        if isinstance(caches, dict):
            names = list(caches.keys()) if not names else names
            caches = [caches[n] for n in names]
        with _RECALL_LOCK:
            pending = {k: v for k, v in _RECALL_STATES.items() if v.load_pending}
        if not pending or not caches:
            return
        for req_id, state in pending.items():
            if not state.target_block_ids:
                continue
            for li, name in enumerate(names):
                if li >= len(caches):
                    break
                blocks = [self.store.get_blocks_for_positions(s, e, name) for s, e in state.recalled_positions]
                blocks = [b for b in blocks if b is not None]
                if not blocks:
                    continue
                self._load_layer(ops, caches[li], blocks, state.target_block_ids)
            with _RECALL_LOCK:
                state.load_pending = False

    def _scratch_for(self, device, num_blocks):
        key = (device.index if device.index is not None else 0, num_blocks)
        if key not in self._scratch:
            self._scratch[key] = (torch.zeros(num_blocks, dtype=torch.int8, device=device),
                                  torch.zeros(num_blocks, dtype=torch.int32, device=device))
        return self._scratch[key]

    def _load_layer(self, ops, gpu_cache, blocks, target_ids):
        k_pages, v_pages = _halves(gpu_cache)
        num_blocks, p, h, d = k_pages.shape
        n_tok = min(sum(b.kv_data.shape[1] for b in blocks), len(target_ids) * p)
        if n_tok == 0:
            return
        host = torch.empty(2, n_tok, h, d, dtype=gpu_cache.dtype, pin_memory=True)
        orig = torch.empty(n_tok, dtype=torch.int32, pin_memory=True)
        at = 0
        for b in blocks:
            take = min(b.kv_data.shape[1], n_tok - at)
            if take <= 0:
                break
            host[:, at:at + take].copy_(b.kv_data[:, :take])
            orig[at:at + take] = torch.arange(b.position_start, b.position_start + take, dtype=torch.int32)
            at += take
        stream = self._get_copy_stream(gpu_cache.device)
        stream.wait_stream(torch.cuda.current_stream(gpu_cache.device))
        with torch.cuda.stream(stream):
            dev = host.to(gpu_cache.device, non_blocking=True)
            tgt_pages = torch.tensor(target_ids[: -(-n_tok // p)], dtype=torch.int32).pin_memory().to(
                gpu_cache.device, non_blocking=True)
            valid, positions = self._scratch_for(gpu_cache.device, num_blocks)
            remap = {}
            if self.rope_theta is not None:
                remap = dict(orig_pos=orig.to(gpu_cache.device, non_blocking=True),
                             tgt_pos=torch.arange(n_tok, dtype=torch.int32, device=gpu_cache.device),
                             rope_theta=float(self.rope_theta))
            ops.page_insert(gpu_cache, dev[0], dev[1], tgt_pages, valid, positions, 0,
                            layout=_layout(gpu_cache), **remap)
            for t in [dev, tgt_pages, *remap.values()]:
                if isinstance(t, torch.Tensor):
                    t.record_stream(stream)

    def wait_for_layer_load(self, layer_name: str, **kwargs):
        """Order the compute stream after the loads (no host wait)."""
        for dev_idx, stream in self._copy_streams.items():
            torch.cuda.current_stream(dev_idx).wait_stream(stream)

    # -- worker side: save ------------------------------------------------------------
    def save_kv_layer(self, layer_name: str, kv_layer, attn_metadata, **kwargs):
        """Copy the layer's blocks of this step's save plan (by default those
        its slot_mapping touches) to the CPU store: page gathers into a device
        staging buffer, then one async D2H copy into pinned memory."""
        from . import ops

        plan = self._save_plan(attn_metadata)
        if not plan or kv_layer is None:
            return
        self._flush_saves(block=False)
        p = self._block_size
        n = len(plan)
        layout = _layout(kv_layer)
        k_pages, _ = _halves(kv_layer)
        _, _, h, d = k_pages.shape
        stream = self._get_copy_stream(kv_layer.device)
        stream.wait_stream(torch.cuda.current_stream(kv_layer.device))
        idx = torch.tensor([b for b, _, _ in plan], dtype=torch.int32).pin_memory()
        with torch.cuda.stream(stream):
            idx_dev = idx.to(kv_layer.device, non_blocking=True)
            if layout == "kv_first":   # K pages and V pages are two contiguous arrays
                staging = torch.empty(2, n, p, h, d, dtype=kv_layer.dtype, device=kv_layer.device)
                ops.page_gather(kv_layer[0], idx_dev, out=staging[0])
                ops.page_gather(kv_layer[1], idx_dev, out=staging[1])
            else:                      # [blocks, 2, P, H, D]: whole blocks
                staging = torch.empty(n, 2, p, h, d, dtype=kv_layer.dtype, device=kv_layer.device)
                ops.page_gather(kv_layer, idx_dev, out=staging)
            host = torch.empty(staging.shape, dtype=kv_layer.dtype, pin_memory=True)
            host.copy_(staging, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(stream)
            staging.record_stream(stream)
            idx_dev.record_stream(stream)
        if layout == "kv_first":
            entries = [(layer_name, bid, host[:, i, :tok], pos) for i, (bid, pos, tok) in enumerate(plan)]
        else:
            entries = [(layer_name, bid, host[i, :, :tok], pos) for i, (bid, pos, tok) in enumerate(plan)]
        self._pending_saves.append((ev, entries))

    def _save_plan(self, meta):
        """[(block_id, position_start, tokens)] of the blocks to save this step
        (those written this step, or every block with ``save_blocks="all"``),
        computed once per step and metadata object (all layers of the step
        share it; a runner that refills one metadata object in place is seen
        again on the next step, which start_load_kv counts).  Table entries
        below zero (padding) are skipped."""
        if meta is None:
            return []
        key = (self._step, id(meta))
        if getattr(self, "_plan_key", None) == key and getattr(self, "_plan_meta", None) is meta:
            return self._plan
        block_tables = getattr(meta, "block_tables", None)
        if block_tables is None:
            block_tables = getattr(meta, "block_table", None)
        seq_lens = getattr(meta, "seq_lens", None)
        slots = getattr(meta, "slot_mapping", None)
        plan = []
        if block_tables is not None and seq_lens is not None:
            p = self._block_size
            tables = block_tables.cpu() if isinstance(block_tables, torch.Tensor) else torch.tensor(block_tables)
            lens = seq_lens.tolist() if hasattr(seq_lens, "tolist") else list(seq_lens)
            touched = None
            if slots is not None and not self._save_all:
                sl = slots.cpu() if isinstance(slots, torch.Tensor) else torch.tensor(slots)
                touched = set((sl[sl >= 0] // p).tolist())
            for si in range(min(len(lens), tables.shape[0])):
                n = int(lens[si])
                for bi in range(-(-n // p)):
                    bid = int(tables[si, bi])
                    if bid < 0 or (touched is not None and bid not in touched):
                        continue
                    plan.append((bid, bi * p, min(p, n - bi * p)))
        self._plan_meta, self._plan_key, self._plan = meta, key, plan
        return plan

    def _flush_saves(self, block: bool):
        keep = []
        for ev, entries in self._pending_saves:
            if block:
                ev.synchronize()
            elif not ev.query():
                keep.append((ev, entries))
                continue
            for layer_name, bid, data, pos in entries:
                self.store._insert(layer_name, bid, data, [], pos)
        self._pending_saves = keep

    def wait_for_save(self, **kwargs):
        """Block until every pending save has landed in the store."""
        self._flush_saves(block=True)

    def _get_copy_stream(self, device) -> torch.cuda.Stream:
        dev_idx = device.index if getattr(device, "index", None) is not None else 0
        if dev_idx not in self._copy_streams:
            self._copy_streams[dev_idx] = torch.cuda.Stream(device=device)
        return self._copy_streams[dev_idx]
