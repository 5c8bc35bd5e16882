"""CPU KV store bookkeeping oracle (test infrastructure only), and the
reference connector's save plan and recall query.

Restates KeSSieCPUKVStore.save_block / _evict_oldest
(kessie_kv_connector.py:91-139, 203-215) as the reference does it: blocks in
an insertion-ordered dict keyed by (layer_name, block_id); before inserting,
while the byte budget would be exceeded, evict the block with the smallest
timestamp by a linear scan (``min`` over the dict's keys, so ties go to the
key inserted first); replacing a key keeps its dict position.  Only the
bookkeeping is modelled: (key, timestamp, bytes, position_start).
"""
from __future__ import annotations

from collections import defaultdict


class StoreModel:
    def __init__(self, max_cpu_bytes: int = 0):
        self.max_cpu_bytes = max_cpu_bytes
        self.blocks: dict = {}          # key -> (timestamp, nbytes, position_start)
        self.position_index = defaultdict(list)
        self.total_bytes = 0
        self.evicted: list = []

    def save(self, key, nbytes: int, position_start: int, timestamp: float):
        if self.max_cpu_bytes > 0:
            while self.total_bytes + nbytes > self.max_cpu_bytes and self.blocks:
                self._evict_oldest()
        old = self.blocks.get(key)
        if old is not None:
            self.total_bytes -= old[1]
        self.blocks[key] = (timestamp, nbytes, position_start)
        self.position_index[position_start].append(key)
        self.total_bytes += nbytes

    def _evict_oldest(self):
        oldest = min(self.blocks.keys(), key=lambda k: self.blocks[k][0])
        ts, nbytes, pos = self.blocks.pop(oldest)
        self.total_bytes -= nbytes
        keys = self.position_index.get(pos, [])
        if oldest in keys:
            keys.remove(oldest)
        self.evicted.append(oldest)


def reference_save_plan(block_tables, seq_lens, block_size: int):
    """[(block_id, position_start, tokens)] in the order the reference's
    save_kv_layer saves them (kessie_kv_connector.py:459-483): every block of
    every sequence, sequence by sequence, ceil(seq_len / block_size) blocks
    each, the last one partial."""
    plan = []
    n_rows = len(block_tables)
    for si in range(min(len(seq_lens), n_rows)):
        seq_len = int(seq_lens[si])
        for b in range((seq_len + block_size - 1) // block_size):
            pos = b * block_size
            plan.append((int(block_tables[si][b]), pos, min(block_size, seq_len - pos)))
    return plan


def reference_query_text(token_ids, transformers_importable: bool = True) -> str:
    """The reference's semantic-search query (kessie_kv_connector.py:335-344):
    md5 over bytes() of the last 128 token ids when its transformers import
    succeeds, of the last 64 otherwise; bytes() raises ValueError for an id
    outside 0..255."""
    import hashlib

    tail = token_ids[-128:] if transformers_importable else token_ids[-64:]
    return f"tokens:{hashlib.md5(bytes(tail)).hexdigest()}"
