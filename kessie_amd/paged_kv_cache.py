"""KeSSiePagedKVCache on the MI355X kernels (kessie_hip_kernels.py:484-570).

Same constructor, properties and methods as the reference class, same page
order semantics:
  * allocate_pages pops ids from the END of the host free list (LIFO), which
    starts as [0, 1, ..., num_pages-1];
  * evict_before(pos) invalidates valid pages with position < pos and appends
    every page that is invalid and not on the free list -- including pages
    allocated but never inserted -- in ascending id order;
  * get_layer_kv returns the valid pages of a layer in ascending physical id
    order, flattened to [tokens, H, D] K and V.
Underneath, evict_before is one kernel (threshold predicate + ordered
compaction of the freed ids) and one device-to-host copy, instead of the
reference's Triton launch followed by one ``.item()`` sync per page (65,536
syncs for a 65,536-page pool); insert_probe_kv is one insert kernel for all
pages instead of two slice copies and two scalar writes per page, and
get_layer_kv is one compaction plus one page-gather launch.
"""
from __future__ import annotations

import logging

import torch

from . import ops

logger = logging.getLogger("KeSSie.PagedKV")


class KeSSiePagedKVCache:
    """Paged KV cache [num_layers, num_pages, page_size, 2, num_heads, head_dim]."""

    def __init__(self, num_pages, page_size, num_layers, num_heads, head_dim, device, dtype=torch.float16):
        self.num_pages = num_pages
        self.page_size = page_size
        self.num_layers = num_layers
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.device = device
        self.dtype = dtype
        self.kv_data = torch.zeros(num_layers, num_pages, page_size, 2, num_heads, head_dim, device=device,
                                   dtype=dtype)
        self.page_positions = torch.zeros(num_pages, dtype=torch.int32, device=device)
        self.page_valid = torch.zeros(num_pages, dtype=torch.int8, device=device)
        # Pages not on the free list (device mirror, read by evict_before).
        self._allocated = torch.zeros(num_pages, dtype=torch.int8, device=device)
        self.free_pages = list(range(num_pages))
        self.total_evictions = 0
        self.total_insertions = 0
        logger.info(f"KeSSiePagedKVCache: {num_pages}p x {page_size}t, {num_layers}L x {num_heads}H x "
                    f"{head_dim}D, VRAM={self.vram_bytes / 1e9:.2f} GB")

    @property
    def vram_bytes(self):
        return self.kv_data.nelement() * self.kv_data.element_size()

    @property
    def active_pages(self):
        return self.num_pages - len(self.free_pages)

    @property
    def active_tokens(self):
        return self.active_pages * self.page_size

    def allocate_pages(self, n):
        """Pop n page ids from the end of the free list; None if too few."""
        if len(self.free_pages) < n:
            return None
        ids = [self.free_pages.pop() for _ in range(n)]
        t = torch.tensor(ids, dtype=torch.int32).to(self.device)
        if n:
            self._allocated.index_fill_(0, t.long(), 1)
        return t

    def evict_before(self, position):
        """Invalidate pages with position < ``position`` and return every
        invalid allocated page to the free list (ascending id order)."""
        freed, count = ops.page_evict_list(self.page_valid, self.page_positions, int(position),
                                           allocated=self._allocated)
        host = torch.cat([count, freed[: self.num_pages]]).cpu()  # one transfer, one sync
        n = int(host[0])
        ids = host[1:1 + n].tolist()
        self.free_pages.extend(ids)
        self.total_evictions += n
        return n

    def insert_probe_kv(self, layer_idx, keys, values, conv_position):
        """Write keys/values [T, H, D] into freshly allocated pages of one
        layer; page i gets position conv_position + i*page_size."""
        num_tokens = keys.shape[0]
        pages_needed = (num_tokens + self.page_size - 1) // self.page_size
        page_ids = self.allocate_pages(pages_needed)
        if page_ids is None:
            return False
        if num_tokens:
            ops.page_insert(self.kv_data[layer_idx], keys.to(self.dtype).contiguous(),
                            values.to(self.dtype).contiguous(), page_ids, self.page_valid, self.page_positions,
                            int(conv_position))
        self.total_insertions += num_tokens
        return True

    def get_layer_kv(self, layer_idx):
        """(K, V), each [valid_pages * page_size, H, D], valid pages in
        ascending physical id order."""
        idx, count = ops.page_valid_list(self.page_valid)
        n = int(count.item())
        if n == 0:
            empty = torch.empty(0, self.num_heads, self.head_dim, device=self.device, dtype=self.dtype)
            return empty, empty.clone()
        pages = ops.page_gather(self.kv_data[layer_idx], idx, n=n)
        kv = pages.reshape(-1, 2, self.num_heads, self.head_dim)
        return kv[:, 0], kv[:, 1]

    def get_stats(self):
        return {"total_pages": self.num_pages, "active_pages": self.active_pages,
                "free_pages": len(self.free_pages), "active_tokens": self.active_tokens,
                "vram_gb": self.vram_bytes / 1e9, "total_evictions": self.total_evictions,
                "total_insertions": self.total_insertions}
