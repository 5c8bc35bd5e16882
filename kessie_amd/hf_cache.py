"""Tiered KV cache of the HF generation path on the MI355X (the KV parts of
the reference's KeSSieCache, kessie_exp3.py:341-533 and :590-625).

Same constructor, attributes and methods -- update, evict_if_needed,
recall_from_cpu, the HF cache accessors, reset / full_reset, get_stats --
and the same observable results (the K returned, the fog-weighted V
returned, what is evicted and recalled, the counters).  The storage is
re-designed for HBM:

  * each layer's K and V live in an arena [B, H, capacity, D] with a window
    offset; update writes the new tokens in place and returns views, instead
    of re-materialising the whole cache with torch.cat on every call;
  * the fog-weighted V is produced by one fused kernel (read V, weight,
    round, write) into a persistent per-layer buffer [B, H, >= window, D],
    instead of
    ``(v.float() * fog).to(dtype)`` -- three passes and two allocations over
    the whole cache per layer per step.  The returned view is overwritten by
    the next update of that layer (HF consumes it within the layer call);
  * evict_if_needed advances the window offset and copies the evicted tokens
    to pinned host memory on a copy stream (asynchronous); the reference
    trims with .contiguous() (a device copy of the window) and copies into
    pageable memory;
  * recall_from_cpu copies the chunk host-to-device into the space in front of
    the window (after its eviction copy has finished), instead of a
    torch.cat prepend of the whole window.
Arena capacity grows by doubling and the window is moved to the front only
when the tail is full, so the amortised cost per token is O(1).
Conversation-token / semantic-index bookkeeping of the reference class is
not part of this path.
"""
from __future__ import annotations

import logging
from typing import Any, List, Optional, Tuple

import torch

from . import ops

logger = logging.getLogger("KeSSie.HFCache")


class _Layer:
    __slots__ = ("k", "v", "vfog", "off", "n")

    def __init__(self):
        self.k = self.v = self.vfog = None
        self.off = 0
        self.n = 0

    def views(self):
        s = slice(self.off, self.off + self.n)
        return self.k[:, :, s], self.v[:, :, s]


class KeSSieCache:
    """Tiered KV cache: hot window in HBM, evicted (fogged) tokens in pinned
    host memory, recalled on demand."""

    def __init__(self, window_size=4096, index_granularity=128, fog_alpha=0.5, fog_start=0.5,
                 kv_cache_dtype=None, max_conversation_tokens=10_000_000):
        self.window_size = window_size
        self.fog_alpha = fog_alpha
        self.fog_start = fog_start
        self.index_granularity = index_granularity
        self.kv_cache_dtype = kv_cache_dtype
        self.max_conversation_tokens = max_conversation_tokens
        self._layers: List[_Layer] = []
        # (start_pos, end_pos, [(k_cpu, v_cpu) per layer]); tensors are pinned
        # and valid once the chunk's copy event has completed.
        self.cpu_kv_store: List[Tuple[int, int, List[Tuple[Any, Any]]]] = []
        self._store_events: List[Optional[torch.cuda.Event]] = []
        self.cpu_kv_bytes = 0
        self.window_start = 0
        self.seen_tokens = 0
        self._seen_tokens = 0
        self.total_evictions = 0
        self.total_recalls = 0
        self.has_previous_state = False
        self._copy_stream = None

    # -- HF cache interface ------------------------------------------------------------
    @property
    def key_cache(self):
        return [L.views()[0] if L.k is not None else torch.tensor([]) for L in self._layers]

    @property
    def value_cache(self):
        return [L.views()[1] if L.k is not None else torch.tensor([]) for L in self._layers]

    def __len__(self):
        return len(self._layers)

    def __getitem__(self, i):
        return self._layers[i].views()

    def get_seq_length(self, li=0):
        if li < len(self._layers) and self._layers[li].k is not None:
            return self._layers[li].n
        return 0

    def get_max_length(self):
        return self.window_size * 2

    def get_usable_length(self, n, li=0):
        return max(0, self.get_seq_length(li))

    def get_mask_sizes(self, cp, li):
        return self.get_seq_length(li) + cp.shape[0], 0

    def reset(self):
        self._layers.clear()
        self.cpu_kv_store.clear()
        self._store_events.clear()
        self.cpu_kv_bytes = 0
        self.window_start = 0
        self.seen_tokens = 0
        self._seen_tokens = 0
        self.has_previous_state = False

    def full_reset(self):
        self.reset()
        self.total_evictions = 0
        self.total_recalls = 0

    @staticmethod
    def _valid(t):
        return t is not None and isinstance(t, torch.Tensor) and t.numel() > 0

    def _cast_kv(self, t):
        if self.kv_cache_dtype is not None and t.dtype != self.kv_cache_dtype:
            return t.to(self.kv_cache_dtype)
        return t

    def _compute_fog_mask(self, seq_len, device, dtype):
        """(1,1,seq_len,1) fp32 fog weights, or None (kessie_exp3.py:415-425)."""
        if self.fog_alpha <= 0 or seq_len == 0:
            return None
        cc = max(1, int(seq_len * self.fog_start))
        if seq_len - cc <= 0:
            return None
        return ops.hf_fog_weights(seq_len, self.fog_alpha, self.fog_start, device=device).view(1, 1, seq_len, 1)

    # -- storage -----------------------------------------------------------------
    def _stream(self, device):
        if self._copy_stream is None or self._copy_stream.device != torch.device(device):
            self._copy_stream = torch.cuda.Stream(device=device)
        return self._copy_stream

    def _wait_evictions(self):
        """Order the compute stream after every pending eviction copy (they
        read arena regions that a move or a prepend may overwrite)."""
        cur = torch.cuda.current_stream()
        for ev in self._store_events:
            if ev is not None:
                cur.wait_event(ev)

    def _realloc(self, L: _Layer, cap: int, front: int):
        """New arena of `cap` tokens with the window moved to offset `front`."""
        self._wait_evictions()
        b, h, _, d = L.k.shape
        for name in ("k", "v"):
            old = getattr(L, name)
            new = torch.empty(b, h, cap, d, dtype=old.dtype, device=old.device)
            new[:, :, front:front + L.n].copy_(old[:, :, L.off:L.off + L.n])
            setattr(L, name, new)
        L.off = front

    def _reserve_tail(self, L: _Layer, t: int):
        cap = L.k.shape[2]
        if L.off + L.n + t <= cap:
            return
        need = L.n + t
        self._realloc(L, cap if need <= cap // 2 else max(2 * cap, need), 0)

    def _reserve_front(self, L: _Layer, c: int):
        if L.off >= c:
            return
        cap = L.k.shape[2]
        need = L.n + c
        self._realloc(L, cap if need <= cap // 2 else max(2 * cap, need), c)

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        """Append key/value_states [B, H, T, D]; return (K, fog-weighted V)
        over the whole window, as views."""
        key_states = self._cast_kv(key_states)
        value_states = self._cast_kv(value_states)
        while len(self._layers) <= layer_idx:
            self._layers.append(_Layer())
        L = self._layers[layer_idx]
        b, h, t, d = key_states.shape
        if L.k is None:
            cap = max(2 * self.window_size + 256, 2 * t)
            L.k = torch.empty(b, h, cap, d, dtype=key_states.dtype, device=key_states.device)
            L.v = torch.empty_like(L.k)
            L.off = L.n = 0
        self._reserve_tail(L, t)
        n_old, n = L.n, L.n + t
        cc = max(1, int(n * self.fog_start))
        fog_on = self.fog_alpha > 0 and n - cc > 0
        vf = None
        if fog_on:
            if L.vfog is None or L.vfog.shape[2] < n:
                L.vfog = torch.empty(b, h, max(n, 2 * self.window_size + 256), d, dtype=L.v.dtype,
                                     device=L.v.device)
            vf = L.vfog[:, :, :n]
        # One launch appends the new tokens and writes the fogged window.
        fused = ops.hf_append_fog(L.k, L.v, L.off, n_old, key_states, value_states, vf, self.fog_alpha,
                                  self.fog_start)
        if not fused:
            end = L.off + n_old
            L.k[:, :, end:end + t].copy_(key_states)
            L.v[:, :, end:end + t].copy_(value_states)
        L.n = n
        if layer_idx == 0:
            self.seen_tokens = self.window_start + L.n
            self._seen_tokens = self.seen_tokens
        k, v = L.views()
        if not fog_on:
            return k, v
        if not fused:
            ops.hf_fog_apply(v, self.fog_alpha, self.fog_start, out=vf)
        return k, vf

    def evict_if_needed(self):
        """Once the window exceeds 2 x window_size, move all but the newest
        window_size tokens of every layer to pinned host memory."""
        if not self._layers or self._layers[0].k is None:
            return
        cl = self._layers[0].n
        if cl <= self.window_size * 2:
            return
        ev = cl - self.window_size
        if ev <= 0:
            return
        device = self._layers[0].k.device
        stream = self._stream(device)
        stream.wait_stream(torch.cuda.current_stream(device))
        cpu_layers, chunk_bytes = [], 0
        with torch.cuda.stream(stream):
            for L in self._layers:
                if L.k is None:
                    cpu_layers.append((None, None))
                    continue
                k, v = L.views()
                kh = torch.empty(k[:, :, :ev].shape, dtype=k.dtype, pin_memory=True)
                vh = torch.empty_like(kh, pin_memory=True)
                kh.copy_(k[:, :, :ev], non_blocking=True)
                vh.copy_(v[:, :, :ev], non_blocking=True)
                L.k.record_stream(stream)
                L.v.record_stream(stream)
                chunk_bytes += 2 * kh.numel() * kh.element_size()
                cpu_layers.append((kh, vh))
                L.off += ev
                L.n -= ev
            event = torch.cuda.Event()
            event.record(stream)
        start = self.window_start
        self.cpu_kv_store.append((start, start + ev, cpu_layers))
        self._store_events.append(event)
        self.cpu_kv_bytes += chunk_bytes
        self.window_start += ev
        self.total_evictions += ev
        self.seen_tokens = self.window_start + self._layers[0].n
        self._seen_tokens = self.seen_tokens
        logger.info(f"KV evict: {ev} tokens -> CPU ({chunk_bytes / 1048576:.1f} MB), "
                    f"{len(self.cpu_kv_store)} chunks in RAM ({self.cpu_kv_bytes / 1048576:.1f} MB total)")

    def recall_from_cpu(self, position: int, device) -> bool:
        """Bring the stored chunk containing `position` back in front of the
        window (window_start becomes the chunk's start, as in the reference)."""
        target = None
        for idx, (start, end, layers) in enumerate(self.cpu_kv_store):
            if start <= position < end:
                target = idx
                break
        if target is None:
            return False
        start, end, cpu_layers = self.cpu_kv_store[target]
        # Wait for every pending eviction copy, not only this chunk's: the
        # prepend below writes the arena slots in front of the window, which
        # are the source of the most recent eviction's copy to host memory.
        self._wait_evictions()
        recalled = 0
        for i, L in enumerate(self._layers):
            if i >= len(cpu_layers) or cpu_layers[i][0] is None:
                continue
            kh, vh = cpu_layers[i]
            c = kh.shape[2]
            recalled += kh.numel() * kh.element_size() * 2
            if L.k is None:
                L.k = torch.empty(kh.shape[0], kh.shape[1], max(2 * self.window_size + 256, 2 * c), kh.shape[3],
                                  dtype=kh.dtype, device=device)
                L.v = torch.empty_like(L.k)
                L.off, L.n = c, 0
            self._reserve_front(L, c)
            L.k[:, :, L.off - c:L.off].copy_(kh, non_blocking=True)
            L.v[:, :, L.off - c:L.off].copy_(vh, non_blocking=True)
            L.off -= c
            L.n += c
        self.window_start = start
        self.seen_tokens = self.window_start + (self._layers[0].n if self._layers else 0)
        self._seen_tokens = self.seen_tokens
        self.total_recalls += 1
        del self.cpu_kv_store[target]
        del self._store_events[target]
        self.cpu_kv_bytes -= recalled // 2
        logger.info(f"KV recall: pos {start}-{end} ({end - start} tokens) -> GPU ({recalled / 1048576:.1f} MB), "
                    f"window now {self.get_seq_length()} tokens")
        return True

    def get_stats(self):
        kv_gpu_bytes, kv_dtype = 0, None
        for L in self._layers:
            if L.k is not None and L.n:
                kv_gpu_bytes += 2 * L.n * L.k.shape[0] * L.k.shape[1] * L.k.shape[3] * L.k.element_size()
                kv_dtype = kv_dtype or str(L.k.dtype)
        kv_seq = self.get_seq_length()
        fog_tokens = int(kv_seq * (1.0 - self.fog_start)) if kv_seq > 0 else 0
        return {
            "kv_seq_len": kv_seq,
            "kv_window_start": self.window_start,
            "kv_layers": len(self._layers),
            "kv_gpu_bytes": kv_gpu_bytes,
            "kv_gpu_mb": round(kv_gpu_bytes / 1048576, 2),
            "kv_cpu_mb": round(self.cpu_kv_bytes / 1048576, 2),
            "kv_cpu_chunks": len(self.cpu_kv_store),
            "kv_cpu_tokens": sum(end - start for start, end, _ in self.cpu_kv_store),
            "kv_dtype": kv_dtype,
            "fog_tokens": fog_tokens,
            "clear_tokens": kv_seq - fog_tokens,
            "window_capacity": self.window_size,
            "window_fill_pct": round(kv_seq / max(self.window_size, 1) * 100, 1),
            "total_evictions": self.total_evictions,
            "total_recalls": self.total_recalls,
        }
