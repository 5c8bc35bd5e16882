"""Oracle for the HF tiered KV cache (test infrastructure only): the KV parts
of KeSSieCache (kessie_exp3.py:341-533) restated as the reference writes them
-- torch.cat appends, fog-weighted V returned by update, eviction of the
oldest tokens to CPU once the window doubles, recall that prepends a chunk.
Tensors are [B, H, seq, D]; runs wherever its inputs live."""
from __future__ import annotations

import torch


def hf_fog_mask(seq_len: int, fog_alpha: float, fog_start: float, device=None, dtype=torch.float32):
    """_compute_fog_mask (kessie_exp3.py:415-425), op for op."""
    if fog_alpha <= 0 or seq_len == 0:
        return None
    cc = max(1, int(seq_len * fog_start))
    fc = seq_len - cc
    if fc <= 0:
        return None
    pos = torch.arange(fc, dtype=dtype, device=device)
    fw = (pos / max(fc - 1, 1)).pow(fog_alpha).clamp(min=0.01)
    cw = torch.ones(cc, dtype=dtype, device=device)
    return torch.cat([fw, cw]).view(1, 1, seq_len, 1)


def hf_fogged_v(v: torch.Tensor, fog_alpha: float, fog_start: float) -> torch.Tensor:
    """The V that update returns (kessie_exp3.py:443-445)."""
    fog = hf_fog_mask(v.shape[-2], fog_alpha, fog_start, v.device, torch.float32)
    return v if fog is None else (v.float() * fog).to(v.dtype)


class HFCacheModel:
    """KeSSieCache.update / evict_if_needed / recall_from_cpu bookkeeping."""

    def __init__(self, window_size=4096, fog_alpha=0.5, fog_start=0.5):
        self.window_size, self.fog_alpha, self.fog_start = window_size, fog_alpha, fog_start
        self.key_cache, self.value_cache = [], []
        self.cpu_kv_store = []
        self.cpu_kv_bytes = 0
        self.window_start = self.seen_tokens = 0
        self.total_evictions = self.total_recalls = 0

    def update(self, k, v, layer_idx):
        while len(self.key_cache) <= layer_idx:
            self.key_cache.append(None)
            self.value_cache.append(None)
        if self.key_cache[layer_idx] is None:
            self.key_cache[layer_idx], self.value_cache[layer_idx] = k, v
        else:
            self.key_cache[layer_idx] = torch.cat([self.key_cache[layer_idx], k], dim=-2)
            self.value_cache[layer_idx] = torch.cat([self.value_cache[layer_idx], v], dim=-2)
        if layer_idx == 0:
            self.seen_tokens = self.window_start + self.key_cache[0].shape[-2]
        return self.key_cache[layer_idx], hf_fogged_v(self.value_cache[layer_idx], self.fog_alpha, self.fog_start)

    def evict_if_needed(self):
        if not self.key_cache or self.key_cache[0] is None:
            return
        cl = self.key_cache[0].shape[-2]
        if cl <= self.window_size * 2:
            return
        ev = cl - self.window_size
        layers, nbytes = [], 0
        for i in range(len(self.key_cache)):
            k, v = self.key_cache[i], self.value_cache[i]
            layers.append((k[:, :, :ev].clone(), v[:, :, :ev].clone()))
            nbytes += 2 * k[:, :, :ev].numel() * k.element_size()
            self.key_cache[i], self.value_cache[i] = k[:, :, ev:].clone(), v[:, :, ev:].clone()
        self.cpu_kv_store.append((self.window_start, self.window_start + ev, layers))
        self.cpu_kv_bytes += nbytes
        self.window_start += ev
        self.total_evictions += ev
        self.seen_tokens = self.window_start + self.key_cache[0].shape[-2]

    def recall_from_cpu(self, position):
        for idx, (start, end, layers) in enumerate(self.cpu_kv_store):
            if start <= position < end:
                break
        else:
            return False
        recalled = 0
        for i in range(len(self.key_cache)):
            k, v = layers[i]
            recalled += k.numel() * k.element_size() * 2
            self.key_cache[i] = torch.cat([k, self.key_cache[i]], dim=-2)
            self.value_cache[i] = torch.cat([v, self.value_cache[i]], dim=-2)
        self.window_start = start
        self.seen_tokens = self.window_start + self.key_cache[0].shape[-2]
        self.total_recalls += 1
        del self.cpu_kv_store[idx]
        self.cpu_kv_bytes -= recalled // 2
        return True
