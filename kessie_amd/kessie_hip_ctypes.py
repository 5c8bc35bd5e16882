"""KeSSie HIP kernels -- ctypes interface (MI355X build).

Drop-in for the reference's ``kessie_hip_ctypes.KeSSieKernels``
(kessie_hip_ctypes.py:39-346): same class name, method names, argument
meaning and defaults, and the same stream convention (``stream=None`` runs on
the current stream and synchronises before returning; a stream or a stream
name from ``create_stream`` runs asynchronously).  Underneath is
libkessie_mi355x.so (include/kessie_mi355x.h) instead of libkessie_hip.so.

Differences a caller can observe:
  * ``rope_remap`` honours the tensor's dtype (fp32 / bf16 / fp16); the
    reference launcher reads any dtype as fp16 (kessie_kernels_v2.hip:671).
  * ``fused_fog_attention`` applies the weights to every query row (the
    reference kernel's rows of warps 1-3 use the wrong Q row,
    kessie_kernels_v2.hip:592); results follow kessie_hip_kernels.py:592-593.
  * failures raise ``KeSSieError`` instead of printing to stderr.
Added: the paged entry points (fog decode / prefill, paged RoPE remap, page
insert / select-evict / compact / gather / valid list / evict list).
"""
from __future__ import annotations

import ctypes
import logging
import math
from typing import Optional

import torch

from . import _lib, ops

logger = logging.getLogger("KeSSie.HIP")


class KeSSieKernels:
    """Python interface to the MI355X KeSSie kernels via ctypes."""

    def __init__(self, lib_path: str = None):
        # Raises FileNotFoundError when the library is absent (no fallback).
        self.lib = _lib.load(lib_path)
        self.lib_path = _lib.lib_path()
        self._streams = {}
        logger.info("KeSSie MI355X kernels loaded from %s", self.lib_path)

    # ------------------------------------------------------------------
    # Streams (kessie_hip_ctypes.py:120-146)
    # ------------------------------------------------------------------
    def create_stream(self, name: str = "probe") -> torch.cuda.Stream:
        s = torch.cuda.Stream()
        self._streams[name] = s
        return s

    def sync_stream(self, name: str = "probe"):
        if name in self._streams:
            self._streams[name].synchronize()

    def _resolve_stream(self, stream):
        if isinstance(stream, str):
            stream = self._streams.get(stream)
        return stream

    def _get_stream_ptr(self, stream=None) -> ctypes.c_void_p:
        stream = self._resolve_stream(stream)
        if isinstance(stream, torch.cuda.Stream):
            return ctypes.c_void_p(stream.cuda_stream)
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    @staticmethod
    def _finish(stream):
        if stream is None:
            torch.cuda.synchronize()

    @staticmethod
    def _ptr(tensor: torch.Tensor) -> ctypes.c_void_p:
        assert tensor.is_cuda, f"Tensor must be on GPU, got {tensor.device}"
        assert tensor.is_contiguous(), "Tensor must be contiguous"
        return ctypes.c_void_p(tensor.data_ptr())

    # ------------------------------------------------------------------
    # Dense attention (kessie_hip_ctypes.py:163-242)
    # ------------------------------------------------------------------
    def windowed_attention(self, Q, K, V, window_size: int = 0, causal: bool = True,
                           sm_scale: Optional[float] = None, stream=None) -> torch.Tensor:
        """Q, K, V: [B, H, N, D] fp16; window_size 0 = full attention."""
        assert Q.dtype == torch.float16
        assert Q.shape == K.shape == V.shape
        B, H, N, D = Q.shape
        assert D in (64, 128)
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        O = torch.empty_like(Q)
        Q, K, V = Q.contiguous(), K.contiguous(), V.contiguous()
        _lib.call_legacy("launch_kessie_windowed_attn", self._ptr(Q), self._ptr(K), self._ptr(V),
                         self._ptr(O), ctypes.c_float(sm_scale), B, H, N, D, window_size,
                         1 if causal else 0, self._get_stream_ptr(stream))
        self._finish(stream)
        return O

    def fused_fog_attention(self, Q, K, V, fog_weights, window_size: int = 0, causal: bool = True,
                            sm_scale: Optional[float] = None, stream=None) -> torch.Tensor:
        """Attention with V rows scaled by fog_weights [N] fp32 (1.0 = clear)."""
        assert Q.dtype == torch.float16
        assert fog_weights.dtype == torch.float32
        assert Q.shape == K.shape == V.shape
        B, H, N, D = Q.shape
        assert fog_weights.shape[0] == N
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        O = torch.empty_like(Q)
        Q, K, V = Q.contiguous(), K.contiguous(), V.contiguous()
        fog_weights = fog_weights.contiguous()
        _lib.call_legacy("launch_kessie_fused_fog_attn", self._ptr(Q), self._ptr(K), self._ptr(V),
                         self._ptr(O), self._ptr(fog_weights), ctypes.c_float(sm_scale), B, H, N, D,
                         window_size, 1 if causal else 0, self._get_stream_ptr(stream))
        self._finish(stream)
        return O

    # ------------------------------------------------------------------
    # RoPE remap (kessie_hip_ctypes.py:248-286)
    # ------------------------------------------------------------------
    def rope_remap(self, k_data: torch.Tensor, orig_positions: torch.Tensor,
                   target_positions: torch.Tensor, rope_theta: float = 10000.0, stream=None):
        """Re-rotate K [tokens, heads, dim] IN PLACE from original to target positions."""
        assert k_data.is_cuda and k_data.is_contiguous()
        num_tokens, num_heads, head_dim = k_data.shape
        assert head_dim % 2 == 0
        orig_positions = orig_positions.contiguous().to(torch.int32)
        target_positions = target_positions.contiguous().to(torch.int32)
        ops.rope_remap_paged(k_data, orig_positions, target_positions, rope_theta,
                             stream=self._resolve_stream(stream))
        self._finish(stream)

    # ------------------------------------------------------------------
    # Page management (kessie_hip_ctypes.py:292-346)
    # ------------------------------------------------------------------
    def page_evict(self, page_valid: torch.Tensor, page_positions: torch.Tensor,
                   evict_before_pos: int, stream=None) -> int:
        """Evict (fog) all KV pages with position below threshold; returns the count."""
        assert page_valid.dtype == torch.int8
        assert page_positions.dtype == torch.int32
        num_pages = page_valid.shape[0]
        evict_count = torch.zeros(1, dtype=torch.int32, device=page_valid.device)
        _lib.call_legacy("launch_kessie_page_evict", self._ptr(page_valid), self._ptr(page_positions),
                         self._ptr(evict_count), evict_before_pos, num_pages, self._get_stream_ptr(stream))
        self._finish(stream)
        return evict_count.item()

    def page_insert(self, kv_cache, new_keys, new_values, target_page_ids, page_valid, page_positions,
                    insert_conv_position: int, stream=None):
        """Insert probe KV [T, H, D] into allocated pages of kv_cache [pages, P, 2, H, D]."""
        assert kv_cache.dtype == new_keys.dtype == new_values.dtype
        ops.page_insert(kv_cache, new_keys, new_values, target_page_ids.to(torch.int32), page_valid,
                        page_positions, insert_conv_position, stream=self._resolve_stream(stream))
        self._finish(stream)

    # ------------------------------------------------------------------
    # Paged entry points (no reference counterpart)
    # ------------------------------------------------------------------
    def fog_decode_paged(self, q, pool, page_table, ctx_lens, max_ctx, fog_weights=None, fog_bias=None,
                         window_size: int = 0, sm_scale=None, layout: str = "native", stream=None):
        out = ops.fog_decode(q, pool, page_table, ctx_lens, max_ctx, fog_vscale=fog_weights,
                             fog_bias=fog_bias, window=window_size, sm_scale=sm_scale, layout=layout,
                             stream=self._resolve_stream(stream))
        self._finish(stream)
        return out

    def fog_prefill_paged(self, q, pool, page_table, ctx_lens, max_ctx, fog_weights=None, fog_bias=None,
                          window_size: int = 0, causal: bool = True, sm_scale=None, layout: str = "native",
                          stream=None):
        out = ops.fog_prefill(q, pool, page_table, ctx_lens, max_ctx, fog_vscale=fog_weights,
                              fog_bias=fog_bias, window=window_size, causal=causal, sm_scale=sm_scale,
                              layout=layout, stream=self._resolve_stream(stream))
        self._finish(stream)
        return out

    def rope_remap_paged(self, pool, page_list, orig_positions, target_positions, rope_theta: float = 10000.0,
                         layout: str = "native", stream=None):
        ops.rope_remap_paged(pool, orig_positions.to(torch.int32), target_positions.to(torch.int32),
                             rope_theta, page_list=page_list.to(torch.int32), layout=layout,
                             stream=self._resolve_stream(stream))
        self._finish(stream)

    def page_select_evict(self, scores, page_valid, k_evict: int = -1, evict_fraction: float = 0.25,
                          stream=None):
        lst, cnt = ops.page_select_evict(scores, page_valid, k_evict, evict_fraction,
                                         stream=self._resolve_stream(stream))
        self._finish(stream)
        return lst, cnt

    def page_compact(self, tables, lens, page_valid, stream=None):
        res = ops.page_compact(tables, lens, page_valid, stream=self._resolve_stream(stream))
        self._finish(stream)
        return res

    def page_gather(self, pool, idx, count=None, n=None, stream=None):
        out = ops.page_gather(pool, idx, count, n=n, stream=self._resolve_stream(stream))
        self._finish(stream)
        return out

    def page_valid_list(self, page_valid, stream=None):
        res = ops.page_valid_list(page_valid, stream=self._resolve_stream(stream))
        self._finish(stream)
        return res

    def page_evict_list(self, page_valid, page_positions, evict_before_pos: int, allocated=None, stream=None):
        res = ops.page_evict_list(page_valid, page_positions, evict_before_pos, allocated,
                                  stream=self._resolve_stream(stream))
        self._finish(stream)
        return res
