"""Tensor-level API over libkessie_mi355x.so (device tensors in, device tensors out).

Every function here launches HIP kernels through the C ABI on the current
torch stream (or the ``stream`` given) and returns without synchronising.
There is no CPU or torch fallback: a missing library or a tensor on the
wrong device raises.

Pool layouts (the innermost head_dim axis must be contiguous):
  "native"    [pages, P, 2, Hkv, D]   (kessie_kernels_v2.hip:415, kessie_hip_kernels.py:496-498)
  "kv_first"  [2, blocks, P, Hkv, D]  (vLLM FLASH_ATTN; kessie_kv_connector.py:309)
  "block_kv"  [blocks, 2, P, Hkv, D]  (vLLM TRITON_ATTN)
"""
from __future__ import annotations

import ctypes as C
import math
import threading
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib

_DTYPES = {
    torch.float32: _lib.DTYPE_F32,
    torch.bfloat16: _lib.DTYPE_BF16,
    torch.float16: _lib.DTYPE_F16,
}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, bfloat16 or float16") from None


def _ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError(f"tensor must be on the GPU, got {t.device}")
    return C.c_void_p(t.data_ptr())


def _contig(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def _stream_ptr(stream, device) -> C.c_void_p:
    if isinstance(stream, int):
        return C.c_void_p(stream)
    if stream is None:
        stream = torch.cuda.current_stream(device)
    if isinstance(stream, torch.cuda.Stream):
        return C.c_void_p(stream.cuda_stream)
    raise TypeError(f"stream must be a torch.cuda.Stream, an int handle or None, got {type(stream)}")


# ---------------------------------------------------------------------------
# Workspace cache (one growable byte buffer per device and purpose)
# ---------------------------------------------------------------------------
_ws_lock = threading.Lock()
_ws: dict = {}
# Buffers a larger request superseded.  They are never freed: a HIP graph
# captured while one of them was current still writes to its address on every
# replay, so handing that memory back to the caching allocator would let the
# replay overwrite whatever tensor is allocated there next.  Growth at least
# doubles the size, so a device/tag pair retires O(log(max bytes)) buffers.
_ws_retired: list = []


def workspace(nbytes: int, device, tag: str = "attn", init=None) -> Optional[torch.Tensor]:
    """A cached uint8 device buffer of at least ``nbytes`` (None when 0).

    Buffers are reused across calls on the same device and tag; callers on
    different streams that overlap must pass their own buffers instead.  A
    buffer outgrown by a larger request is kept alive, not freed (graphs
    captured earlier may still address it).
    """
    if nbytes <= 0:
        return None
    dev = torch.device(device)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), tag)
    with _ws_lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 1 << 16)
            if buf is not None:
                _ws_retired.append(buf)
                size = max(size, 2 * buf.numel())
            buf = torch.empty(size, dtype=torch.uint8, device=dev)
            if init is not None:
                init(buf)
            _ws[key] = buf
        return buf


# ---------------------------------------------------------------------------
# Pool descriptions
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class PoolView:
    base: torch.Tensor          # the pool tensor (K at kv index 0 is the base pointer)
    num_pages: int
    page_size: int
    num_kv_heads: int
    head_dim: int
    page_stride: int
    tok_stride: int
    kv_stride: int
    head_stride: int

    @property
    def k_ptr(self) -> int:
        return self.base.data_ptr()


def pool_view(pool: torch.Tensor, layout: str = "native") -> PoolView:
    if pool.dim() != 5:
        raise ValueError(f"pool must be 5-D, got shape {tuple(pool.shape)}")
    s = pool.stride()
    if s[4] != 1:
        raise ValueError("pool head_dim axis must be contiguous")
    if layout == "native":
        n, p, two, h, d = pool.shape
        ps, ts, kvs, hs = s[0], s[1], s[2], s[3]
    elif layout == "kv_first":
        two, n, p, h, d = pool.shape
        kvs, ps, ts, hs = s[0], s[1], s[2], s[3]
    elif layout == "block_kv":
        n, two, p, h, d = pool.shape
        ps, kvs, ts, hs = s[0], s[1], s[2], s[3]
    else:
        raise ValueError(f"unknown pool layout {layout!r}")
    if two != 2:
        raise ValueError(f"pool K/V axis must have size 2, got {two}")
    # Storage-offset-aware base: element [0,...] of K.
    return PoolView(pool, n, p, h, d, ps, ts, kvs, hs)


# ---------------------------------------------------------------------------
# Fog attention
# ---------------------------------------------------------------------------
def _fog_arg(t: Optional[torch.Tensor], batch: int, name: str, max_ctx: int = 0):
    if t is None:
        return None, 0
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on the GPU")
    if t.shape[-1] < max_ctx:
        raise ValueError(f"{name} covers {t.shape[-1]} positions, fewer than max_ctx={max_ctx}")
    if t.dim() == 1:
        return _contig(t, name), 0
    if t.dim() == 2 and t.shape[0] == batch:
        if t.stride(1) != 1:
            raise ValueError(f"{name} rows must be contiguous")
        return t, t.stride(0)
    raise ValueError(f"{name} must be [N] or [B, N], got {tuple(t.shape)}")


def fog_decode(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor, ctx_lens: torch.Tensor,
               max_ctx: int, fog_vscale: Optional[torch.Tensor] = None,
               fog_bias: Optional[torch.Tensor] = None, window: int = 0,
               sm_scale: Optional[float] = None, layout: str = "native",
               out: Optional[torch.Tensor] = None, ws: Optional[torch.Tensor] = None,
               stream=None) -> torch.Tensor:
    """Fog decode: q [B, Hq, D] -> out [B, Hq, D] (q's dtype) over a paged pool.

    page_table int32 [B, W]; ctx_lens int32 [B] on the device; ``max_ctx`` is
    a host-side upper bound of ctx_lens (it sizes the split-K grid).
    """
    pv = pool_view(pool, layout)
    q = _contig(q, "q")
    b, hq, d = q.shape
    if d != pv.head_dim or q.dtype != pool.dtype:
        raise ValueError("q and pool disagree on head_dim or dtype")
    if page_table.dtype != torch.int32 or ctx_lens.dtype != torch.int32:
        raise TypeError("page_table and ctx_lens must be int32")
    if page_table.dim() != 2 or page_table.shape[0] != b or page_table.stride(1) != 1:
        raise ValueError("page_table must be [B, W] with contiguous rows")
    if max_ctx > page_table.shape[1] * pv.page_size:
        raise ValueError(f"max_ctx={max_ctx} exceeds the page table's {page_table.shape[1]} pages")
    if out is None:
        out = torch.empty_like(q)
    out = _contig(out, "out")
    dt = dtype_code(q.dtype)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    vs, vs_bs = _fog_arg(fog_vscale, b, "fog_vscale", max_ctx)
    bi, bi_bs = _fog_arg(fog_bias, b, "fog_bias", max_ctx)
    lib = _lib.load()
    need = lib.kessie_fog_decode_workspace_bytes(b, hq, pv.num_kv_heads, d, max_ctx, pv.page_size, dt)
    if ws is None:
        ws = workspace(need, q.device, "attn")
    wsz = 0 if ws is None else ws.numel() * ws.element_size()
    _lib.check("kessie_fog_decode_paged", lib.kessie_fog_decode_paged(
        _ptr(q), C.c_void_p(pv.k_ptr), pv.num_pages, pv.page_stride, pv.tok_stride, pv.kv_stride,
        pv.head_stride, _ptr(page_table), page_table.stride(0), _ptr(ctx_lens), _ptr(vs), vs_bs,
        _ptr(bi), bi_bs, _ptr(out), b, hq, pv.num_kv_heads, d, pv.page_size, int(max_ctx), int(window),
        float(sm_scale), dt, _ptr(ws), wsz, _stream_ptr(stream, q.device)))
    return out


def decode_num_splits(batch: int, num_kv_heads: int, max_ctx: int, page_size: int) -> int:
    return _lib.load().kessie_fog_decode_num_splits(batch, num_kv_heads, max_ctx, page_size)


def fog_decode_partials(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor, ctx_lens: torch.Tensor,
                        max_ctx: int, ws: torch.Tensor, fog_vscale: Optional[torch.Tensor] = None,
                        fog_bias: Optional[torch.Tensor] = None, window: int = 0,
                        sm_scale: Optional[float] = None, layout: str = "native", stream=None) -> torch.Tensor:
    """The streaming half of fog_decode: per-split (m, l, o) partials into ``ws``
    (layout in include/kessie_mi355x.h).  Returns ws."""
    pv = pool_view(pool, layout)
    q = _contig(q, "q")
    b, hq, d = q.shape
    if d != pv.head_dim or q.dtype != pool.dtype:
        raise ValueError("q and pool disagree on head_dim or dtype")
    if page_table.dtype != torch.int32 or ctx_lens.dtype != torch.int32:
        raise TypeError("page_table and ctx_lens must be int32")
    if page_table.dim() != 2 or page_table.shape[0] != b or page_table.stride(1) != 1:
        raise ValueError("page_table must be [B, W] with contiguous rows")
    if max_ctx > page_table.shape[1] * pv.page_size:
        raise ValueError(f"max_ctx={max_ctx} exceeds the page table's {page_table.shape[1]} pages")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    vs, vs_bs = _fog_arg(fog_vscale, b, "fog_vscale", max_ctx)
    bi, bi_bs = _fog_arg(fog_bias, b, "fog_bias", max_ctx)
    lib = _lib.load()
    _lib.check("kessie_fog_decode_partials", lib.kessie_fog_decode_partials(
        _ptr(q), C.c_void_p(pv.k_ptr), pv.num_pages, pv.page_stride, pv.tok_stride, pv.kv_stride,
        pv.head_stride, _ptr(page_table), page_table.stride(0), _ptr(ctx_lens), _ptr(vs), vs_bs,
        _ptr(bi), bi_bs, b, hq, pv.num_kv_heads, d, pv.page_size, int(max_ctx), int(window),
        float(sm_scale), dtype_code(q.dtype), _ptr(ws), ws.numel() * ws.element_size(),
        _stream_ptr(stream, q.device)))
    return ws


def fog_decode_combine(ws: torch.Tensor, out: torch.Tensor, num_kv_heads: int, max_ctx: int, page_size: int,
                       stream=None) -> torch.Tensor:
    """Merge the partials of fog_decode_partials into out [B, Hq, D]."""
    out = _contig(out, "out")
    b, hq, d = out.shape
    lib = _lib.load()
    _lib.check("kessie_fog_decode_combine", lib.kessie_fog_decode_combine(
        _ptr(ws), ws.numel() * ws.element_size(), _ptr(out), b, hq, num_kv_heads, d, int(max_ctx),
        int(page_size), dtype_code(out.dtype), _stream_ptr(stream, out.device)))
    return out


def fog_prefill(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor, ctx_lens: torch.Tensor,
                max_ctx: int, fog_vscale: Optional[torch.Tensor] = None,
                fog_bias: Optional[torch.Tensor] = None, window: int = 0, causal: bool = True,
                sm_scale: Optional[float] = None, layout: str = "native",
                out: Optional[torch.Tensor] = None, ws: Optional[torch.Tensor] = None,
                stream=None) -> torch.Tensor:
    """Chunked prefill: q [B, C, Hq, D]; query i of sequence b sits at ctx_lens[b]-C+i.

    ws: workspace for split partials (a cached one when None); the MFMA kernel
    uses it only when the chunk is too small to fill the device."""
    pv = pool_view(pool, layout)
    q = _contig(q, "q")
    b, c, hq, d = q.shape
    if d != pv.head_dim or q.dtype != pool.dtype:
        raise ValueError("q and pool disagree on head_dim or dtype")
    if page_table.dtype != torch.int32 or ctx_lens.dtype != torch.int32:
        raise TypeError("page_table and ctx_lens must be int32")
    if page_table.dim() != 2 or page_table.shape[0] != b or page_table.stride(1) != 1:
        raise ValueError("page_table must be [B, W] with contiguous rows")
    if max_ctx > page_table.shape[1] * pv.page_size:
        raise ValueError(f"max_ctx={max_ctx} exceeds the page table's {page_table.shape[1]} pages")
    if out is None:
        out = torch.empty_like(q)
    out = _contig(out, "out")
    dt = dtype_code(q.dtype)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    vs, vs_bs = _fog_arg(fog_vscale, b, "fog_vscale", max_ctx)
    bi, bi_bs = _fog_arg(fog_bias, b, "fog_bias", max_ctx)
    lib = _lib.load()
    need = lib.kessie_fog_prefill_workspace_bytes(b, c, hq, pv.num_kv_heads, d, max_ctx, pv.page_size, dt)
    if ws is None:
        ws = workspace(need, q.device, "attn")
    wsz = 0 if ws is None else ws.numel() * ws.element_size()
    _lib.check("kessie_fog_prefill_paged", lib.kessie_fog_prefill_paged(
        _ptr(q), C.c_void_p(pv.k_ptr), pv.num_pages, pv.page_stride, pv.tok_stride, pv.kv_stride,
        pv.head_stride, _ptr(page_table), page_table.stride(0), _ptr(ctx_lens), _ptr(vs), vs_bs,
        _ptr(bi), bi_bs, _ptr(out), b, c, hq, pv.num_kv_heads, d, pv.page_size, int(max_ctx),
        int(window), float(sm_scale), 1 if causal else 0, dt, _ptr(ws), wsz,
        _stream_ptr(stream, q.device)))
    return out


def fog_prefill_varlen(q: torch.Tensor, query_start_loc: torch.Tensor, max_query_len: int, pool: torch.Tensor,
                       page_table: torch.Tensor, ctx_lens: torch.Tensor, max_ctx: int,
                       fog_vscale: Optional[torch.Tensor] = None, fog_bias: Optional[torch.Tensor] = None,
                       window: int = 0, causal: bool = True, sm_scale: Optional[float] = None,
                       layout: str = "native", out: Optional[torch.Tensor] = None,
                       ws: Optional[torch.Tensor] = None, stream=None) -> bool:
    """Chunked prefill of B sequences with different chunk lengths in one
    launch: q/out [T, Hq, D] packed, sequence b's queries at rows
    query_start_loc[b] - query_start_loc[0] .. (int32 [B+1] on the device, e.g.
    a slice of vLLM's query_start_loc), query i of it at ctx_lens[b] - C_b + i.
    Returns False, having launched nothing, for shapes the MFMA kernels do not
    take (the caller then runs fog_prefill per sequence).  ws: split-K
    workspace (a cached one when None), used when the chunks are too few to
    fill the device."""
    pv = pool_view(pool, layout)
    q = _contig(q, "q")
    t, hq, d = q.shape
    b = ctx_lens.numel()
    if d != pv.head_dim or q.dtype != pool.dtype:
        raise ValueError("q and pool disagree on head_dim or dtype")
    if page_table.dtype != torch.int32 or ctx_lens.dtype != torch.int32 or query_start_loc.dtype != torch.int32:
        raise TypeError("page_table, ctx_lens and query_start_loc must be int32")
    if query_start_loc.numel() != b + 1 or query_start_loc.stride(0) != 1:
        raise ValueError("query_start_loc must hold B+1 contiguous entries")
    if page_table.dim() != 2 or page_table.shape[0] != b or page_table.stride(1) != 1:
        raise ValueError("page_table must be [B, W] with contiguous rows")
    if max_ctx > page_table.shape[1] * pv.page_size:
        raise ValueError(f"max_ctx={max_ctx} exceeds the page table's {page_table.shape[1]} pages")
    if out is None:
        out = torch.empty_like(q)
    if out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [T, Hq, D] tensor of q's dtype")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    vs, vs_bs = _fog_arg(fog_vscale, b, "fog_vscale", max_ctx)
    bi, bi_bs = _fog_arg(fog_bias, b, "fog_bias", max_ctx)
    lib = _lib.load()
    dt = dtype_code(q.dtype)
    if ws is None:
        need = lib.kessie_fog_prefill_workspace_bytes(b, int(max_query_len), hq, pv.num_kv_heads, d, max_ctx,
                                                      pv.page_size, dt)
        ws = workspace(need, q.device, "attn")
    wsz = 0 if ws is None else ws.numel() * ws.element_size()
    st = lib.kessie_fog_prefill_varlen(
        _ptr(q), _ptr(query_start_loc), int(max_query_len), C.c_void_p(pv.k_ptr), pv.num_pages, pv.page_stride,
        pv.tok_stride, pv.kv_stride, pv.head_stride, _ptr(page_table), page_table.stride(0), _ptr(ctx_lens),
        _ptr(vs), vs_bs, _ptr(bi), bi_bs, _ptr(out), b, hq, pv.num_kv_heads, d, pv.page_size, int(max_ctx),
        int(window), float(sm_scale), 1 if causal else 0, dt, _ptr(ws), wsz, _stream_ptr(stream, q.device))
    if st == _lib.ERR_UNSUPPORTED:
        return False
    _lib.check("kessie_fog_prefill_varlen", st)
    return True


# ---------------------------------------------------------------------------
# RoPE remap
# ---------------------------------------------------------------------------
_inv_cache: dict = {}


def inv_freq_table(head_dim: int, rope_theta: float, device) -> torch.Tensor:
    """fp32 [D/2] device table, computed on the host with the exact torch
    expression of kessie_hip_kernels.py:600 (1/(theta ** (arange(half)/half)))
    and cached per (D, theta, device)."""
    dev = torch.device(device)
    key = (head_dim, float(rope_theta), dev.type, dev.index)
    t = _inv_cache.get(key)
    if t is None:
        half = head_dim // 2
        host = 1.0 / (rope_theta ** (torch.arange(half, dtype=torch.float32) / half))
        t = host.to(dev)
        _inv_cache[key] = t
    return t


def rope_remap_paged(pool: torch.Tensor, orig_pos: torch.Tensor, tgt_pos: torch.Tensor,
                     rope_theta: float, page_list: Optional[torch.Tensor] = None,
                     layout: str = "native", stream=None) -> None:
    """In-place remap of K for T tokens: token t in page page_list[t//P], slot t%P.

    With page_list None, ``pool`` is a dense K tensor [T, H, D] instead.
    """
    if orig_pos.dtype != torch.int32 or tgt_pos.dtype != torch.int32:
        raise TypeError("positions must be int32")
    t = orig_pos.numel()
    if tgt_pos.numel() != t:
        raise ValueError("orig_pos and tgt_pos differ in length")
    if page_list is None:
        k = _contig(pool, "k")
        tt, h, d = k.shape
        if tt != t:
            raise ValueError("k and positions disagree on token count")
        ptr, ps, ts, hs, n_pages, p_size = C.c_void_p(k.data_ptr()), 0, h * d, d, 0, 0
        dt = dtype_code(k.dtype)
        device = k.device
    else:
        pv = pool_view(pool, layout)
        if page_list.dtype != torch.int32:
            raise TypeError("page_list must be int32")
        if page_list.numel() * pv.page_size < t:
            raise ValueError("page_list too short for the token count")
        ptr, ps, ts, hs = C.c_void_p(pv.k_ptr), pv.page_stride, pv.tok_stride, pv.head_stride
        n_pages, p_size, h, d = pv.num_pages, pv.page_size, pv.num_kv_heads, pv.head_dim
        dt = dtype_code(pool.dtype)
        device = pool.device
    inv = inv_freq_table(d, rope_theta, device)
    lib = _lib.load()
    _lib.check("kessie_rope_remap_paged", lib.kessie_rope_remap_paged(
        ptr, ps, ts, hs, _ptr(page_list), n_pages, _ptr(_contig(orig_pos, "orig_pos")),
        _ptr(_contig(tgt_pos, "tgt_pos")), _ptr(inv), t, h, d, p_size, dt, _stream_ptr(stream, device)))


# ---------------------------------------------------------------------------
# Page management
# ---------------------------------------------------------------------------
def _init_page_workspace(buf: torch.Tensor) -> None:
    _lib.check("kessie_page_workspace_init", _lib.load().kessie_page_workspace_init(
        _ptr(buf), buf.numel(), _stream_ptr(None, buf.device)))


def page_workspace(num_pages: int, device) -> Optional[torch.Tensor]:
    """The cached page-management workspace, prepared by
    kessie_page_workspace_init when it is (re)allocated."""
    return workspace(_lib.load().kessie_page_workspace_bytes(num_pages), device, "pages", init=_init_page_workspace)


def page_insert(pool: torch.Tensor, new_k: torch.Tensor, new_v: torch.Tensor, target_pages: torch.Tensor,
                page_valid: torch.Tensor, page_positions: torch.Tensor, conv_pos: int,
                orig_pos: Optional[torch.Tensor] = None, tgt_pos: Optional[torch.Tensor] = None,
                rope_theta: Optional[float] = None, layout: str = "native", stream=None) -> None:
    """Insert new_k/new_v [T, H, D] into pages (optionally remapping K)."""
    pv = pool_view(pool, layout)
    new_k, new_v = _contig(new_k, "new_k"), _contig(new_v, "new_v")
    t, h, d = new_k.shape
    if new_v.shape != new_k.shape or h != pv.num_kv_heads or d != pv.head_dim:
        raise ValueError("new_k/new_v shape does not match the pool")
    if new_k.dtype != pool.dtype or new_v.dtype != pool.dtype:
        raise TypeError("new_k/new_v dtype must match the pool")
    if target_pages.dtype != torch.int32 or page_valid.dtype != torch.int8 or page_positions.dtype != torch.int32:
        raise TypeError("target_pages int32, page_valid int8, page_positions int32 expected")
    if target_pages.numel() * pv.page_size < t:
        raise ValueError("target_pages too short for the token count")
    if page_valid.numel() < pv.num_pages or page_positions.numel() < pv.num_pages:
        raise ValueError("page_valid / page_positions shorter than the pool")
    inv = None
    if orig_pos is not None or tgt_pos is not None:
        if orig_pos is None or tgt_pos is None or rope_theta is None:
            raise ValueError("orig_pos, tgt_pos and rope_theta go together")
        inv = inv_freq_table(d, rope_theta, pool.device)
    lib = _lib.load()
    _lib.check("kessie_page_insert_paged", lib.kessie_page_insert_paged(
        C.c_void_p(pv.k_ptr), pv.page_stride, pv.tok_stride, pv.kv_stride, pv.head_stride, _ptr(new_k),
        _ptr(new_v), _ptr(_contig(target_pages, "target_pages")), _ptr(page_valid), _ptr(page_positions),
        int(conv_pos), _ptr(orig_pos), _ptr(tgt_pos), _ptr(inv), t, h, d, pv.page_size, pv.num_pages,
        dtype_code(pool.dtype), _stream_ptr(stream, pool.device)))


def page_evict_list(page_valid: torch.Tensor, page_positions: torch.Tensor, evict_before_pos: int,
                    allocated: Optional[torch.Tensor] = None, stream=None):
    """Threshold eviction reporting freed ids ascending.  Returns (list[n_pages], count[1])
    device tensors; the first count entries of the list are valid."""
    n = page_valid.numel()
    dev = page_valid.device
    freed = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = page_workspace(n, dev)
    lib = _lib.load()
    _lib.check("kessie_page_evict_list", lib.kessie_page_evict_list(
        _ptr(page_valid), _ptr(page_positions), _ptr(allocated), int(evict_before_pos), n, _ptr(freed),
        _ptr(count), _ptr(ws), ws.numel(), _stream_ptr(stream, dev)))
    return freed, count


def page_select_evict(scores: torch.Tensor, page_valid: torch.Tensor, k_evict: int = -1,
                      evict_fraction: float = 0.25, evict_list: Optional[torch.Tensor] = None,
                      evict_count: Optional[torch.Tensor] = None, stream=None):
    """Evict the k lowest (score, id) valid pages.  Returns (evict_list, evict_count)."""
    n = page_valid.numel()
    dev = page_valid.device
    if scores.dtype != torch.float32 or scores.numel() < n:
        raise ValueError("scores must be float32 with one entry per page")
    if evict_list is None:
        evict_list = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    if evict_count is None:
        evict_count = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = page_workspace(n, dev)
    lib = _lib.load()
    _lib.check("kessie_page_select_evict", lib.kessie_page_select_evict(
        _ptr(_contig(scores, "scores")), _ptr(page_valid), n, int(k_evict), float(evict_fraction),
        _ptr(evict_list), _ptr(evict_count), _ptr(ws), ws.numel(), _stream_ptr(stream, dev)))
    return evict_list, evict_count


def page_compact(tables: torch.Tensor, lens: torch.Tensor, page_valid: torch.Tensor,
                 new_tables: Optional[torch.Tensor] = None, new_lens: Optional[torch.Tensor] = None,
                 gather_idx: Optional[torch.Tensor] = None, gather_count: Optional[torch.Tensor] = None,
                 stream=None):
    """Compact page tables [S, W] by page_valid.  Returns (new_tables, new_lens, gather_idx, gather_count)."""
    tables = _contig(tables, "tables")
    s, w = tables.shape
    dev = tables.device
    if new_tables is None:
        new_tables = torch.empty_like(tables)
    if new_lens is None:
        new_lens = torch.empty(s, dtype=torch.int32, device=dev)
    if gather_idx is None:
        gather_idx = torch.empty(max(s * w, 1), dtype=torch.int32, device=dev)
    if gather_count is None:
        gather_count = torch.zeros(1, dtype=torch.int32, device=dev)
    n = max(s * w, s)
    ws = page_workspace(n, dev)
    lib = _lib.load()
    _lib.check("kessie_page_compact", lib.kessie_page_compact(
        _ptr(tables), _ptr(_contig(lens, "lens")), _ptr(page_valid), _ptr(new_tables), _ptr(new_lens),
        _ptr(gather_idx), _ptr(gather_count), s, w, page_valid.numel(), _ptr(ws), ws.numel(),
        _stream_ptr(stream, dev)))
    return new_tables, new_lens, gather_idx, gather_count


def page_evict_compact(scores: torch.Tensor, page_valid: torch.Tensor, tables: torch.Tensor, lens: torch.Tensor,
                       k_evict: int = -1, evict_fraction: float = 0.25, evict_list: Optional[torch.Tensor] = None,
                       evict_count: Optional[torch.Tensor] = None, new_tables: Optional[torch.Tensor] = None,
                       new_lens: Optional[torch.Tensor] = None, gather_idx: Optional[torch.Tensor] = None,
                       gather_count: Optional[torch.Tensor] = None, stream=None):
    """page_select_evict then page_compact by the post-eviction flags, fused
    into one launch.  Returns (evict_list, evict_count, new_tables, new_lens,
    gather_idx, gather_count), each equal to the two calls' outputs."""
    n = page_valid.numel()
    dev = page_valid.device
    if scores.dtype != torch.float32 or scores.numel() < n:
        raise ValueError("scores must be float32 with one entry per page")
    tables = _contig(tables, "tables")
    if tables.dtype != torch.int32 or lens.dtype != torch.int32:
        raise TypeError("tables and lens must be int32")
    s, w = tables.shape
    if evict_list is None:
        evict_list = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    if evict_count is None:
        evict_count = torch.zeros(1, dtype=torch.int32, device=dev)
    if new_tables is None:
        new_tables = torch.empty_like(tables)
    if new_lens is None:
        new_lens = torch.empty(s, dtype=torch.int32, device=dev)
    if gather_idx is None:
        gather_idx = torch.empty(max(s * w, 1), dtype=torch.int32, device=dev)
    if gather_count is None:
        gather_count = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = page_workspace(max(n, s), dev)
    lib = _lib.load()
    _lib.check("kessie_page_evict_compact", lib.kessie_page_evict_compact(
        _ptr(_contig(scores, "scores")), _ptr(page_valid), n, int(k_evict), float(evict_fraction),
        _ptr(evict_list), _ptr(evict_count), _ptr(tables), _ptr(_contig(lens, "lens")), s, w, _ptr(new_tables),
        _ptr(new_lens), _ptr(gather_idx), _ptr(gather_count), _ptr(ws), ws.numel(), _stream_ptr(stream, dev)))
    return evict_list, evict_count, new_tables, new_lens, gather_idx, gather_count


def page_valid_list(page_valid: torch.Tensor, stream=None):
    """Valid page ids ascending (get_layer_kv order).  Returns (idx, count) device tensors."""
    n = page_valid.numel()
    dev = page_valid.device
    idx = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = page_workspace(n, dev)
    lib = _lib.load()
    _lib.check("kessie_page_valid_list", lib.kessie_page_valid_list(
        _ptr(page_valid), n, _ptr(idx), _ptr(count), _ptr(ws), ws.numel(), _stream_ptr(stream, dev)))
    return idx, count


def page_gather(pool: torch.Tensor, idx: torch.Tensor, count: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, n: Optional[int] = None, stream=None) -> torch.Tensor:
    """dst[i] = pool[idx[i]] (whole pages, byte copy) for i < min(n, *count)."""
    pool = _contig(pool, "pool")
    num_pages = pool.shape[0]
    page_bytes = pool[0].numel() * pool.element_size()
    if n is None:
        n = idx.numel()
    if out is None:
        out = torch.empty((n,) + tuple(pool.shape[1:]), dtype=pool.dtype, device=pool.device)
    lib = _lib.load()
    _lib.check("kessie_page_gather", lib.kessie_page_gather(
        _ptr(pool), page_bytes, _ptr(_contig(idx, "idx")), _ptr(count), int(n), num_pages, _ptr(out),
        _stream_ptr(stream, pool.device)))
    return out


# ---------------------------------------------------------------------------
# Producers around the attention call
# ---------------------------------------------------------------------------
def fog_bias_fill(buf: torch.Tensor, kv_len: int, fog_alpha: float, fog_start: float,
                  recall_positions: Optional[torch.Tensor] = None, recall_boost: float = 0.1,
                  stream=None) -> torch.Tensor:
    """Fog logit bias into buf[:kv_len] in buf's dtype (the device version of
    _FogCache._compute_into, kessie_attention.py:114-139).  recall_positions:
    int32 device tensor (any order, duplicates allowed) or None.  Returns the
    buf[:kv_len] view."""
    if buf.dim() != 1 or not buf.is_contiguous():
        raise ValueError("buf must be a contiguous 1-D tensor")
    if kv_len < 0 or kv_len > buf.numel():
        raise ValueError(f"kv_len {kv_len} outside [0, {buf.numel()}]")
    n = 0
    if recall_positions is not None:
        if recall_positions.dtype != torch.int32 or recall_positions.device != buf.device:
            raise TypeError("recall_positions must be int32 on the buffer's device")
        recall_positions = _contig(recall_positions.reshape(-1), "recall_positions")
        n = recall_positions.numel()
    lib = _lib.load()
    _lib.check("kessie_fog_bias_fill", lib.kessie_fog_bias_fill(
        _ptr(buf), dtype_code(buf.dtype), int(kv_len), float(fog_alpha), float(fog_start),
        _ptr(recall_positions) if n else None, n, float(recall_boost), _stream_ptr(stream, buf.device)))
    return buf[:kv_len]


def fog_bias_rows(out: torch.Tensor, seq_lens: torch.Tensor, dtype: torch.dtype, fog_alpha: float,
                  fog_start: float, recall_positions: Optional[torch.Tensor] = None, recall_boost: float = 0.1,
                  stream=None) -> torch.Tensor:
    """Per-sequence fog bias: row b of ``out`` (fp32 [B, N], rows contiguous)
    receives fog_bias_fill's vector for kv_len = seq_lens[b] (int32 device
    tensor), computed in ``dtype`` and widened to fp32; positions at or past
    seq_lens[b] are 0.  Returns out."""
    if out.dtype != torch.float32 or out.dim() != 2 or out.stride(1) != 1:
        raise ValueError("out must be fp32 [B, N] with contiguous rows")
    b, n = out.shape
    if seq_lens.dtype != torch.int32 or seq_lens.numel() < b or seq_lens.device != out.device:
        raise ValueError("seq_lens must be int32 with one entry per row, on out's device")
    nr = 0
    if recall_positions is not None:
        if recall_positions.dtype != torch.int32 or recall_positions.device != out.device:
            raise TypeError("recall_positions must be int32 on out's device")
        recall_positions = _contig(recall_positions.reshape(-1), "recall_positions")
        nr = recall_positions.numel()
    lib = _lib.load()
    _lib.check("kessie_fog_bias_fill_rows", lib.kessie_fog_bias_fill_rows(
        _ptr(out), out.stride(0), _ptr(_contig(seq_lens, "seq_lens")), b, n, dtype_code(dtype), float(fog_alpha),
        float(fog_start), _ptr(recall_positions) if nr else None, nr, float(recall_boost),
        _stream_ptr(stream, out.device)))
    return out


def fog_weights(seq_len: int, fog_alpha: float = 0.5, fog_start: float = 0.5, device=None,
                out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Fog V weights, fp32 [seq_len], computed on the device (the device
    version of kessie_build_fog_weights, kessie_hip_kernels.py:403-413)."""
    if out is None:
        out = torch.empty(seq_len, dtype=torch.float32, device=device or "cuda")
    if out.dtype != torch.float32 or out.dim() != 1 or not out.is_contiguous() or out.numel() < seq_len:
        raise ValueError("out must be a contiguous fp32 vector of at least seq_len elements")
    lib = _lib.load()
    _lib.check("kessie_fog_weights_fill", lib.kessie_fog_weights_fill(
        _ptr(out), int(seq_len), float(fog_alpha), float(fog_start), _stream_ptr(stream, out.device)))
    return out[:seq_len]


def kv_cache_write(pool: torch.Tensor, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor,
                   layout: str = "native", stream=None) -> None:
    """Write key/value [T, Hkv, D] (any token/head strides, D contiguous) into
    the paged pool at slot_mapping[t] (int64; page = slot // P, offset
    slot % P; negative slots skipped)."""
    pv = pool_view(pool, layout)
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError("key/value must both be [T, Hkv, D]")
    t, h, d = key.shape
    if h != pv.num_kv_heads or d != pv.head_dim:
        raise ValueError("key/value heads or head_dim do not match the pool")
    if key.dtype != pool.dtype or value.dtype != pool.dtype:
        raise TypeError("key/value dtype must match the pool")
    if key.stride(2) != 1 or value.stride(2) != 1:
        raise ValueError("key/value head_dim axis must be contiguous")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() < t:
        raise ValueError("slot_mapping must be int64 with one entry per token")
    lib = _lib.load()
    _lib.check("kessie_kv_cache_write", lib.kessie_kv_cache_write(
        C.c_void_p(pv.k_ptr), pv.page_stride, pv.tok_stride, pv.kv_stride, pv.head_stride,
        _ptr(key), key.stride(0), key.stride(1), _ptr(value), value.stride(0), value.stride(1),
        _ptr(_contig(slot_mapping, "slot_mapping")), t, h, d, pv.page_size, pv.num_pages,
        dtype_code(pool.dtype), _stream_ptr(stream, pool.device)))


# ---------------------------------------------------------------------------
# Semantic index query
# ---------------------------------------------------------------------------
def index_query(embeds: torch.Tensor, query: torch.Tensor, top_k: int = 0, norm_mode: int = 0,
                sims: Optional[torch.Tensor] = None, stream=None):
    """Cosine similarity of ``query`` (fp32 [D]) against every row of
    ``embeds`` ([N, D], fp32/bf16/fp16, rows contiguous) and the top_k rows
    (similarity descending, ties by ascending row).  Returns (sims [N] fp32,
    ids [top_k] int32 or None, scores [top_k] fp32 or None); ids past N are -1."""
    if embeds.dim() != 2 or embeds.stride(1) != 1:
        raise ValueError("embeds must be [N, D] with contiguous rows")
    n, d = embeds.shape
    dev = embeds.device
    query = query.reshape(-1)
    if query.dtype != torch.float32 or query.numel() != d or query.device != dev:
        raise ValueError("query must be fp32 [D] on the embeddings' device")
    query = _contig(query, "query")
    if sims is None:
        sims = torch.empty(n, dtype=torch.float32, device=dev)
    ids = scores = None
    lib = _lib.load()
    need = lib.kessie_index_query_workspace_bytes(n, int(top_k)) if top_k > 0 else 0
    ws = workspace(need, dev, "index") if need else None
    if top_k > 0:
        ids = torch.empty(top_k, dtype=torch.int32, device=dev)
        scores = torch.empty(top_k, dtype=torch.float32, device=dev)
    _lib.check("kessie_index_query", lib.kessie_index_query(
        _ptr(embeds) if n else None, embeds.stride(0), n, d, dtype_code(embeds.dtype), int(norm_mode),
        _ptr(query), _ptr(sims), int(top_k), _ptr(ids), _ptr(scores), _ptr(ws),
        0 if ws is None else ws.numel(), _stream_ptr(stream, dev)))
    return sims, ids, scores


# ---------------------------------------------------------------------------
# Fog of the HF tiered cache
# ---------------------------------------------------------------------------
def hf_fog_weights(seq_len: int, fog_alpha: float, fog_start: float, device=None,
                   out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """KeSSieCache fog weights, fp32 [seq_len] (kessie_exp3.py:415-425)."""
    if out is None:
        out = torch.empty(seq_len, dtype=torch.float32, device=device or "cuda")
    if out.dtype != torch.float32 or out.dim() != 1 or not out.is_contiguous() or out.numel() < seq_len:
        raise ValueError("out must be a contiguous fp32 vector of at least seq_len elements")
    lib = _lib.load()
    _lib.check("kessie_hf_fog_weights_fill", lib.kessie_hf_fog_weights_fill(
        _ptr(out), int(seq_len), float(fog_alpha), float(fog_start), _stream_ptr(stream, out.device)))
    return out[:seq_len]


def hf_append_fog(k_arena: torch.Tensor, v_arena: torch.Tensor, off: int, n_old: int, new_k: torch.Tensor,
                  new_v: torch.Tensor, vfog: Optional[torch.Tensor], fog_alpha: float, fog_start: float,
                  stream=None) -> bool:
    """One KeSSieCache layer update in one launch: new_k/new_v [B, H, T, D] go
    to arena positions off+n_old .. off+n_old+T-1, and, if ``vfog`` (a
    [B, H, n_old+T, D] view) is given, it receives the fog-weighted V of the
    whole window.  Returns False, having done nothing, when a row is not a
    16-byte aligned multiple of 16 bytes (the caller then copies and calls
    hf_fog_apply)."""
    b, h, t, d = new_k.shape
    if (k_arena.dim() != 4 or k_arena.shape != v_arena.shape or k_arena.stride() != v_arena.stride()
            or new_v.shape != new_k.shape or k_arena.dtype != new_k.dtype or new_v.dtype != new_k.dtype
            or k_arena.shape[0] != b or k_arena.shape[1] != h or k_arena.shape[3] != d
            or off + n_old + t > k_arena.shape[2] or k_arena.stride(3) != 1 or new_k.stride(3) != 1
            or new_v.stride(3) != 1):
        raise ValueError("hf_append_fog: arena / new state shapes do not match")
    if vfog is not None and (vfog.shape != (b, h, n_old + t, d) or vfog.dtype != new_k.dtype or vfog.stride(3) != 1):
        raise ValueError("hf_append_fog: vfog must be [B, H, n_old+T, D] of the cache dtype")
    es = k_arena.element_size()
    kp = k_arena.data_ptr() + off * k_arena.stride(2) * es
    vp = v_arena.data_ptr() + off * v_arena.stride(2) * es
    lib = _lib.load()
    st = lib.kessie_hf_append_fog(
        C.c_void_p(kp), C.c_void_p(vp), k_arena.stride(0), k_arena.stride(1), k_arena.stride(2),
        _ptr(new_k), new_k.stride(0), new_k.stride(1), new_k.stride(2),
        _ptr(new_v), new_v.stride(0), new_v.stride(1), new_v.stride(2),
        _ptr(vfog),
        vfog.stride(0) if vfog is not None else 0, vfog.stride(1) if vfog is not None else 0,
        vfog.stride(2) if vfog is not None else 0,
        b, h, n_old, t, d, float(fog_alpha), float(fog_start), dtype_code(new_k.dtype),
        _stream_ptr(stream, k_arena.device))
    if st == _lib.ERR_UNSUPPORTED:
        return False
    _lib.check("kessie_hf_append_fog", st)
    return True


def hf_fog_apply(v: torch.Tensor, fog_alpha: float, fog_start: float, out: Optional[torch.Tensor] = None,
                 stream=None) -> torch.Tensor:
    """out = dtype(fp32(v) * w[t]) for v [B, H, N, D] (head_dim contiguous) with
    KeSSieCache's fog weights over N positions, in one pass."""
    if v.dim() != 4 or v.stride(3) != 1:
        raise ValueError("v must be [B, H, N, D] with a contiguous head_dim")
    if out is None:
        out = torch.empty_like(v)
    if out.shape != v.shape or out.dtype != v.dtype or out.stride(3) != 1:
        raise ValueError("out must match v")
    b, h, n, d = v.shape
    lib = _lib.load()
    _lib.check("kessie_hf_fog_apply", lib.kessie_hf_fog_apply(
        _ptr(v), v.stride(0), v.stride(1), v.stride(2), _ptr(out), out.stride(0), out.stride(1), out.stride(2),
        b, h, n, d, float(fog_alpha), float(fog_start), dtype_code(v.dtype), _stream_ptr(stream, v.device)))
    return out
