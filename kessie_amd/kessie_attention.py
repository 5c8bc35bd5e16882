"""KeSSie fog-of-war attention backend on the MI355X kernels.

Mirrors the surface of the reference's kessie_attention.py -- the global
parameter state (KeSSieAttentionState / KESSIE_STATE, :27-62), the shared
per-step fog cache (_FogCache, :67-185), register_kessie_attention (:188-213)
and the backend / impl pair (:234-307) -- with the same names, signatures,
defaults and bypass rules.  What changes is underneath:

  * the fog bias is produced on the device in one launch (plus one for the
    recall scatter) by kessie_fog_bias_fill instead of a chain of torch ops and
    one host-driven scalar write per recalled position (:137-139);
  * the next step's bias is precomputed on a side stream that first waits for
    the compute stream (the buffer it overwrites may still be read there), and
    the consumer makes its stream wait on the side stream's event instead of
    blocking the host (:160-161);
  * KeSSieAttentionImpl.forward runs attention itself -- slot-mapped K/V write,
    paged fog decode for single-token queries and chunked fog prefill for the
    rest -- with kv_len taken from the attention metadata, instead of handing an
    ``attn_bias`` to vLLM's inner backend (whose TRITON_ATTN / FLASH_ATTN
    kernels take no such argument, and whose ``key.shape[-2]`` is the number of
    kv heads, not the context length: :293).

When vLLM is importable the backend also keeps the original backend's
metadata class and KV-cache shape, and bypassed calls go to the original
implementation exactly as in the reference.  Without vLLM the classes are
still usable on their own with a metadata object carrying vLLM's field names
(KeSSieAttentionMetadata).
"""
from __future__ import annotations

import logging
import os
import threading
from dataclasses import dataclass
from typing import Optional, Set

import torch

logger = logging.getLogger("KeSSie.Attention")


# --- Global KeSSie attention state (thread-safe, set per request) -------------

class KeSSieAttentionState:
    """Thread-safe global fog parameters (kessie_attention.py:27-60)."""

    def __init__(self):
        self._lock = threading.Lock()
        self.fog_alpha: float = 0.5
        self.fog_start: float = 0.5
        self.prompt_len: int = 0
        self.recall_positions: Set[int] = set()
        self.recall_boost: float = 0.1
        self.enabled: bool = True
        self.generation: int = 0

    def update(self, fog_alpha=None, fog_start=None, prompt_len=None,
               recall_positions=None, recall_boost=None):
        with self._lock:
            if fog_alpha is not None:
                self.fog_alpha = fog_alpha
            if fog_start is not None:
                self.fog_start = fog_start
            if prompt_len is not None:
                self.prompt_len = prompt_len
            if recall_positions is not None:
                self.recall_positions = set(recall_positions)
            if recall_boost is not None:
                self.recall_boost = recall_boost
            self.generation += 1

    def get(self):
        with self._lock:
            return {
                "fog_alpha": self.fog_alpha,
                "fog_start": self.fog_start,
                "prompt_len": self.prompt_len,
                "recall_positions": set(self.recall_positions),
                "recall_boost": self.recall_boost,
                "enabled": self.enabled,
                "generation": self.generation,
            }


KESSIE_STATE = KeSSieAttentionState()


# --- Shared per-step fog cache -------------------------------------------------

class _FogCache:
    """Fog bias computed once per generation and shared by every layer of the
    step (kessie_attention.py:67-185): two ping-pong buffers, the next
    generation precomputed on a side stream, a cached (1,1,1,kv_len) view."""

    def __init__(self):
        self._gen = -1
        self._kv_len = 0
        self._buf_a = None
        self._buf_b = None
        self._active = 0
        self._alloc_len = 0
        self._device = None
        self._dtype = None
        self._stream = None
        self._event = None
        self._pending = False
        self._pending_gen = -1
        self._pending_key = None
        self._view = None
        self._view_kv_len = 0
        self._compute_lock = threading.Lock()
        self._recall_key = None
        self._recall_dev = None
        self._rows_cache = None  # (key, view) of get_fog_bias_rows
        self._rows_buf = None
        self._rows_graph_buf = None
        self._rows_retired = []

    def _ensure_alloc(self, kv_len, device, dtype):
        if self._alloc_len >= kv_len and self._device == device and self._dtype == dtype:
            return
        alloc = max(kv_len, 2048)
        alloc = (alloc + 255) & ~255
        self._buf_a = torch.zeros(alloc, device=device, dtype=dtype)
        self._buf_b = torch.zeros(alloc, device=device, dtype=dtype)
        self._alloc_len = alloc
        self._device = device
        self._dtype = dtype
        self._gen = -1
        self._view = None
        self._pending = False
        if self._stream is None or self._stream.device != torch.device(device):
            self._stream = torch.cuda.Stream(device=device)
            self._event = torch.cuda.Event()

    @staticmethod
    def _recall_tensor(recall_pos, device) -> Optional[torch.Tensor]:
        pos = sorted(int(p) for p in recall_pos if -(1 << 31) <= int(p) < (1 << 31))
        if not pos:
            return None
        host = torch.tensor(pos, dtype=torch.int32).pin_memory()
        return host.to(device, non_blocking=True)

    @staticmethod
    def _compute_into(buf, kv_len, fog_alpha, fog_start, recall_pos, recall_boost=0.1):
        """Fog bias into buf[:kv_len] (kessie_attention.py:114-139), on the
        device, on the current stream: -fog_alpha*(1-p/B)^2 for p < B =
        int(kv_len*(1-fog_start)), 0 in the clear zone, recall_boost at every
        recalled position in [0, kv_len)."""
        from . import ops

        rec = recall_pos if isinstance(recall_pos, torch.Tensor) else _FogCache._recall_tensor(recall_pos, buf.device)
        ops.fog_bias_fill(buf, kv_len, fog_alpha, fog_start, rec, recall_boost)

    def _recall_for(self, recall_pos, device):
        key = (frozenset(recall_pos), str(device))
        if key != self._recall_key:
            self._recall_dev = self._recall_tensor(recall_pos, device)
            self._recall_key = key
        return self._recall_dev

    def get_fog_bias(self, kv_len, device, dtype, state):
        """Return the (1,1,1,kv_len) fog bias, computed once per generation."""
        gen = state["generation"]
        if self._gen == gen and self._kv_len == kv_len and self._view is not None:
            return self._view
        with self._compute_lock:
            if self._gen == gen and self._kv_len == kv_len and self._view is not None:
                return self._view
            self._ensure_alloc(kv_len, device, dtype)
            recall_pos = frozenset(state["recall_positions"])
            fog_alpha = state["fog_alpha"]
            fog_start = state["fog_start"]
            recall_boost = state.get("recall_boost", 0.1)
            params = (kv_len, fog_alpha, fog_start, recall_pos, recall_boost)
            main = torch.cuda.current_stream(device)
            recall = self._recall_for(recall_pos, device)

            if self._pending and self._pending_gen == gen and self._pending_key == params:
                # The side stream already produced this generation: order the
                # compute stream after it and swap buffers (no host wait).
                main.wait_event(self._event)
                self._pending = False
                self._active = 1 - self._active
            else:
                self._pending = False
                active = self._buf_a if self._active == 0 else self._buf_b
                self._compute_into(active, kv_len, fog_alpha, fog_start, recall, recall_boost)

            self._gen = gen
            self._kv_len = kv_len
            active = self._buf_a if self._active == 0 else self._buf_b
            self._view = active[:kv_len].view(1, 1, 1, kv_len)
            self._view_kv_len = kv_len

            # Precompute the next generation with the same parameters into the
            # other buffer, after everything already queued on the compute
            # stream (which may still read that buffer).
            next_buf = self._buf_b if self._active == 0 else self._buf_a
            self._stream.wait_stream(main)
            with torch.cuda.stream(self._stream):
                self._compute_into(next_buf, kv_len, fog_alpha, fog_start, recall, recall_boost)
                self._event.record(self._stream)
            if recall is not None:
                recall.record_stream(self._stream)
            self._pending = True
            self._pending_gen = gen + 1
            self._pending_key = params
            return self._view


    def get_fog_bias_rows(self, seq_lens, kv_len, device, dtype, state, seq_lens_host=None):
        """fp32 [B, kv_len] bias for a batch: row b is the vector get_fog_bias
        builds (in ``dtype``, widened to fp32) for that sequence's own kv_len =
        seq_lens[b], zero past it.  One launch on the current stream, no host
        synchronisation.  Shared by the layers of a step when the lengths are
        known on the host (``seq_lens_host``): cached per generation and length
        tuple; without them it is recomputed on every call.

        Under HIP graph capture the fill is always recorded (a cached view
        would leave the graph without it, replaying whatever an eager call
        left there) into a buffer of its own that is never freed, so replays
        neither read stale rows nor write into memory handed out again."""
        from . import ops

        b = int(seq_lens.numel())
        capturing = torch.device(device).type == "cuda" and torch.cuda.is_current_stream_capturing()
        key = None
        if seq_lens_host is not None and not capturing:
            key = (state["generation"], kv_len, str(device), dtype, tuple(int(x) for x in seq_lens_host.tolist()))
            cached = self._rows_cache  # (key, view), replaced as one attribute
            if cached is not None and cached[0] == key:
                return cached[1]
        with self._compute_lock:
            attr = "_rows_graph_buf" if capturing else "_rows_buf"
            rows_buf = getattr(self, attr, None)
            if (rows_buf is None or rows_buf.shape[0] < b or rows_buf.shape[1] < kv_len
                    or rows_buf.device != torch.device(device)):
                if rows_buf is not None:
                    # A graph captured with it (or a stream still reading it)
                    # may use it later: keep it alive.
                    self._rows_retired.append(rows_buf)
                cols = (max(kv_len, 2048) + 255) & ~255
                rows_buf = torch.empty(max(b, 16), cols, dtype=torch.float32, device=device)
                setattr(self, attr, rows_buf)
            view = rows_buf[:b, :kv_len]
            lens = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
            recall = self._recall_for(frozenset(state["recall_positions"]), device)
            ops.fog_bias_rows(view, lens, dtype, state["fog_alpha"], state["fog_start"], recall,
                              state.get("recall_boost", 0.1))
            if not capturing:
                self._rows_cache = (key, view) if key is not None else None
            return view

    def get_fog_bias_f32(self, kv_len, device, dtype, state):
        """The current generation's bias (computed in ``dtype`` as above)
        widened to fp32 [kv_len] for the kernels, once per generation."""
        view = self.get_fog_bias(kv_len, device, dtype, state)
        if view.dtype == torch.float32:
            return view.view(kv_len)
        key = (self._gen, kv_len, view.data_ptr())
        if getattr(self, "_f32_key", None) != key:
            self._f32 = view.view(kv_len).float()
            self._f32_key = key
        return self._f32


def register_kessie_attention():
    """Register the KeSSie backend with vLLM (kessie_attention.py:188-213).
    Call before engine creation.  Returns False when vLLM's V1 registry is
    not importable."""
    try:
        from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend
    except ImportError:
        logger.warning("vLLM V1 attention registry not available")
        return False
    is_rocm = getattr(torch.version, "hip", None) is not None
    target = AttentionBackendEnum.TRITON_ATTN if is_rocm else AttentionBackendEnum.FLASH_ATTN
    os.environ["_KESSIE_ORIGINAL_ATTN_PATH"] = target.value
    register_backend(target, "kessie_amd.kessie_attention.KeSSieAttentionBackend")
    logger.info(f"  KeSSie attention registered (wrapping {target.value})")
    return True


# --- Backend and per-layer implementation ---------------------------------------

try:
    from vllm.utils.import_utils import resolve_obj_by_qualname
    from vllm.v1.attention.backend import AttentionBackend
    HAS_VLLM = True
except ImportError:
    HAS_VLLM = False

    class AttentionBackend:  # noqa: D401 - stand-in base when vLLM is absent
        pass

# Singleton fog cache (the reference creates it only with vLLM; here the
# kernels run either way).
_FOG_CACHE: Optional[_FogCache] = _FogCache()


@dataclass
class KeSSieAttentionMetadata:
    """The attention metadata fields the backend reads, named as in vLLM V1's
    FlashAttention / TritonAttention metadata.  Device tensors: query_start_loc
    int32 [B+1], seq_lens int32 [B], block_table int32 [B, max_blocks],
    slot_mapping int64 [num_tokens].  The *_cpu copies avoid a device sync
    when given."""
    num_actual_tokens: int
    max_query_len: int
    query_start_loc: torch.Tensor
    max_seq_len: int
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    query_start_loc_cpu: Optional[torch.Tensor] = None
    seq_lens_cpu: Optional[torch.Tensor] = None


class KeSSieAttentionBackend(AttentionBackend):
    """vLLM attention backend named "KeSSie" (kessie_attention.py:234-262)."""

    _original_cls = None

    @classmethod
    def _get_original(cls):
        if not HAS_VLLM:
            return None
        if cls._original_cls is None:
            path = os.environ.get("_KESSIE_ORIGINAL_ATTN_PATH", "")
            if path:
                cls._original_cls = resolve_obj_by_qualname(path)
            else:
                from vllm.v1.attention.backends.triton_attn import TritonAttentionBackend
                cls._original_cls = TritonAttentionBackend
        return cls._original_cls

    @classmethod
    def get_name(cls) -> str:
        return "KeSSie"

    @classmethod
    def get_impl_cls(cls):
        return KeSSieAttentionImpl

    @classmethod
    def get_metadata_cls(cls):
        orig = cls._get_original()
        return orig.get_metadata_cls() if orig is not None else KeSSieAttentionMetadata

    @classmethod
    def get_kv_cache_shape(cls, *args, **kwargs):
        orig = cls._get_original()
        if orig is not None:
            return orig.get_kv_cache_shape(*args, **kwargs)
        num_blocks, block_size, num_kv_heads, head_size = args[:4]
        return (2, num_blocks, block_size, num_kv_heads, head_size)


_IMPL_ARGS = ("num_heads", "head_size", "scale", "num_kv_heads", "alibi_slopes", "sliding_window",
              "kv_cache_dtype", "logits_soft_cap")


def _kv_layout(kv_cache: torch.Tensor) -> str:
    """'kv_first' for [2, blocks, P, H, D] (FLASH_ATTN), 'block_kv' for
    [blocks, 2, P, H, D] (TRITON_ATTN)."""
    if kv_cache.dim() != 5:
        raise ValueError(f"kv_cache must be 5-D, got {tuple(kv_cache.shape)}")
    if kv_cache.shape[0] == 2 and kv_cache.shape[1] != 2:
        return "kv_first"
    if kv_cache.shape[1] == 2 and kv_cache.shape[0] != 2:
        return "block_kv"
    return os.environ.get("KESSIE_KV_LAYOUT", "kv_first")


class KeSSieAttentionImpl:
    """Per-layer attention (kessie_attention.py:265-307).

    Constructed with vLLM's AttentionImpl arguments (num_heads, head_size,
    scale, num_kv_heads, alibi_slopes, sliding_window, kv_cache_dtype,
    logits_soft_cap, ...).  forward(layer, query, key, value, kv_cache,
    attn_metadata, output=None, ...) follows the reference's bypass rules
    (disabled, fog_alpha <= 0, prompt_len <= 0, an explicit attn_bias, fewer
    than four positional arguments) and otherwise attends with the fog bias of
    the current generation, each sequence's bias built for its own length
    (seq_lens[b]).
    """

    def __init__(self, *args, **kwargs):
        cfg = dict(zip(_IMPL_ARGS, args))
        for k in _IMPL_ARGS:
            if k in kwargs:
                cfg[k] = kwargs[k]
        self.num_heads = int(cfg["num_heads"])
        self.head_size = int(cfg["head_size"])
        self.scale = float(cfg.get("scale") or self.head_size ** -0.5)
        self.num_kv_heads = int(cfg.get("num_kv_heads") or self.num_heads)
        sw = cfg.get("sliding_window")
        if isinstance(sw, (tuple, list)):
            sw = sw[0] + 1 if sw[0] >= 0 else None
        self.window = int(sw) if sw else 0
        self.kv_cache_dtype = cfg.get("kv_cache_dtype", "auto")
        self.unsupported = bool(cfg.get("alibi_slopes") is not None or cfg.get("logits_soft_cap"))
        self._inner = None
        orig = KeSSieAttentionBackend._get_original()
        if orig is not None:
            self._inner = orig.get_impl_cls()(*args, **kwargs)

    # -- reference entry -------------------------------------------------------
    def forward(self, *args, **kwargs):
        state = KESSIE_STATE.get()
        fog_on = state["enabled"] and state["fog_alpha"] > 0 and state["prompt_len"] > 0
        if "attn_bias" in kwargs or len(args) < 4:
            return self._bypass(args, kwargs)
        if not fog_on:
            return self._bypass(args, kwargs)
        query, key = args[1], args[2]
        if not (hasattr(query, "shape") and hasattr(key, "shape") and key.dim() >= 2):
            return self._bypass(args, kwargs)
        return self._attend(args, kwargs, state)

    def _bypass(self, args, kwargs):
        if self._inner is not None:
            return self._inner.forward(*args, **kwargs)
        if len(args) < 6:
            raise TypeError("forward(layer, query, key, value, kv_cache, attn_metadata, output=None)")
        return self._attend(args, kwargs, None)

    def __getattr__(self, name):
        inner = self.__dict__.get("_inner")
        if inner is None:
            raise AttributeError(name)
        return getattr(inner, name)

    # -- the kernels --------------------------------------------------------------
    # (key, value) of the last split, replaced as one attribute so a reader
    # never pairs one call's key with another call's split.
    _split_cache = None

    @classmethod
    def _split(cls, meta):
        """(query_start_loc on the host, decode sequences, prefill sequences).
        Keyed by the content of the metadata's host copy query_start_loc_cpu,
        so every layer of a step shares one computation and a runner that
        refills one metadata object in place between steps is still seen;
        without a host copy, query_start_loc is copied from the device on each
        call."""
        host = getattr(meta, "query_start_loc_cpu", None)
        if host is not None:
            key = tuple(int(x) for x in host.tolist())
            cached = cls._split_cache
            if cached is not None and cached[0] == key:
                return cached[1]
            qsl = list(key)
        else:
            key = None
            qsl = [int(x) for x in meta.query_start_loc.cpu().tolist()]
        nseq = len(qsl) - 1
        decode = [i for i in range(nseq) if qsl[i + 1] - qsl[i] == 1]
        prefill = [i for i in range(nseq) if qsl[i + 1] - qsl[i] > 1]
        val = (qsl, decode, prefill)
        if key is not None:
            cls._split_cache = (key, val)
        return val

    def _attend(self, args, kwargs, state):
        from . import ops

        layer, query, key, value, kv_cache, meta = (list(args) + [None] * 6)[:6]
        output = args[6] if len(args) > 6 else kwargs.get("output")
        if meta is None:  # profiling run
            return output.fill_(0) if output is not None else torch.zeros_like(query)
        if self.unsupported or self.kv_cache_dtype not in ("auto", None) or kv_cache.dtype != query.dtype:
            if self._inner is not None:
                return self._inner.forward(*args, **kwargs)
            raise NotImplementedError("KeSSie kernels: ALiBi, soft-capping and quantised KV caches are not supported")
        hq, d = self.num_heads, self.head_size
        n_tok = int(getattr(meta, "num_actual_tokens", query.shape[0]))
        q = query[:n_tok].reshape(n_tok, hq, d)
        if not q.is_contiguous():
            q = q.contiguous()
        if output is None:
            output = torch.empty(query.shape[0], hq * d, dtype=query.dtype, device=query.device)
        out = output[:n_tok].view(n_tok, hq, d)
        layout = _kv_layout(kv_cache)
        # One stream lookup per call (each torch.cuda.current_stream costs a
        # few microseconds of host time, which short contexts notice).
        sp = torch.cuda.current_stream(query.device).cuda_stream

        # New K/V rows into the cache (skipped for layers that share a cache).
        if key is not None and value is not None:
            ops.kv_cache_write(kv_cache, key[:n_tok].reshape(n_tok, self.num_kv_heads, d),
                               value[:n_tok].reshape(n_tok, self.num_kv_heads, d), meta.slot_mapping[:n_tok],
                               layout=layout, stream=sp)

        kv_len = int(meta.max_seq_len)
        qsl, decode, prefill = self._split(meta)
        nseq = len(qsl) - 1
        table = meta.block_table[:nseq]
        lens = meta.seq_lens[:nseq]
        # Fog bias per sequence (row b built for that sequence's own length),
        # rows read with a batch stride by the kernels.
        bias = None
        if state is not None and kv_len > 0 and nseq > 0:
            lens_host = getattr(meta, "seq_lens_cpu", None)
            bias = _FOG_CACHE.get_fog_bias_rows(lens, kv_len, query.device, query.dtype, state,
                                                lens_host[:nseq] if lens_host is not None else None)

        if decode:
            if decode == list(range(decode[0], decode[0] + len(decode))):
                lo, hi = decode[0], decode[-1] + 1
                q_dec = q[qsl[lo]:qsl[lo] + (hi - lo)]
                ops.fog_decode(q_dec, kv_cache, table[lo:hi], lens[lo:hi], kv_len,
                               fog_bias=None if bias is None else bias[lo:hi],
                               window=self.window, sm_scale=self.scale, layout=layout,
                               out=out[qsl[lo]:qsl[lo] + (hi - lo)], stream=sp)
            else:
                idx = torch.tensor(decode, device=q.device)
                rows = torch.tensor([qsl[i] for i in decode], device=q.device)
                o_dec = ops.fog_decode(q.index_select(0, rows).contiguous(), kv_cache, table.index_select(0, idx),
                                       lens.index_select(0, idx), kv_len,
                                       fog_bias=None if bias is None else bias.index_select(0, idx), window=self.window,
                                       sm_scale=self.scale, layout=layout, stream=sp)
                out.index_copy_(0, rows, o_dec)
        if len(prefill) > 1 and prefill == list(range(prefill[0], prefill[-1] + 1)):
            # One launch for the whole run of prefill sequences (their chunk
            # lengths differ): query_start_loc's slice locates each one.
            lo, hi = prefill[0], prefill[-1] + 1
            s0, s1 = qsl[lo], qsl[hi]
            qs = meta.query_start_loc[lo:hi + 1]
            if qs.dtype != torch.int32:
                qs = qs.to(torch.int32)
            if ops.fog_prefill_varlen(q[s0:s1], qs, max(qsl[i + 1] - qsl[i] for i in prefill), kv_cache,
                                      table[lo:hi], lens[lo:hi], kv_len,
                                      fog_bias=None if bias is None else bias[lo:hi], window=self.window,
                                      causal=True, sm_scale=self.scale, layout=layout, out=out[s0:s1],
                                      stream=sp):
                prefill = []
        for i in prefill:
            s, e = qsl[i], qsl[i + 1]
            ops.fog_prefill(q[s:e].unsqueeze(0), kv_cache, table[i:i + 1], lens[i:i + 1], kv_len,
                            fog_bias=None if bias is None else bias[i:i + 1],
                            window=self.window, causal=True, sm_scale=self.scale, layout=layout,
                            out=out[s:e].unsqueeze(0), stream=sp)
        return output
