"""ctypes bindings of libkessie_mi355x.so (every symbol of include/kessie_mi355x.h).

The library is located, in order, at $KESSIE_MI355X_LIB, next to this file
(the in-tree build of ``python -m kessie_amd.build``), and ./build/.  There is
no fallback: if the library is absent, ``load()`` raises.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

LIB_NAME = "libkessie_mi355x.so"

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

OK = 0
ERR_INVALID = 1
ERR_UNSUPPORTED = 2
ERR_WORKSPACE = 3
ERR_HIP = 4

_P = C.c_void_p
_I = C.c_int
_I64 = C.c_int64
_F = C.c_float
_D = C.c_double
_SZ = C.c_size_t

# name -> (restype, argtypes).  Kept in the order of include/kessie_mi355x.h.
SIGNATURES = {
    "kessie_get_last_error": (_I, [C.c_char_p, _SZ]),
    "kessie_version": (_I, []),
    # legacy launchers (reference signatures, void return)
    "launch_kessie_windowed_attn": (None, [_P, _P, _P, _P, _F, _I, _I, _I, _I, _I, _I, _P]),
    "launch_kessie_fused_fog_attn": (None, [_P, _P, _P, _P, _P, _F, _I, _I, _I, _I, _I, _I, _P]),
    "launch_kessie_page_evict": (None, [_P, _P, _P, _I, _I, _P]),
    "launch_kessie_page_insert": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "launch_kessie_rope_remap": (None, [_P, _P, _P, _F, _I, _I, _I, _P]),
    # paged fog attention
    "kessie_fog_decode_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I, _I]),
    # q, pool, num_pages, 4 strides, table, table_stride, ctx_lens, vscale, vs_bstride,
    # bias, bias_bstride, out, B, Hq, Hkv, D, P, max_ctx, window, sm_scale, dtype, ws, ws_bytes, stream
    "kessie_fog_decode_paged": (_I, [
        _P, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P, _I64,
        _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _SZ, _P]),
    # as kessie_fog_decode_paged without ws, ws_bytes
    "kessie_fog_decode_paged_noalloc": (_I, [
        _P, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P, _I64,
        _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P]),
    "kessie_fog_decode_num_splits": (_I, [_I, _I, _I, _I]),
    # as kessie_fog_decode_paged without `out`
    "kessie_fog_decode_partials": (_I, [
        _P, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P, _I64,
        _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _SZ, _P]),
    "kessie_fog_decode_combine": (_I, [_P, _SZ, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "kessie_fog_prefill_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I, _I, _I]),
    # ... out, B, C, Hq, Hkv, D, P, max_ctx, window, sm_scale, causal, dtype, ws, ws_bytes, stream
    "kessie_fog_prefill_paged": (_I, [
        _P, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P, _I64,
        _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P, _SZ, _P]),
    "kessie_fog_prefill_varlen": (_I, [
        _P, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P, _I64,
        _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P, _SZ, _P]),
    # rope remap
    "kessie_rope_remap_paged": (_I, [_P, _I64, _I64, _I64, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    # page management
    "kessie_page_insert_paged": (_I, [
        _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I, _P, _P, _P,
        _I, _I, _I, _I, _I, _I, _P]),
    "kessie_page_evict_list": (_I, [_P, _P, _P, _I, _I, _P, _P, _P, _SZ, _P]),
    "kessie_page_workspace_bytes": (_SZ, [_I]),
    "kessie_page_workspace_init": (_I, [_P, _SZ, _P]),
    "kessie_page_select_evict": (_I, [_P, _P, _I, _I, _F, _P, _P, _P, _SZ, _P]),
    "kessie_page_compact": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _SZ, _P]),
    # scores, valid, num_pages, k, frac, evict_list, evict_count, tables, lens, S, W, new_tables, new_lens,
    # gather_idx, gather_count, ws, ws_bytes, stream
    "kessie_page_evict_compact": (_I, [_P, _P, _I, _I, _F, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _P, _SZ, _P]),
    "kessie_page_valid_list": (_I, [_P, _I, _P, _P, _P, _SZ, _P]),
    "kessie_page_gather": (_I, [_P, _I64, _P, _P, _I, _I, _P, _P]),
    # buf, dtype, kv_len, fog_alpha, fog_start, recall, num_recall, boost, stream
    "kessie_fog_bias_fill": (_I, [_P, _I, _I, _D, _D, _P, _I, _D, _P]),
    # out, row_stride, seq_lens, rows, max_len, dtype, fog_alpha, fog_start, recall, num_recall, boost, stream
    "kessie_fog_bias_fill_rows": (_I, [_P, _I64, _P, _I, _I, _I, _D, _D, _P, _I, _D, _P]),
    "kessie_fog_weights_fill": (_I, [_P, _I, _D, _D, _P]),
    # pool + 4 strides, key + 2 strides, value + 2 strides, slots, T, H, D, P, pages, dtype, stream
    "kessie_hf_fog_weights_fill": (_I, [_P, _I, _D, _D, _P]),
    "kessie_hf_append_fog": (_I, [_P, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64,
                                  _P, _I64, _I64, _I64, _I, _I, _I, _I, _I, _D, _D, _I, _P]),
    # v + 3 strides, out + 3 strides, B, H, N, D, fog_alpha, fog_start, dtype, stream
    "kessie_hf_fog_apply": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I, _I, _I, _I, _D, _D, _I, _P]),
    "kessie_index_query_workspace_bytes": (_SZ, [_I, _I]),
    # index, row_stride, num_chunks, embed_dim, dtype, norm_mode, query, sims, top_k, ids, scores, ws, ws_bytes, stream
    "kessie_index_query": (_I, [_P, _I64, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P, _SZ, _P]),
    "kessie_kv_cache_write": (_I, [
        _P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P,
        _I, _I, _I, _I, _I, _I, _P]),
}

_lock = threading.Lock()
_lib = None
_path = None


class KeSSieError(RuntimeError):
    """A libkessie_mi355x entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed (status {status}): {message}")
        self.fn = fn
        self.status = status
        self.message = message


def candidates() -> list[str]:
    here = os.path.dirname(os.path.abspath(__file__))
    out = []
    env = os.environ.get("KESSIE_MI355X_LIB")
    if env:
        out.append(env)
    out.append(os.path.join(here, LIB_NAME))
    out.append(os.path.join(os.getcwd(), "build", LIB_NAME))
    return out


def load(path: str | None = None):
    """Open the library (once) and declare every entry point's argtypes."""
    global _lib, _path
    with _lock:
        if _lib is not None and (path is None or path == _path):
            return _lib
        if path is None:
            for cand in candidates():
                if os.path.exists(cand):
                    path = cand
                    break
        if path is None or not os.path.exists(path):
            raise FileNotFoundError(
                f"{LIB_NAME} not found (searched {candidates()}); build it with "
                f"`python -m kessie_amd.build`")
        lib = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib, _path = lib, path
        return lib


def lib_path() -> str | None:
    return _path


def last_error() -> tuple[int, str]:
    lib = load()
    buf = C.create_string_buffer(512)
    status = lib.kessie_get_last_error(buf, len(buf))
    return status, buf.value.decode(errors="replace")


def check(fn: str, status: int) -> None:
    if status != OK:
        _, msg = last_error()
        raise KeSSieError(fn, status, msg)


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise on failure."""
    lib = load()
    check(name, getattr(lib, name)(*args))


def call_legacy(name: str, *args) -> None:
    """Call a void legacy launcher, then raise if it recorded an error."""
    lib = load()
    getattr(lib, name)(*args)
    status, msg = last_error()
    if status != OK:
        raise KeSSieError(name, status, msg)
