"""Attention oracles (test infrastructure only).

The reference's attention math is ``kessie_windowed_attention_ref`` /
``kessie_fused_fog_attention_ref`` (kessie_hip_kernels.py:577-593): dense
scores q@k^T*s, causal via tril, window 0 <= i-j < W, softmax, @ (v * w).
Its callers upcast to fp32 (kessie_hip_kernels.py:632,652), so the oracle
computes in fp32 on upcast inputs.

The paged / GQA / decode / chunked-prefill forms below are that same math
applied to the tokens a page table names: q head h reads kv head h // G
(HF repeat_kv order), restated by reshaping q to [Hkv, G, ...] rather than
materialising repeated K/V.  Decode = the last row of the dense math over ctx
tokens; chunked prefill = its last C rows.  Bias-mode fog adds b[j] to the
scaled scores (kessie_attention.py:114-139 producer, applied as attn_bias).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch


def windowed_attention_ref(q, k, v, window_size=0, causal=True, sm_scale=None):
    """kessie_windowed_attention_ref (kessie_hip_kernels.py:577-589), restated."""
    z, h, n, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    scores = torch.matmul(q, k.transpose(-2, -1)) * sm_scale
    if causal:
        scores = scores.masked_fill(~torch.tril(torch.ones(n, n, dtype=torch.bool)), float("-inf"))
    if window_size > 0:
        pos = torch.arange(n)
        dist = pos[:, None] - pos[None, :]
        scores = scores.masked_fill(~((dist >= 0) & (dist < window_size)), float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), v)


def fused_fog_attention_ref(q, k, v, fog_weights, window_size=0, causal=True, sm_scale=None):
    """kessie_fused_fog_attention_ref (kessie_hip_kernels.py:592-593): V rows scaled by w."""
    return windowed_attention_ref(q, k, v * fog_weights[None, None, :, None], window_size, causal, sm_scale)


def gather_seq_kv(pool: torch.Tensor, table_row: torch.Tensor, ctx: int):
    """K, V [ctx, Hkv, D] of one sequence from a native pool [pages, P, 2, Hkv, D]."""
    p = pool.shape[1]
    n_pages = (ctx + p - 1) // p
    pages = table_row[:n_pages].long()
    kv = pool[pages].reshape(n_pages * p, 2, pool.shape[3], pool.shape[4])[:ctx]
    return kv[:, 0], kv[:, 1]


def _attend_rows(qg: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_pos: torch.Tensor,
                 causal: bool, window: int, sm_scale: float,
                 vscale: Optional[torch.Tensor], bias: Optional[torch.Tensor]) -> torch.Tensor:
    """qg [Hkv, G, R, D] fp32 rows at absolute positions q_pos [R]; k, v [N, Hkv, D] fp32.

    Returns [Hkv, G, R, D].  Keys are positions 0..N-1.
    """
    n = k.shape[0]
    kt = k.permute(1, 2, 0).contiguous()              # [Hkv, D, N]
    vv = v if vscale is None else v * vscale[:, None, None]
    vt = vv.permute(1, 0, 2).contiguous()             # [Hkv, N, D]
    scores = torch.matmul(qg, kt[:, None]) * sm_scale  # [Hkv, G, R, N]
    if bias is not None:
        scores = scores + bias[None, None, None, :]
    j = torch.arange(n)
    dist = q_pos[:, None] - j[None, :]                 # [R, N]
    keep = torch.ones_like(dist, dtype=torch.bool)
    if causal:
        keep &= dist >= 0
    if window > 0:
        keep &= (dist >= 0) & (dist < window)
    scores = scores.masked_fill(~keep[None, None], float("-inf"))
    p = torch.softmax(scores, dim=-1)
    return torch.matmul(p, vt[:, None])


def paged_decode_ref(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor,
                     ctx_lens: torch.Tensor, fog_vscale: Optional[torch.Tensor] = None,
                     fog_bias: Optional[torch.Tensor] = None, window: int = 0,
                     sm_scale: Optional[float] = None) -> torch.Tensor:
    """Fog decode over paged KV (CPU, fp32).  q [B, Hq, D]; pool [pages, P, 2, Hkv, D].

    fog_vscale / fog_bias: None, [N] (shared) or [B, N] (per sequence).
    Returns fp32 [B, Hq, D].  A sequence with ctx 0 yields zeros (no keys).
    """
    b_, hq, d = q.shape
    hkv = pool.shape[3]
    g = hq // hkv
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    out = torch.zeros(b_, hq, d, dtype=torch.float32)
    for b in range(b_):
        ctx = int(ctx_lens[b])
        if ctx == 0:
            continue
        k, v = gather_seq_kv(pool, page_table[b], ctx)
        k, v = k.float(), v.float()
        vs = None if fog_vscale is None else (fog_vscale if fog_vscale.dim() == 1 else fog_vscale[b])[:ctx].float()
        bs = None if fog_bias is None else (fog_bias if fog_bias.dim() == 1 else fog_bias[b])[:ctx].float()
        qg = q[b].float().reshape(hkv, g, 1, d)
        o = _attend_rows(qg, k, v, torch.tensor([ctx - 1]), True, window, sm_scale, vs, bs)
        out[b] = o.reshape(hq, d)
    return out


def paged_prefill_ref(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor,
                      ctx_lens: torch.Tensor, fog_vscale: Optional[torch.Tensor] = None,
                      fog_bias: Optional[torch.Tensor] = None, window: int = 0, causal: bool = True,
                      sm_scale: Optional[float] = None, rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Chunked prefill over paged KV (CPU, fp32).  q [B, C, Hq, D]; query i at ctx-C+i.

    ``rows`` optionally restricts the evaluation to those chunk rows (sampled
    parity at large contexts).  Returns fp32 [B, C or len(rows), Hq, D].
    """
    b_, c, hq, d = q.shape
    hkv = pool.shape[3]
    g = hq // hkv
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    sel = torch.arange(c) if rows is None else rows.long()
    out = torch.zeros(b_, len(sel), hq, d, dtype=torch.float32)
    for b in range(b_):
        ctx = int(ctx_lens[b])
        k, v = gather_seq_kv(pool, page_table[b], ctx)
        k, v = k.float(), v.float()
        vs = None if fog_vscale is None else (fog_vscale if fog_vscale.dim() == 1 else fog_vscale[b])[:ctx].float()
        bs = None if fog_bias is None else (fog_bias if fog_bias.dim() == 1 else fog_bias[b])[:ctx].float()
        qpos = ctx - c + sel
        qg = q[b, sel].float().permute(1, 0, 2).reshape(hkv, g, len(sel), d)
        o = _attend_rows(qg, k, v, qpos, causal, window, sm_scale, vs, bs)  # [Hkv, G, R, D]
        out[b] = o.reshape(hq, len(sel), d).permute(1, 0, 2)
    return out


def paged_prefill_blockwise(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor,
                            ctx_lens: torch.Tensor, rows: torch.Tensor,
                            fog_vscale: Optional[torch.Tensor] = None, window: int = 0, causal: bool = True,
                            sm_scale: Optional[float] = None, block_pages: int = 512,
                            kv_head: Optional[int] = None, q_heads: Optional[Sequence[int]] = None) -> torch.Tensor:
    """paged_prefill_ref for selected chunk rows, blockwise with an online
    softmax so a million-token context fits in CPU memory.  ``pool`` may live
    on the GPU: each block of pages is gathered there and copied over.
    q [B, C, Hq, D] (CPU); returns fp32 [B, len(rows), Hq, D].  With
    ``kv_head`` only that kv head's query heads are computed (or the subset
    ``q_heads`` of them, heads numbered within the group); the other heads of
    the result stay zero."""
    b_, c, hq, d = q.shape
    p = pool.shape[1]
    hkv_all = pool.shape[3]
    g_all = hq // hkv_all
    kvs = list(range(hkv_all)) if kv_head is None else [int(kv_head)]
    sub = list(range(g_all)) if q_heads is None else [int(x) for x in q_heads]
    hkv, g = len(kvs), len(sub)
    heads = torch.tensor([kh * g_all + x for kh in kvs for x in sub])  # computed q heads, (kv head, sub) order
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    rows = rows.long()
    r = len(rows)
    out = torch.zeros(b_, r, hq, d, dtype=torch.float32)
    for b in range(b_):
        ctx = int(ctx_lens[b])
        qpos = ctx - c + rows                                          # [R]
        qg = q[b][rows][:, heads].float().view(r, hkv, g, d).permute(1, 2, 0, 3).reshape(hkv, g * r, d)
        pos_col = qpos.repeat(g)                                       # column (g, r) -> qpos[r]
        m = torch.full((hkv, g * r), float("-inf"))
        l = torch.zeros(hkv, g * r)
        acc = torch.zeros(hkv, g * r, d)
        hi = ctx if not causal else min(ctx, int(qpos.max()) + 1)
        lo = 0 if window <= 0 else max(0, int(qpos.min()) - window + 1)
        n_pages = (hi + p - 1) // p
        for p0 in range(lo // p, n_pages, block_pages):
            p1 = min(n_pages, p0 + block_pages)
            kv = pool[page_table[b, p0:p1].long().to(pool.device)][:, :, :, kvs].cpu()
            kv = kv.reshape((p1 - p0) * p, 2, hkv, d).float()
            t0 = p0 * p
            t1 = min(hi, p1 * p)
            kb = kv[: t1 - t0, 0].permute(1, 2, 0)                    # [Hkv, D, n]
            vb = kv[: t1 - t0, 1]
            if fog_vscale is not None:
                vs = (fog_vscale if fog_vscale.dim() == 1 else fog_vscale[b])[t0:t1].float().cpu()
                vb = vb * vs[:, None, None]
            s = torch.bmm(qg, kb) * sm_scale                          # [Hkv, G*R, n]
            j = torch.arange(t0, t1)
            dist = pos_col[:, None] - j[None, :]
            keep = torch.ones_like(dist, dtype=torch.bool)
            if causal:
                keep &= dist >= 0
            if window > 0:
                keep &= (dist >= 0) & (dist < window)
            s = s.masked_fill(~keep[None], float("-inf"))
            m_new = torch.maximum(m, s.amax(-1))
            m_safe = torch.where(torch.isinf(m_new), torch.zeros_like(m_new), m_new)
            corr = torch.where(torch.isinf(m), torch.zeros_like(m), torch.exp(m - m_safe))
            pexp = torch.exp(s - m_safe[..., None])
            l = l * corr + pexp.sum(-1)
            acc = acc * corr[..., None] + torch.bmm(pexp, vb.permute(1, 0, 2).contiguous())
            m = m_new
        o = acc / l[..., None]                                         # [Hkv, G*R, D]
        out[b][:, heads] = o.view(hkv, g, r, d).permute(2, 0, 1, 3).reshape(r, hkv * g, d)
    return out


def paged_decode_blockwise(q: torch.Tensor, pool: torch.Tensor, page_table: torch.Tensor,
                           ctx_lens: torch.Tensor, fog_vscale: Optional[torch.Tensor] = None,
                           window: int = 0, sm_scale: Optional[float] = None,
                           block_pages: int = 512) -> torch.Tensor:
    """Same result as paged_decode_ref, evaluated blockwise with an online
    softmax so that 128K-token contexts fit in CPU memory (the CPU baseline's
    timed path).  V-mode fog only."""
    b_, hq, d = q.shape
    p = pool.shape[1]
    hkv = pool.shape[3]
    g = hq // hkv
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    out = torch.zeros(b_, hq, d, dtype=torch.float32)
    for b in range(b_):
        ctx = int(ctx_lens[b])
        lo = 0 if window <= 0 else max(0, ctx - window)
        qg = q[b].float().reshape(hkv, g, d)
        m = torch.full((hkv, g), float("-inf"))
        l = torch.zeros(hkv, g)
        acc = torch.zeros(hkv, g, d)
        n_pages = (ctx + p - 1) // p
        for p0 in range(lo // p, n_pages, block_pages):
            p1 = min(n_pages, p0 + block_pages)
            kv = pool[page_table[b, p0:p1].long()].reshape((p1 - p0) * p, 2, hkv, d).float()
            t0 = p0 * p
            t1 = min(ctx, p1 * p)
            a = max(lo, t0)
            kb = kv[a - t0:t1 - t0, 0].permute(1, 2, 0)          # [Hkv, D, n]
            vb = kv[a - t0:t1 - t0, 1]
            if fog_vscale is not None:
                vs = (fog_vscale if fog_vscale.dim() == 1 else fog_vscale[b])[a:t1].float()
                vb = vb * vs[:, None, None]
            s = torch.bmm(qg, kb) * sm_scale                     # [Hkv, G, n]
            m_new = torch.maximum(m, s.amax(-1))
            corr = torch.exp(m - m_new)
            pexp = torch.exp(s - m_new[..., None])
            l = l * corr + pexp.sum(-1)
            acc = acc * corr[..., None] + torch.bmm(pexp, vb.permute(1, 0, 2).contiguous())
            m = m_new
        out[b] = (acc / l[..., None]).reshape(hq, d)
    return out
