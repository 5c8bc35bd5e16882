"""Seeded synthetic inputs shared by the parity tests and bench.py.

Large tensors are generated on the device with torch.Generator(device).manual_seed(s),
in a fixed order per workload; the CPU oracle receives copies.
"""
from __future__ import annotations

import torch


def gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def randn(shape, dtype, device, seed):
    return torch.randn(shape, generator=gen(device, seed), device=device, dtype=torch.float32).to(dtype)


def randperm(n, device, seed):
    return torch.randperm(n, generator=gen(device, seed), device=device).to(torch.int32)


def paged_pool(num_pages, page_size, hkv, d, dtype, device, seed=0):
    """Native pool [pages, P, 2, Hkv, D] with N(0,1) entries."""
    return randn((num_pages, page_size, 2, hkv, d), dtype, device, seed)


def decode_case(b, hq, hkv, d, ctx, page_size, dtype, device, seed=0, extra_pages=0, ctx_lens=None):
    """q [B,Hq,D], pool, page_table [B, W] (random permutation of pool pages), ctx_lens."""
    pages_per_seq = (ctx + page_size - 1) // page_size
    num_pages = b * pages_per_seq + extra_pages
    q = randn((b, hq, d), dtype, device, seed + 100)
    pool = paged_pool(num_pages, page_size, hkv, d, dtype, device, seed)
    perm = randperm(num_pages, device, seed + 1)[: b * pages_per_seq]
    table = perm.view(b, pages_per_seq).contiguous()
    if ctx_lens is None:
        ctx_lens = [ctx] * b
    lens = torch.tensor(ctx_lens, dtype=torch.int32, device=device)
    return q, pool, table, lens
