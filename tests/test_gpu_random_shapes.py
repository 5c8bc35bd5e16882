"""GPU parity over seeded random shapes: decode, chunked prefill and varlen
prefill with random batch, ragged contexts (including empty ones), chunk
lengths, GQA ratio, window, fog mode (none / V-scale per batch / bias / both),
dtype and key split count, each case against the CPU oracle.  The cases are fixed by their seeds (no randomness between
runs).  Tolerance |gpu - ref| <= 2e-2 + 1e-2*|ref|."""
import random

import pytest
import torch

from oracle.attention import paged_decode_ref, paged_prefill_ref
from tests.inputs import gen, paged_pool, randperm

pytestmark = pytest.mark.gpu

GQA = [(32, 8), (16, 8), (8, 8), (64, 8), (8, 1), (12, 3), (32, 4), (16, 1)]


def _check(got, ref):
    g = got.float().cpu()
    diff = (g - ref).abs()
    bad = diff > 2e-2 + 1e-2 * ref.abs()
    assert not bad.any(), f"{int(bad.sum())}/{bad.numel()} outside tol, max diff {diff.max().item():.3e}"


def _page_size(seed):
    """16, 32 or 64-token pages, drawn apart from the other shape choices so
    that a seed's other draws do not depend on it."""
    return random.Random(5000 + seed).choice([16, 16, 32, 64])


def _setup(dev, rng, b, ctxs, hkv, dtype, seed, p=16):
    pages = [max(1, -(-c // p)) for c in ctxs]
    w = max(pages)
    num_pages = sum(pages) + rng.randint(0, 5)
    pool = paged_pool(num_pages, p, hkv, 128, dtype, dev, seed)
    perm = randperm(num_pages, dev, seed + 1)
    table = torch.full((b, w), -1, dtype=torch.int32, device=dev)
    at = 0
    for i, n in enumerate(pages):
        table[i, :n] = perm[at:at + n]
        at += n
    return pool, table, torch.tensor(ctxs, dtype=torch.int32, device=dev)


def _fog(dev, rng, b, mx, seed):
    mode = rng.choice(["none", "vscale", "bias", "both"])
    vs = torch.rand(b, mx, generator=gen(dev, seed + 7), device=dev) if mode in ("vscale", "both") else None
    bias = (torch.randn(mx, generator=gen(dev, seed + 8), device=dev) * 0.3) if mode in ("bias", "both") else None
    return mode, vs, bias


@pytest.mark.parametrize("seed", range(12))
def test_random_decode(dev, seed):
    from kessie_amd import ops

    rng = random.Random(1000 + seed)
    b = rng.randint(1, 6)
    hq, hkv = rng.choice(GQA)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    ctxs = [rng.choice([0, 1, 15, 16, 17, rng.randint(2, 3000)]) for _ in range(b)]
    mx = max(max(ctxs), 1)
    window = rng.choice([0, 0, 1, 16, rng.randint(2, 2000)])
    pool, table, lens = _setup(dev, rng, b, ctxs, hkv, dtype, seed, _page_size(seed))
    mode, vs, bias = _fog(dev, rng, b, mx, seed)
    q = torch.randn(b, hq, 128, generator=gen(dev, seed + 9), device=dev).to(dtype)
    out = ops.fog_decode(q, pool, table, lens, max_ctx=mx, fog_vscale=vs, fog_bias=bias, window=window)
    torch.cuda.synchronize()
    ref = paged_decode_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), None if vs is None else vs.cpu(),
                           None if bias is None else bias.cpu(), window)
    _check(out, ref)


@pytest.mark.parametrize("seed", range(12))
def test_random_prefill(dev, seed):
    from kessie_amd import ops

    rng = random.Random(2000 + seed)
    b = rng.randint(1, 4)
    hq, hkv = rng.choice(GQA)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    c = rng.choice([1, 2, 17, 64, 65, rng.randint(3, 400)])
    ctxs = [c + rng.choice([0, 1, 16, rng.randint(2, 2500)]) for _ in range(b)]
    mx = max(ctxs)
    window = rng.choice([0, 0, 1, 33, rng.randint(2, 1500)])
    causal = rng.random() < 0.85
    pool, table, lens = _setup(dev, rng, b, ctxs, hkv, dtype, seed, _page_size(seed))
    mode, vs, bias = _fog(dev, rng, b, mx, seed)
    q = torch.randn(b, c, hq, 128, generator=gen(dev, seed + 9), device=dev).to(dtype)
    out = ops.fog_prefill(q, pool, table, lens, mx, fog_vscale=vs, fog_bias=bias, window=window, causal=causal)
    torch.cuda.synchronize()
    for i in range(b):
        ref = paged_prefill_ref(q[i:i + 1].cpu(), pool.cpu(), table[i:i + 1].cpu(), lens[i:i + 1].cpu(),
                                None if vs is None else vs[i].cpu(), None if bias is None else bias.cpu(), window,
                                causal=causal)
        _check(out[i:i + 1], ref)


@pytest.mark.parametrize("seed", range(10))
def test_random_varlen(dev, seed, monkeypatch):
    from kessie_amd import ops

    rng = random.Random(3000 + seed)
    b = rng.randint(1, 8)
    hq, hkv = rng.choice(GQA)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    chunks = [rng.choice([0, 1, 16, 63, 64, 65, rng.randint(2, 300)]) for _ in range(b)]
    if not any(chunks):
        chunks[0] = 5
    ctxs = [c + rng.choice([0, 1, rng.randint(2, 3000)]) for c in chunks]
    ctxs = [max(x, 1) for x in ctxs]
    mx = max(ctxs)
    window = rng.choice([0, 0, 1, rng.randint(2, 1500)])
    splits = rng.choice([None, 1, 3, 8])
    if splits:
        monkeypatch.setenv("KESSIE_PREFILL_SPLITS", str(splits))
    pool, table, lens = _setup(dev, rng, b, ctxs, hkv, dtype, seed)
    mode, vs, bias = _fog(dev, rng, b, mx, seed)
    off = rng.randint(0, 7)
    starts = [off]
    for c in chunks:
        starts.append(starts[-1] + c)
    qsl = torch.tensor(starts, dtype=torch.int32, device=dev)
    q_all = torch.randn(starts[-1], hq, 128, generator=gen(dev, seed + 9), device=dev).to(dtype)
    q = q_all[off:]
    out = torch.full_like(q, float("nan"))
    assert ops.fog_prefill_varlen(q, qsl, max(chunks), pool, table, lens, mx, fog_vscale=vs, fog_bias=bias,
                                  window=window, out=out)
    torch.cuda.synchronize()
    for i, c in enumerate(chunks):
        if c == 0:
            continue
        s = starts[i] - off
        ref = paged_prefill_ref(q[s:s + c].unsqueeze(0).cpu(), pool.cpu(), table[i:i + 1].cpu(),
                                lens[i:i + 1].cpu(), None if vs is None else vs[i].cpu(),
                                None if bias is None else bias.cpu(), window)
        _check(out[s:s + c].unsqueeze(0), ref)
    assert not torch.isnan(out).any()
