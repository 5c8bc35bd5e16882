"""HIP graph capture of the hot path: fog decode (partials + combine), the
score-evict -> compact -> gather pipeline and the paged RoPE remap are each
captured once and replayed several times, with eager work (new inputs, resets)
and synchronisations between the replays.  Every replay must equal an eager run
on the same inputs bit for bit: the kernels are deterministic, take no host
round trip, and clear their own scratch with fill kernels (no memset nodes)."""
import pytest
import torch

from tests.inputs import decode_case, paged_pool, randn, randperm

pytestmark = pytest.mark.gpu


def _capture(fn):
    fn()  # warm-up outside the capture: workspaces, cached tables, LDS attributes
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def test_graph_decode(dev):
    from kessie_amd import ops

    ctx = 3000
    q, pool, table, lens = decode_case(2, 32, 8, 128, ctx, 16, torch.bfloat16, dev, seed=3)
    vs = torch.rand(ctx, generator=torch.Generator(device=dev).manual_seed(4), device=dev)
    out = torch.empty_like(q)
    g = _capture(lambda: ops.fog_decode(q, pool, table, lens, max_ctx=ctx, fog_vscale=vs, out=out))
    for i in range(3):
        q.copy_(randn(q.shape, torch.bfloat16, dev, 100 + i))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = ops.fog_decode(q, pool, table, lens, max_ctx=ctx, fog_vscale=vs)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"


def test_graph_evict_pipeline(dev):
    from kessie_amd import ops

    num_pages, s, w = 4096, 8, 512
    pool = paged_pool(num_pages, 16, 2, 64, torch.bfloat16, dev, seed=5)
    tables = randperm(num_pages, dev, 6).view(s, w).contiguous()
    lens = torch.full((s,), w, dtype=torch.int32, device=dev)
    scores = torch.empty(num_pages, device=dev)
    valid = torch.ones(num_pages, dtype=torch.int8, device=dev)
    ev_list = torch.empty(num_pages, dtype=torch.int32, device=dev)
    ev_cnt = torch.zeros(1, dtype=torch.int32, device=dev)
    nt, nl = torch.empty_like(tables), torch.empty(s, dtype=torch.int32, device=dev)
    gi, gc = torch.empty(s * w, dtype=torch.int32, device=dev), torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.empty((s * w,) + tuple(pool.shape[1:]), dtype=pool.dtype, device=dev)

    def pipeline():
        ops.page_select_evict(scores, valid, -1, 0.25, ev_list, ev_cnt)
        ops.page_compact(tables, lens, valid, nt, nl, gi, gc)
        ops.page_gather(pool, gi, gc, out=out, n=s * w)

    def snapshot():
        c, n = int(ev_cnt.item()), int(gc.item())
        return c, ev_list[:c].clone(), nt.clone(), nl.clone(), gi[:n].clone(), out[:n].clone()

    scores.copy_(torch.rand(num_pages, generator=torch.Generator(device=dev).manual_seed(7), device=dev))
    g = _capture(pipeline)
    for i in range(3):
        gen = torch.Generator(device=dev).manual_seed(20 + i)
        scores.copy_(torch.rand(num_pages, generator=gen, device=dev))
        if i == 2:
            scores[::3] = 0.5  # heavy ties
        valid.fill_(1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = snapshot()
        valid.fill_(1)
        pipeline()
        torch.cuda.synchronize()
        want = snapshot()
        assert got[0] == want[0] == num_pages // 4, f"replay {i}"
        for a, b in zip(got[1:], want[1:]):
            assert torch.equal(a, b), f"replay {i}"


def test_graph_remap(dev):
    from kessie_amd import ops

    n_tok, hkv, d = 2048, 8, 128
    pool = torch.empty(256, 16, 2, hkv, d, dtype=torch.bfloat16, device=dev)
    plist = randperm(256, dev, 8)[: n_tok // 16].contiguous()
    orig = torch.randint(0, 1_000_000, (n_tok,), generator=torch.Generator(device=dev).manual_seed(9), device=dev,
                         dtype=torch.int32)
    tgt = torch.arange(n_tok, dtype=torch.int32, device=dev)
    pool.copy_(randn(pool.shape, torch.bfloat16, dev, 10))
    g = _capture(lambda: ops.rope_remap_paged(pool, orig, tgt, 500000.0, page_list=plist))
    for i in range(3):
        src = randn(pool.shape, torch.bfloat16, dev, 30 + i)
        pool.copy_(src)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = src.clone()
        ops.rope_remap_paged(ref, orig, tgt, 500000.0, page_list=plist)
        torch.cuda.synchronize()
        assert torch.equal(pool, ref), f"replay {i}"


def test_graph_prefill_split(dev):
    """A small chunk on a long context (key range split, partials + combine)
    captured once and replayed with new queries."""
    from kessie_amd import ops

    ctx, c = 20000, 128
    q, pool, table, lens = decode_case(1, 32, 8, 128, ctx, 16, torch.bfloat16, dev, seed=11)
    q = randn((1, c, 32, 128), torch.bfloat16, dev, 12)
    vs = torch.rand(ctx, generator=torch.Generator(device=dev).manual_seed(13), device=dev)
    out = torch.empty_like(q)
    g = _capture(lambda: ops.fog_prefill(q, pool, table, lens, ctx, fog_vscale=vs, out=out))
    for i in range(3):
        q.copy_(randn(q.shape, torch.bfloat16, dev, 200 + i))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = ops.fog_prefill(q, pool, table, lens, ctx, fog_vscale=vs)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"


def test_graph_prefill_varlen_split(dev, monkeypatch):
    """The serving path's prefill launch (varlen, key range split in two,
    partials + combine) captured once and replayed with new queries."""
    from kessie_amd import ops

    monkeypatch.setenv("KESSIE_PREFILL_SPLITS", "2")
    chunks, ctxs = [96, 1, 200], [5000, 3000, 7000]
    pages = [(c + 15) // 16 for c in ctxs]
    pool = paged_pool(sum(pages) + 4, 16, 8, 128, torch.bfloat16, dev, seed=41)
    perm = randperm(sum(pages) + 4, dev, 42)
    table = torch.full((3, max(pages)), -1, dtype=torch.int32, device=dev)
    at = 0
    for i, n in enumerate(pages):
        table[i, :n] = perm[at:at + n]
        at += n
    lens = torch.tensor(ctxs, dtype=torch.int32, device=dev)
    qsl = torch.tensor([0, 96, 97, 297], dtype=torch.int32, device=dev)
    q = randn((297, 32, 128), torch.bfloat16, dev, 43)
    bias = torch.randn(max(ctxs), generator=torch.Generator(device=dev).manual_seed(44), device=dev) * 0.1
    out = torch.empty_like(q)
    g = _capture(lambda: ops.fog_prefill_varlen(q, qsl, 200, pool, table, lens, max(ctxs), fog_bias=bias, out=out))
    for i in range(3):
        q.copy_(randn(q.shape, torch.bfloat16, dev, 300 + i))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = torch.empty_like(q)
        ops.fog_prefill_varlen(q, qsl, 200, pool, table, lens, max(ctxs), fog_bias=bias, out=want)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"
