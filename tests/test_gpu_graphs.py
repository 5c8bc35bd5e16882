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


def test_graph_decode_lengths_change_between_replays(dev):
    """A serving loop's decode graph: captured once for a batch of 16 with a
    host bound on the context, replayed while the sequence lengths change on
    the device (uniform, ragged, spread, empty sequences).  The split
    workgroups are dealt out from the lengths the kernels read at run time,
    so each replay equals an eager call on the same lengths bit for bit, and
    the ragged replay matches the oracle."""
    from oracle.attention import paged_decode_blockwise

    from kessie_amd import ops

    b, max_ctx = 16, 8192
    q, pool, table, lens = decode_case(b, 32, 8, 128, max_ctx, 16, torch.bfloat16, dev, seed=13)
    vs = torch.rand(max_ctx, generator=torch.Generator(device=dev).manual_seed(14), device=dev)
    out = torch.empty_like(q)
    g = _capture(lambda: ops.fog_decode(q, pool, table, lens, max_ctx=max_ctx, fog_vscale=vs, out=out))
    schedules = {
        "uniform": [max_ctx] * b,
        "ragged": [max_ctx, max_ctx] + [512] * 14,
        "spread": [512 * (i + 1) for i in range(b)],
        "empty": [0, max_ctx, 0, 1, 17, 0, 4096, 0] * 2,
    }
    for name, new_lens in schedules.items():
        lens.copy_(torch.tensor(new_lens, dtype=torch.int32))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = ops.fog_decode(q, pool, table, lens, max_ctx=max_ctx, fog_vscale=vs)
        torch.cuda.synchronize()
        assert torch.equal(got, want), name
        if name == "ragged":
            for i in (0, 1, 2, 15):
                sub_pool = pool[table[i].long()].cpu()
                sub_table = torch.arange(table.shape[1], dtype=torch.int32).view(1, -1)
                ref = paged_decode_blockwise(q[i:i + 1].cpu(), sub_pool, sub_table, lens[i:i + 1].cpu(), vs.cpu())
                diff = (got[i:i + 1].float().cpu() - ref).abs()
                assert (diff <= 2e-2 + 1e-2 * ref.abs()).all(), (name, i, diff.max().item())
        if name == "empty":
            assert not got[torch.tensor(new_lens, device=dev) == 0].any()


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


def test_graph_evict_compact_fused(dev):
    """The fused evict + compact call (clear + one grid-barrier launch)
    captured with the gather and replayed; each replay equals the eager
    two-call pipeline (select_evict, compact) bit for bit."""
    from kessie_amd import ops

    num_pages, s, w = 20000, 16, 1000
    pool = paged_pool(num_pages, 16, 2, 64, torch.bfloat16, dev, seed=15)
    tables = randperm(num_pages, dev, 16)[: s * w].view(s, w).contiguous()
    lens = torch.randint(0, w + 1, (s,), generator=torch.Generator(device=dev).manual_seed(17), device=dev,
                         dtype=torch.int32)
    scores = torch.empty(num_pages, device=dev)
    valid = torch.ones(num_pages, dtype=torch.int8, device=dev)
    bufs = dict(evict_list=torch.empty(num_pages, dtype=torch.int32, device=dev),
                evict_count=torch.zeros(1, dtype=torch.int32, device=dev), new_tables=torch.empty_like(tables),
                new_lens=torch.empty(s, dtype=torch.int32, device=dev),
                gather_idx=torch.empty(s * w, dtype=torch.int32, device=dev),
                gather_count=torch.zeros(1, dtype=torch.int32, device=dev))
    out = torch.empty((s * w,) + tuple(pool.shape[1:]), dtype=pool.dtype, device=dev)

    def pipeline():
        ops.page_evict_compact(scores, valid, tables, lens, -1, 0.3, **bufs)
        ops.page_gather(pool, bufs["gather_idx"], bufs["gather_count"], out=out, n=s * w)

    scores.copy_(torch.rand(num_pages, generator=torch.Generator(device=dev).manual_seed(18), device=dev))
    g = _capture(pipeline)
    for i in range(3):
        scores.copy_(torch.rand(num_pages, generator=torch.Generator(device=dev).manual_seed(50 + i), device=dev))
        if i == 1:
            scores[::2] = 0.25  # heavy ties at the threshold
        valid.fill_(1)
        valid[::7] = 0
        v0 = valid.clone()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        c, n = int(bufs["evict_count"].item()), int(bufs["gather_count"].item())
        got = (bufs["evict_list"][:c].clone(), valid.clone(), bufs["new_tables"].clone(), bufs["new_lens"].clone(),
               bufs["gather_idx"][:n].clone(), out[:n].clone())
        valid.copy_(v0)
        lst, cnt = ops.page_select_evict(scores, valid, -1, 0.3)
        nt, nl, gi, gc = ops.page_compact(tables, lens, valid)
        ref_out = ops.page_gather(pool, gi, gc, n=s * w)
        torch.cuda.synchronize()
        assert c == int(cnt.item()) and n == int(gc.item()), f"replay {i}"
        want = (lst[:c], valid, nt, nl, gi[:n], ref_out[:n])
        for a, b in zip(got, want):
            assert torch.equal(a, b), f"replay {i}"


def test_graph_survives_workspace_growth(dev):
    """A captured decode keeps writing its split partials to the cached
    workspace it was captured with.  A later, larger eager call replaces the
    cached buffer; the superseded one must stay allocated, so a tensor
    allocated afterwards is never overwritten by a replay."""
    from kessie_amd import ops

    ctx = 3000
    q, pool, table, lens = decode_case(2, 32, 8, 128, ctx, 16, torch.bfloat16, dev, seed=21)
    out = torch.empty_like(q)
    g = _capture(lambda: ops.fog_decode(q, pool, table, lens, max_ctx=ctx, out=out))
    old = ops.workspace(1, dev, "attn")  # the buffer the graph was captured with
    # A larger call (here: a request one byte past the cached size, as a split
    # prefill's larger workspace would make) replaces the cached buffer.
    ops.workspace(old.numel() + 1, dev, "attn")
    torch.cuda.synchronize()
    assert ops.workspace(1, dev, "attn").data_ptr() != old.data_ptr(), "the workspace did not grow"
    n_old = old.numel()
    del old
    sentinels = [torch.full((n_old,), 0x5A, dtype=torch.uint8, device=dev) for _ in range(4)]
    torch.cuda.synchronize()
    for i in range(2):
        q.copy_(randn(q.shape, torch.bfloat16, dev, 400 + i))
        g.replay()
        torch.cuda.synchronize()
        for t in sentinels:
            assert bool((t == 0x5A).all()), f"replay {i} overwrote a tensor allocated after the growth"
        want = ops.fog_decode(q, pool, table, lens, max_ctx=ctx)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
