"""GPU parity: chunked-prefill fog attention (MFMA kernel and the generic
kernel) vs the CPU oracle.  bf16/fp16: |gpu - ref| <= 2e-2 + 1e-2*|ref|;
fp32 (fp32 MFMA kernel for head_dim 128, else the generic kernel): 1e-5."""
import pytest
import torch

from oracle.attention import paged_prefill_blockwise, paged_prefill_ref
from oracle.fog import build_fog_weights, fog_bias
from tests.inputs import gen, paged_pool, randperm

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-2, 1e-2), torch.float32: (1e-5, 1e-5)}


def _check(got, ref, dtype):
    atol, rtol = TOL[dtype]
    g = got.float().cpu()
    diff = (g - ref).abs()
    bad = diff > atol + rtol * ref.abs()
    assert not bad.any(), f"{int(bad.sum())}/{bad.numel()} outside tol, max diff {diff.max().item():.3e}"


def _case(dev, b, c, ctxs, hq, hkv, dtype, seed=0, page_size=16):
    p, d = page_size, 128
    pages_per = max((x + p - 1) // p for x in ctxs)
    num_pages = b * pages_per + 3
    pool = paged_pool(num_pages, p, hkv, d, dtype, dev, seed)
    table = randperm(num_pages, dev, seed + 1)[: b * pages_per].view(b, pages_per).contiguous()
    q = torch.randn(b, c, hq, d, generator=gen(dev, seed + 2), device=dev).to(dtype)
    lens = torch.tensor(ctxs, dtype=torch.int32, device=dev)
    return q, pool, table, lens


@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (16, 8), (64, 8), (8, 1), (12, 3), (32, 4),
                                     (16, 1), (128, 8)])
def test_prefill_bf16_gqa(dev, hq, hkv):
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 2, 100, [1000, 777], hq, hkv, torch.bfloat16)
    fog = build_fog_weights(1000).to(dev)
    out = ops.fog_prefill(q, pool, table, lens, 1000, fog_vscale=fog)
    torch.cuda.synchronize()
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), fog.cpu())
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("c,ctx", [(1, 1), (1, 64), (17, 17), (64, 200), (300, 300), (129, 4000)])
def test_prefill_chunk_shapes(dev, c, ctx):
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 1, c, [ctx], 32, 8, torch.bfloat16, seed=c)
    out = ops.fog_prefill(q, pool, table, lens, ctx)
    torch.cuda.synchronize()
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu())
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("dtype,c", [(torch.bfloat16, 1024), (torch.bfloat16, 1536), (torch.float32, 128),
                                     (torch.float32, 256)])
def test_prefill_fresh_prompts_at_the_split_rule_edges(dev, dtype, c):
    """Fresh prompts (chunk = context, causal, V-fog) where the automatic key
    split count turns on what is counted: bf16 prompts of 1,024 and 1,536
    tokens stay unsplit because a causal query tile sees half the context on
    average, fp32 prompts of 128 and 256 tokens split 2 and 4 ways at four key
    blocks per split; each against the oracle."""
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 1, c, [c], 32, 8, dtype, seed=c + 7)
    fog = build_fog_weights(c).to(dev)
    out = ops.fog_prefill(q, pool, table, lens, c, fog_vscale=fog)
    torch.cuda.synchronize()
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), fog.cpu())
    _check(out, ref, dtype)


@pytest.mark.parametrize("window", [1, 16, 37, 100, 10000])
def test_prefill_window(dev, window):
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 1, 90, [700], 32, 8, torch.bfloat16, seed=5)
    out = ops.fog_prefill(q, pool, table, lens, 700, window=window)
    torch.cuda.synchronize()
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), window=window)
    _check(out, ref, torch.bfloat16)


def test_prefill_bias_and_fp16(dev):
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 2, 70, [500, 333], 32, 8, torch.float16, seed=6)
    bias = fog_bias(500, 0.5, 0.5, {3, 99, 498}, 0.1).to(dev)
    out = ops.fog_prefill(q, pool, table, lens, 500, fog_bias=bias)
    torch.cuda.synchronize()
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), None, bias.cpu())
    _check(out, ref, torch.float16)


def test_prefill_non_causal_and_bad_pages(dev):
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 1, 40, [400], 32, 8, torch.bfloat16, seed=7)
    table[0, 3] = -1
    out = ops.fog_prefill(q, pool, table, lens, 400, causal=False)
    torch.cuda.synchronize()
    keep = [i for i in range(table.shape[1]) if i != 3]
    pool_c = pool.cpu()
    # Oracle: the same context without logical page 3 (non-causal, so only membership matters).
    t2 = table.cpu()[:, keep].contiguous()
    ref = paged_prefill_ref(q.cpu(), pool_c, t2, torch.tensor([400 - 16]), causal=False)
    _check(out, ref, torch.bfloat16)


def test_prefill_fp32_generic(dev):
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 1, 33, [300], 32, 8, torch.float32, seed=8)
    fog = build_fog_weights(300).to(dev)
    out = ops.fog_prefill(q, pool, table, lens, 300, fog_vscale=fog)
    torch.cuda.synchronize()
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), fog.cpu())
    _check(out, ref, torch.float32)


@pytest.mark.parametrize("page_size,dtype,fog,window", [(32, torch.bfloat16, "vscale", 0),
                                                         (64, torch.float16, "bias", 37),
                                                         (128, torch.bfloat16, "vscale", 0)])
def test_prefill_larger_pages(dev, page_size, dtype, fog, window):
    """Pages of 32, 64 and 128 tokens on the MFMA kernel (read as 16-token
    blocks), ragged contexts: against the oracle."""
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 2, 100, [1000, 777], 32, 8, dtype, seed=31, page_size=page_size)
    vs = build_fog_weights(1000).to(dev) if fog == "vscale" else None
    bias = fog_bias(1000, 0.5, 0.5, {3, 500}, 0.1).to(dev) if fog == "bias" else None
    out = ops.fog_prefill(q, pool, table, lens, 1000, fog_vscale=vs, fog_bias=bias, window=window)
    torch.cuda.synchronize()
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), None if vs is None else vs.cpu(),
                            None if bias is None else bias.cpu(), window)
    _check(out, ref, dtype)


def test_prefill_larger_pages_bad_page(dev):
    """An invalid page id in a table of 32-token pages masks all 32 of its
    tokens: non-causal, so the oracle is the same context without that page."""
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 1, 40, [400], 32, 8, torch.bfloat16, seed=7, page_size=32)
    table[0, 3] = -1
    out = ops.fog_prefill(q, pool, table, lens, 400, causal=False)
    torch.cuda.synchronize()
    keep = [i for i in range(table.shape[1]) if i != 3]
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu()[:, keep].contiguous(), torch.tensor([400 - 32]),
                            causal=False)
    _check(out, ref, torch.bfloat16)


def test_prefill_larger_pages_varlen_and_split(dev, monkeypatch):
    """32-token pages: the varlen entry takes them (it launches only on the
    MFMA kernel) and matches per-sequence launches bit for bit at a forced key
    split, and both match the oracle."""
    from kessie_amd import ops

    p, c = 32, 64
    ctxs = [3000, 1500]
    _, pool, table, lens = _case(dev, 2, 1, ctxs, 32, 8, torch.bfloat16, seed=33, page_size=p)
    chunks = [c, 40]
    qsl = torch.tensor([0, chunks[0], chunks[0] + chunks[1]], dtype=torch.int32, device=dev)
    q = torch.randn(sum(chunks), 32, 128, generator=gen(dev, 34), device=dev).bfloat16()
    monkeypatch.setenv("KESSIE_PREFILL_SPLITS", "3")
    out = torch.zeros_like(q)
    assert ops.fog_prefill_varlen(q, qsl, c, pool, table, lens, max(ctxs), out=out)
    torch.cuda.synchronize()
    for i in range(2):
        qi = q[qsl[i]:qsl[i + 1]].unsqueeze(0).contiguous()
        one = ops.fog_prefill(qi, pool, table[i:i + 1].contiguous(), lens[i:i + 1], ctxs[i])
        torch.cuda.synchronize()
        assert torch.equal(out[qsl[i]:qsl[i + 1]], one[0])
        ref = paged_prefill_ref(qi.cpu(), pool.cpu(), table[i:i + 1].cpu(), lens[i:i + 1].cpu())
        _check(one, ref, torch.bfloat16)


def test_prefill_larger_pages_match_generic(dev, monkeypatch):
    """The MFMA kernel on 64-token pages against the generic kernel on the same
    inputs (the generic one takes any page size)."""
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 2, 150, [2000, 1500], 32, 8, torch.bfloat16, seed=35, page_size=64)
    fog = build_fog_weights(2000).to(dev)
    a = ops.fog_prefill(q, pool, table, lens, 2000, fog_vscale=fog)
    monkeypatch.setenv("KESSIE_FORCE_GENERIC", "1")
    b = ops.fog_prefill(q, pool, table, lens, 2000, fog_vscale=fog)
    torch.cuda.synchronize()
    assert (a.float() - b.float()).abs().max().item() < 2e-2


def test_prefill_mfma_matches_generic(dev, monkeypatch):
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 2, 150, [2000, 1500], 32, 8, torch.bfloat16, seed=9)
    fog = build_fog_weights(2000).to(dev)
    a = ops.fog_prefill(q, pool, table, lens, 2000, fog_vscale=fog)
    monkeypatch.setenv("KESSIE_FORCE_GENERIC", "1")
    b = ops.fog_prefill(q, pool, table, lens, 2000, fog_vscale=fog)
    torch.cuda.synchronize()
    assert (a.float() - b.float()).abs().max().item() < 2e-2


def test_prefill_1m_context_every_query_tile(dev):
    """Config: bf16, 2,048-query chunk appended to a 1,048,576-token paged KV
    (65,664 pages), 32 q / 8 kv heads, D=128, causal, V-fog over the full
    context.  Full-size GPU run; the first and the last query position of each
    of the kernel's 32 query tiles (64 positions x the 4 heads of a kv head per
    tile), all 32 heads, and all 2,048 positions of one head, checked against
    the blockwise oracle."""
    from kessie_amd import ops

    c, L = 2048, 1 << 20
    ctx = L + c
    n_pages = ctx // 16
    pool = paged_pool(n_pages, 16, 8, 128, torch.bfloat16, dev, 0)
    table = randperm(n_pages, dev, 1).view(1, n_pages).contiguous()
    q = torch.randn(1, c, 32, 128, generator=gen(dev, 2), device=dev).bfloat16()
    lens = torch.tensor([ctx], dtype=torch.int32, device=dev)
    fog = build_fog_weights(ctx).to(dev)
    out = ops.fog_prefill(q, pool, table, lens, ctx, fog_vscale=fog)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    rows = torch.tensor(sorted([64 * t for t in range(32)] + [64 * t + 63 for t in range(32)] + [777, 1500]))
    ref = paged_prefill_blockwise(q.cpu(), pool, table.cpu(), lens.cpu(), rows, fog.cpu(), block_pages=4096)
    _check(out[:, rows], ref, torch.bfloat16)
    # Every one of the 2,048 rows of q head 13 (kv head 3, the second head of
    # its group), so each row's causal boundary at 1M context is checked.
    every = torch.arange(c)
    ref13 = paged_prefill_blockwise(q.cpu(), pool, table.cpu(), lens.cpu(), every, fog.cpu(), block_pages=2048,
                                    kv_head=3, q_heads=[1])
    _check(out[:, :, 13:14], ref13[:, :, 13:14], torch.bfloat16)


@pytest.mark.parametrize("fog", ["vscale", "bias", "none"])
@pytest.mark.parametrize("window", [0, 50])
def test_prefill_varlen_matches_per_sequence(dev, fog, window, monkeypatch):
    """One varlen launch over sequences with different chunk lengths (incl. a
    one-token chunk and an empty one) equals the per-sequence launches bit for
    bit, and the oracle within tolerance; the query_start_loc slice may start
    at a non-zero offset.  Both forms are held to one key split
    (KESSIE_PREFILL_SPLITS=1), which makes the summation orders equal."""
    from kessie_amd import ops

    monkeypatch.setenv("KESSIE_PREFILL_SPLITS", "1")

    chunks, ctxs = [37, 1, 300, 0, 129], [900, 64, 300, 50, 4000]
    b, hq, hkv, d = len(chunks), 32, 8, 128
    _, pool, table, lens = _case(dev, b, 1, ctxs, hq, hkv, torch.bfloat16, seed=11)
    starts = [5]
    for c in chunks:
        starts.append(starts[-1] + c)
    qsl = torch.tensor(starts, dtype=torch.int32, device=dev)
    q_all = torch.randn(starts[-1], hq, d, generator=gen(dev, 12), device=dev).to(torch.bfloat16)
    q = q_all[5:]
    mx = max(ctxs)
    vs = bias = None
    if fog == "vscale":
        vs = torch.rand(b, mx, generator=gen(dev, 13), device=dev)
    elif fog == "bias":
        bias = fog_bias(mx, 0.5, 0.5, {3, 17, 200}, 0.1).to(dev)
    out = torch.full_like(q, float("nan"))
    assert ops.fog_prefill_varlen(q, qsl, max(chunks), pool, table, lens, mx, fog_vscale=vs, fog_bias=bias,
                                  window=window, out=out)
    torch.cuda.synchronize()
    for i, c in enumerate(chunks):
        if c == 0:
            continue
        s = starts[i] - 5
        one = ops.fog_prefill(q[s:s + c].unsqueeze(0).contiguous(), pool, table[i:i + 1], lens[i:i + 1], mx,
                              fog_vscale=None if vs is None else vs[i:i + 1], fog_bias=bias, window=window)
        torch.cuda.synchronize()
        assert torch.equal(out[s:s + c], one[0]), f"sequence {i}"
        ref = paged_prefill_ref(q[s:s + c].unsqueeze(0).cpu(), pool.cpu(), table[i:i + 1].cpu(),
                                lens[i:i + 1].cpu(), None if vs is None else vs[i].cpu(),
                                None if bias is None else bias.cpu(), window)
        _check(one, ref, torch.bfloat16)


def test_prefill_varlen_unsupported_shape_launches_nothing(dev):
    """8-token pages: neither MFMA kernel takes them, so the varlen entry
    returns False and leaves the output as it was."""
    from kessie_amd import ops

    _, pool, table, lens = _case(dev, 2, 1, [40, 40], 32, 8, torch.float32, seed=14, page_size=8)
    qsl = torch.tensor([0, 3, 8], dtype=torch.int32, device=dev)
    q = torch.randn(8, 32, 128, device=dev)
    out = torch.full_like(q, 7.0)
    assert not ops.fog_prefill_varlen(q, qsl, 5, pool, table, lens, 40, out=out)
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)


@pytest.mark.parametrize("c,ctx,fog,window,force", [(300, 20000, "vscale", 0, 0), (512, 40000, "bias", 0, 0),
                                                    (64, 9000, "none", 0, 0), (200, 30000, "vscale", 5000, 0),
                                                    (100, 3000, "vscale", 0, 64), (700, 2000, "bias", 300, 5)])
def test_prefill_split_k(dev, c, ctx, fog, window, force, monkeypatch):
    """A small chunk on a long context takes the MFMA kernel's split-K path
    (partials + combine): checked against the blockwise oracle on sampled rows,
    including the chunk's first and last rows.  Forced counts cover splits that
    get no key tile (64 splits of 47 tiles; a window leaves most splits empty)."""
    from kessie_amd import _lib, ops

    if force:
        monkeypatch.setenv("KESSIE_PREFILL_SPLITS", str(force))
    assert _lib.load().kessie_fog_prefill_workspace_bytes(1, c, 32, 8, 128, ctx, 16, 1) > 0
    q, pool, table, lens = _case(dev, 1, c, [ctx], 32, 8, torch.bfloat16, seed=c)
    vs = build_fog_weights(ctx).to(dev) if fog == "vscale" else None
    bias = fog_bias(ctx, 0.5, 0.5, {3, 17, ctx - 2}, 0.1).to(dev) if fog == "bias" else None
    out = ops.fog_prefill(q, pool, table, lens, ctx, fog_vscale=vs, fog_bias=bias, window=window)
    torch.cuda.synchronize()
    rows = torch.unique(torch.tensor([0, 1, c // 3, c // 2, c - 2, c - 1]))
    if bias is None:
        ref = paged_prefill_blockwise(q.cpu(), pool, table, lens.cpu(), rows,
                                      fog_vscale=None if vs is None else vs.cpu(), window=window)
    else:
        ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), None, bias.cpu(), window, rows=rows)
    _check(out[:, rows.long()], ref, torch.bfloat16)


@pytest.mark.parametrize("chunks,ctxs,force", [([200, 150], [30000, 20000], 0),
                                               ([37, 1, 300, 0, 129], [900, 64, 300, 50, 4000], 16)])
def test_prefill_varlen_split_k(dev, chunks, ctxs, force, monkeypatch):
    """Varlen launches that split the key range (two short chunks on long
    contexts: sized split; ragged chunks incl. an empty one: forced 16 splits,
    most of them empty) match the oracle, every packed row written."""
    from kessie_amd import ops

    if force:
        monkeypatch.setenv("KESSIE_PREFILL_SPLITS", str(force))
    b, hq, hkv, d = len(chunks), 32, 8, 128
    _, pool, table, lens = _case(dev, b, 1, ctxs, hq, hkv, torch.bfloat16, seed=21)
    starts = [0]
    for c in chunks:
        starts.append(starts[-1] + c)
    qsl = torch.tensor(starts, dtype=torch.int32, device=dev)
    q = torch.randn(starts[-1], hq, d, generator=gen(dev, 22), device=dev).to(torch.bfloat16)
    mx = max(ctxs)
    vs = torch.rand(b, mx, generator=gen(dev, 23), device=dev)
    out = torch.full_like(q, float("nan"))
    assert ops.fog_prefill_varlen(q, qsl, max(chunks), pool, table, lens, mx, fog_vscale=vs, out=out)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    for i, c in enumerate(chunks):
        if c == 0:
            continue
        s = starts[i]
        rows = torch.unique(torch.tensor([0, c // 2, c - 1]))
        qq = q[s:s + c].unsqueeze(0).cpu()
        if ctxs[i] > 8192:
            ref = paged_prefill_blockwise(qq, pool, table[i:i + 1].cpu(), lens[i:i + 1].cpu(), rows,
                                          fog_vscale=vs[i].cpu())
        else:
            ref = paged_prefill_ref(qq, pool.cpu(), table[i:i + 1].cpu(), lens[i:i + 1].cpu(), vs[i].cpu(), None, 0,
                                    rows=rows)
        _check(out[s:s + c][rows.long()].unsqueeze(0), ref, torch.bfloat16)
        if force:
            # at an equal (forced) split count the per-sequence launch sums the
            # same partials in the same order
            one = ops.fog_prefill(q[s:s + c].unsqueeze(0).contiguous(), pool, table[i:i + 1], lens[i:i + 1], mx,
                                  fog_vscale=vs[i:i + 1])
            torch.cuda.synchronize()
            assert torch.equal(out[s:s + c], one[0]), f"sequence {i}"


def test_prefill_varlen_many_sequences(dev):
    """70 sequences (the tile numbering scans query_start_loc 64 at a time),
    chunk lengths 0..80 with empty ones, every row against the oracle."""
    from kessie_amd import ops

    g = torch.Generator().manual_seed(31)
    b, hq, hkv, d = 70, 16, 8, 128
    chunks = torch.randint(0, 81, (b,), generator=g).tolist()
    chunks[3] = chunks[64] = 0
    ctxs = [c + int(x) for c, x in zip(chunks, torch.randint(1, 400, (b,), generator=g))]
    _, pool, table, lens = _case(dev, b, 1, ctxs, hq, hkv, torch.bfloat16, seed=32)
    starts = [0]
    for c in chunks:
        starts.append(starts[-1] + c)
    qsl = torch.tensor(starts, dtype=torch.int32, device=dev)
    q = torch.randn(starts[-1], hq, d, generator=gen(dev, 33), device=dev).to(torch.bfloat16)
    out = torch.full_like(q, float("nan"))
    assert ops.fog_prefill_varlen(q, qsl, max(chunks), pool, table, lens, max(ctxs), out=out)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    pool_c, table_c, lens_c, out_c, q_c = pool.cpu(), table.cpu(), lens.cpu(), out.cpu(), q.cpu()
    for i, c in enumerate(chunks):
        if c == 0:
            continue
        s = starts[i]
        ref = paged_prefill_ref(q_c[s:s + c].unsqueeze(0), pool_c, table_c[i:i + 1], lens_c[i:i + 1])
        _check(out_c[s:s + c].unsqueeze(0), ref, torch.bfloat16)


@pytest.mark.parametrize("hq,dtype,fog,causal,window", [(8, torch.bfloat16, "vscale", True, 0),
                                                        (16, torch.float16, "bias", True, 300),
                                                        (64, torch.bfloat16, "both", True, 0),
                                                        (32, torch.float16, "none", False, 0)])
def test_prefill_split_k_forced_shapes(dev, hq, dtype, fog, causal, window, monkeypatch):
    """Three forced key splits for every GQA ratio and fog mode, fp16 and bf16,
    ragged contexts, a window and the non-causal form: all rows against the
    oracle."""
    from kessie_amd import ops

    monkeypatch.setenv("KESSIE_PREFILL_SPLITS", "3")
    ctxs = [2000, 1337]
    q, pool, table, lens = _case(dev, 2, 150, ctxs, hq, 8, dtype, seed=hq)
    vs = torch.rand(2, 2000, generator=gen(dev, 41), device=dev) if fog in ("vscale", "both") else None
    bias = fog_bias(2000, 0.5, 0.5, {5, 700, 1999}, 0.1).to(dev) if fog in ("bias", "both") else None
    out = ops.fog_prefill(q, pool, table, lens, 2000, fog_vscale=vs, fog_bias=bias, window=window, causal=causal)
    torch.cuda.synchronize()
    for b in range(2):
        ref = paged_prefill_ref(q[b:b + 1].cpu(), pool.cpu(), table[b:b + 1].cpu(), lens[b:b + 1].cpu(),
                                None if vs is None else vs[b].cpu(), None if bias is None else bias.cpu(), window,
                                causal=causal)
        _check(out[b:b + 1], ref, dtype)


def test_prefill_varlen_chunk_longer_than_max_query_len(dev, monkeypatch):
    """A chunk longer than max_query_len is read as its first max_query_len
    queries at the last max_query_len positions of its context (the rest of
    its rows untouched) and the other sequences are unaffected, also when the
    key range is split: partial rows are indexed by max_query_len and must not
    overrun the workspace."""
    from kessie_amd import ops

    monkeypatch.setenv("KESSIE_PREFILL_SPLITS", "4")
    chunks, ctxs, mq = [300, 50], [3000, 2000], 200
    _, pool, table, lens = _case(dev, 2, 1, ctxs, 32, 8, torch.bfloat16, seed=51)
    qsl = torch.tensor([0, 300, 350], dtype=torch.int32, device=dev)
    q = torch.randn(350, 32, 128, generator=gen(dev, 52), device=dev).to(torch.bfloat16)
    out = torch.full_like(q, float("nan"))
    assert ops.fog_prefill_varlen(q, qsl, mq, pool, table, lens, 3000, out=out)
    torch.cuda.synchronize()
    assert torch.isnan(out[mq:300]).all()
    ref0 = paged_prefill_ref(q[:mq].unsqueeze(0).cpu(), pool.cpu(), table[:1].cpu(), lens[:1].cpu())
    _check(out[:mq].unsqueeze(0), ref0, torch.bfloat16)
    ref1 = paged_prefill_ref(q[300:].unsqueeze(0).cpu(), pool.cpu(), table[1:].cpu(), lens[1:].cpu())
    _check(out[300:].unsqueeze(0), ref1, torch.bfloat16)


def test_prefill_longest_first_dispatch(dev, monkeypatch):
    """A causal batch whose chunks are most of their contexts and whose grid
    takes several rounds dispatches query tiles longest first: same arithmetic
    per tile, so it equals one-sequence launches (one round, plain order, held
    to one key split) bit for bit, and the oracle on sampled rows."""
    from kessie_amd import ops

    monkeypatch.setenv("KESSIE_PREFILL_SPLITS", "1")
    c, ctxs = 1500, [1500, 2000, 2900]
    q, pool, table, lens = _case(dev, 3, c, ctxs, 32, 8, torch.bfloat16, seed=61)
    vs = torch.rand(3, 2900, generator=gen(dev, 62), device=dev)
    out = ops.fog_prefill(q, pool, table, lens, 2900, fog_vscale=vs)
    torch.cuda.synchronize()
    rows = torch.tensor([0, 700, 1499])
    for i in range(3):
        one = ops.fog_prefill(q[i:i + 1].contiguous(), pool, table[i:i + 1], lens[i:i + 1], 2900,
                              fog_vscale=vs[i:i + 1])
        torch.cuda.synchronize()
        assert torch.equal(out[i:i + 1], one), f"sequence {i}"
        ref = paged_prefill_ref(q[i:i + 1].cpu(), pool.cpu(), table[i:i + 1].cpu(), lens[i:i + 1].cpu(),
                                vs[i].cpu(), None, 0, rows=rows)
        _check(out[i:i + 1, rows], ref, torch.bfloat16)


@pytest.mark.parametrize("hq,hkv,c,ctxs,fog,window,page_size,splits", [
    (32, 8, 100, [1000, 777], "vscale", 0, 16, 0),    # two sequences, one ragged
    (8, 8, 33, [300], "bias", 0, 16, 0),               # GQA 1
    (12, 3, 65, [900], "both", 50, 16, 0),             # GQA 4 with three kv heads, window
    (24, 8, 40, [2000], "none", 0, 32, 0),             # GQA 3 (positions per workgroup not a power of two), 32-token pages
    (32, 8, 300, [300], "vscale", 0, 16, 0),           # a fresh prompt: the chunk is the whole context
    (32, 8, 50, [51], "none", 0, 16, 0),               # one cached token before the chunk
    (16, 4, 20, [5000], "vscale", 0, 64, 5),           # forced key splits (partials + combine), 64-token pages
    (128, 8, 7, [4000, 7], "bias", 1000, 16, 0),       # GQA 16, window, a context that is only the chunk
])
def test_prefill_fp32_mfma_matches_oracle_and_generic(dev, monkeypatch, hq, hkv, c, ctxs, fog, window, page_size,
                                                      splits):
    """fp32 chunked prefill on v_mfma_f32_16x16x4_f32 (fp32 throughout):
    within the fp32 tolerance (1e-5) of the oracle and of the generic kernel,
    and not the generic kernel's bits (the MFMA route ran)."""
    from kessie_amd import ops

    if splits:
        monkeypatch.setenv("KESSIE_PREFILL_SPLITS", str(splits))
    b = len(ctxs)
    mx = max(ctxs)
    q, pool, table, lens = _case(dev, b, c, ctxs, hq, hkv, torch.float32, seed=hq + c, page_size=page_size)
    vs = torch.rand(b, mx, generator=gen(dev, 41), device=dev) if fog in ("vscale", "both") else None
    bias = fog_bias(mx, 0.5, 0.5, {3, mx // 2}, 0.1).to(dev) if fog in ("bias", "both") else None
    out = ops.fog_prefill(q, pool, table, lens, mx, fog_vscale=vs, fog_bias=bias, window=window)
    monkeypatch.setenv("KESSIE_FORCE_GENERIC", "1")
    gen_out = ops.fog_prefill(q, pool, table, lens, mx, fog_vscale=vs, fog_bias=bias, window=window)
    torch.cuda.synchronize()
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), None if vs is None else vs.cpu(),
                            None if bias is None else bias.cpu(), window)
    _check(out, ref, torch.float32)
    _check(gen_out, ref, torch.float32)
    assert not torch.equal(out, gen_out)


def test_prefill_fp32_mfma_bad_page(dev):
    """An invalid page id on the fp32 MFMA route masks its 16 tokens:
    non-causal, so the oracle is the same context without that page."""
    from kessie_amd import ops

    q, pool, table, lens = _case(dev, 1, 40, [400], 32, 8, torch.float32, seed=9)
    table[0, 3] = -1
    out = ops.fog_prefill(q, pool, table, lens, 400, causal=False)
    torch.cuda.synchronize()
    keep = [i for i in range(table.shape[1]) if i != 3]
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu()[:, keep].contiguous(), torch.tensor([400 - 16]),
                            causal=False)
    _check(out, ref, torch.float32)


@pytest.mark.parametrize("splits,window", [(300, 0), (7, 100)])
def test_prefill_fp32_mfma_many_splits(dev, monkeypatch, splits, window):
    """fp32 MFMA prefill with more key splits than the load-ahead combine
    takes (300: the per-row combine merges them) and a windowed split: both
    at 1e-5 of the oracle; most of the 300 splits hold no key block and store
    empty partials."""
    from kessie_amd import ops

    monkeypatch.setenv("KESSIE_PREFILL_SPLITS", str(splits))
    q, pool, table, lens = _case(dev, 2, 24, [3000, 1200], 32, 8, torch.float32, seed=77)
    vs = torch.rand(2, 3000, generator=gen(dev, 78), device=dev)
    out = ops.fog_prefill(q, pool, table, lens, 3000, fog_vscale=vs, window=window)
    torch.cuda.synchronize()
    ref = paged_prefill_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), vs.cpu(), None, window)
    _check(out, ref, torch.float32)


def _varlen_q(dev, chunks, hq, dtype, seed, lead=0):
    starts = [lead]
    for c in chunks:
        starts.append(starts[-1] + c)
    qsl = torch.tensor(starts, dtype=torch.int32, device=dev)
    q_all = torch.randn(starts[-1], hq, 128, generator=gen(dev, seed), device=dev).to(dtype)
    return qsl, q_all[lead:], [x - lead for x in starts]


@pytest.mark.parametrize("hq,hkv,page_size,fog,window,splits", [
    (32, 8, 16, "vscale", 0, 1),     # one key split: every row written by the attention kernel
    (32, 8, 16, "bias", 50, 5),      # five forced splits (partials + combine), window
    (24, 8, 32, "none", 0, 3),       # GQA 3, 32-token pages
    (128, 8, 16, "both", 300, 2),    # GQA 16
])
def test_prefill_fp32_varlen_matches_per_sequence(dev, monkeypatch, hq, hkv, page_size, fog, window, splits):
    """fp32 varlen prefill (one launch of the fp32 MFMA kernel over ragged
    chunks incl. a one-token chunk and an empty one, query_start_loc starting
    at 5) equals the per-sequence fp32 launches bit for bit at an equal key
    split count, and the oracle within 1e-5."""
    from kessie_amd import ops

    monkeypatch.setenv("KESSIE_PREFILL_SPLITS", str(splits))
    chunks, ctxs = [37, 1, 300, 0, 129], [900, 64, 300, 50, 4000]
    b, mx = len(chunks), max(ctxs)
    _, pool, table, lens = _case(dev, b, 1, ctxs, hq, hkv, torch.float32, seed=61, page_size=page_size)
    qsl, q, starts = _varlen_q(dev, chunks, hq, torch.float32, 62, lead=5)
    vs = torch.rand(b, mx, generator=gen(dev, 63), device=dev) if fog in ("vscale", "both") else None
    bias = fog_bias(mx, 0.5, 0.5, {3, 17, 200}, 0.1).to(dev) if fog in ("bias", "both") else None
    out = torch.full_like(q, float("nan"))
    assert ops.fog_prefill_varlen(q, qsl, max(chunks), pool, table, lens, mx, fog_vscale=vs, fog_bias=bias,
                                  window=window, out=out)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    for i, c in enumerate(chunks):
        if c == 0:
            continue
        s = starts[i]
        one = ops.fog_prefill(q[s:s + c].unsqueeze(0).contiguous(), pool, table[i:i + 1], lens[i:i + 1], mx,
                              fog_vscale=None if vs is None else vs[i:i + 1], fog_bias=bias, window=window)
        torch.cuda.synchronize()
        assert torch.equal(out[s:s + c], one[0]), f"sequence {i}"
        ref = paged_prefill_ref(q[s:s + c].unsqueeze(0).cpu(), pool.cpu(), table[i:i + 1].cpu(),
                                lens[i:i + 1].cpu(), None if vs is None else vs[i].cpu(),
                                None if bias is None else bias.cpu(), window)
        _check(out[s:s + c].unsqueeze(0), ref, torch.float32)


def test_prefill_fp32_varlen_many_sequences_sized_splits(dev):
    """70 ragged fp32 sequences (the tile numbering scans query_start_loc 64
    at a time; empty chunks at 3 and 64) at the sized split count, every row
    against the oracle within 1e-5."""
    from kessie_amd import ops

    g = torch.Generator().manual_seed(71)
    b, hq, hkv = 70, 16, 8
    chunks = torch.randint(0, 81, (b,), generator=g).tolist()
    chunks[3] = chunks[64] = 0
    ctxs = [c + int(x) for c, x in zip(chunks, torch.randint(1, 400, (b,), generator=g))]
    _, pool, table, lens = _case(dev, b, 1, ctxs, hq, hkv, torch.float32, seed=72)
    qsl, q, starts = _varlen_q(dev, chunks, hq, torch.float32, 73)
    out = torch.full_like(q, float("nan"))
    assert ops.fog_prefill_varlen(q, qsl, max(chunks), pool, table, lens, max(ctxs), out=out)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    pool_c, table_c, lens_c, out_c, q_c = pool.cpu(), table.cpu(), lens.cpu(), out.cpu(), q.cpu()
    for i, c in enumerate(chunks):
        if c == 0:
            continue
        s = starts[i]
        ref = paged_prefill_ref(q_c[s:s + c].unsqueeze(0), pool_c, table_c[i:i + 1], lens_c[i:i + 1])
        _check(out_c[s:s + c].unsqueeze(0), ref, torch.float32)


@pytest.mark.parametrize("splits", [1, 4])
def test_prefill_fp32_varlen_chunk_longer_than_max_query_len(dev, monkeypatch, splits):
    """fp32 varlen: a chunk longer than max_query_len is read as its first
    max_query_len queries at the last max_query_len positions of its context,
    its other rows untouched, the next sequence unaffected, with and without
    key splits (partial rows indexed by max_query_len)."""
    from kessie_amd import ops

    monkeypatch.setenv("KESSIE_PREFILL_SPLITS", str(splits))
    mq = 200
    _, pool, table, lens = _case(dev, 2, 1, [3000, 2000], 32, 8, torch.float32, seed=81)
    qsl, q, _ = _varlen_q(dev, [300, 50], 32, torch.float32, 82)
    out = torch.full_like(q, float("nan"))
    assert ops.fog_prefill_varlen(q, qsl, mq, pool, table, lens, 3000, out=out)
    torch.cuda.synchronize()
    assert torch.isnan(out[mq:300]).all()
    ref0 = paged_prefill_ref(q[:mq].unsqueeze(0).cpu(), pool.cpu(), table[:1].cpu(), lens[:1].cpu())
    _check(out[:mq].unsqueeze(0), ref0, torch.float32)
    ref1 = paged_prefill_ref(q[300:].unsqueeze(0).cpu(), pool.cpu(), table[1:].cpu(), lens[1:].cpu())
    _check(out[300:].unsqueeze(0), ref1, torch.float32)
