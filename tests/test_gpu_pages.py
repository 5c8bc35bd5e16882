"""GPU parity: paged-KV management vs the CPU oracle (bit-exact: page tables,
gather indices, eviction order, valid masks, gathered bytes)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import pages as P
from tests.inputs import gen, paged_pool, randperm

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def test_legacy_page_evict_known_answer(dev):
    """kessie_kernels_v2.hip:1008-1023: 128 valid pages at pos i*128, thr 8192 -> 64."""
    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    kk = KeSSieKernels()
    valid = torch.zeros(256, dtype=torch.int8, device=dev)
    valid[:128] = 1
    pos = torch.zeros(256, dtype=torch.int32, device=dev)
    pos[:128] = torch.arange(128, device=dev, dtype=torch.int32) * 128
    ref_valid, ref_count = P.threshold_evict(_np(valid), _np(pos), 8192)
    n = kk.page_evict(valid, pos, 8192)
    assert n == 64 == ref_count
    assert np.array_equal(_np(valid), ref_valid)


@pytest.mark.parametrize("seed", [0, 1])
def test_evict_list_matches_free_list_order(dev, seed):
    from kessie_amd import ops

    rng = np.random.default_rng(seed)
    n = 5000
    valid = rng.integers(0, 2, n).astype(np.int8)
    allocated = np.where(valid == 1, 1, rng.integers(0, 2, n)).astype(np.int8)
    pos = rng.integers(0, 100000, n).astype(np.int32)
    ref_valid, ref_alloc, ref_freed = P.evict_list(valid, pos, allocated, 50000)
    dv, dp, da = (torch.from_numpy(x).to(dev) for x in (valid, pos, allocated))
    lst, cnt = ops.page_evict_list(dv, dp, 50000, da)
    torch.cuda.synchronize()
    c = int(cnt.item())
    assert c == len(ref_freed)
    assert np.array_equal(_np(lst[:c]), ref_freed)
    assert np.array_equal(_np(dv), ref_valid)
    assert np.array_equal(_np(da), ref_alloc)


@pytest.mark.parametrize("n,frac,k", [(65536, 0.25, -1), (1000, 0.25, -1), (3000, 0.0, 17), (777, 0.5, -1),
                                      (4096, 0.25, 100000)])
def test_select_evict_bit_exact(dev, n, frac, k):
    from kessie_amd import ops

    g = torch.Generator().manual_seed(n)
    scores = torch.rand(n, generator=g)
    # Plant duplicates, -0/+0 and negative scores to exercise the tie order.
    scores[: n // 10] = scores[n // 10: 2 * (n // 10)]
    scores[5] = -0.0
    scores[6] = 0.0
    scores[7] = -1.5
    valid = (torch.rand(n, generator=g) < 0.9).to(torch.int8)
    ref_valid, ref_list = P.select_evict(scores.numpy(), valid.numpy(), k, frac)
    dv = valid.to(dev)
    lst, cnt = ops.page_select_evict(scores.to(dev), dv, k, frac)
    torch.cuda.synchronize()
    c = int(cnt.item())
    assert c == len(ref_list)
    assert np.array_equal(_np(lst[:c]), ref_list)
    assert np.array_equal(_np(dv), ref_valid)


@pytest.mark.parametrize("n,distinct,frac", [
    (5000, 50, 0.25),       # many ties at the threshold score: id resolution on the LDS copy
    (65536, 1, 0.25),       # one score for every page: the bucket overflows LDS -> streaming passes
    (40000, 3, 0.5),        # three values, buckets above the LDS capacity
    (20000, 20000, 0.999),  # nearly everything evicted
])
def test_select_evict_ties_bit_exact(dev, n, distinct, frac):
    from kessie_amd import ops

    g = torch.Generator().manual_seed(distinct)
    values = torch.rand(distinct, generator=g)
    scores = values[torch.randint(0, distinct, (n,), generator=g)]
    valid = (torch.rand(n, generator=g) < 0.95).to(torch.int8)
    ref_valid, ref_list = P.select_evict(scores.numpy(), valid.numpy(), -1, frac)
    dv = valid.to(dev)
    lst, cnt = ops.page_select_evict(scores.to(dev), dv, -1, frac)
    torch.cuda.synchronize()
    c = int(cnt.item())
    assert c == len(ref_list)
    assert np.array_equal(_np(lst[:c]), ref_list)
    assert np.array_equal(_np(dv), ref_valid)


def test_compact_and_gather_bit_exact(dev):
    from kessie_amd import ops

    num_pages, s, w = 4096, 8, 512
    pool = paged_pool(num_pages, 16, 8, 128, torch.bfloat16, dev, 0)
    tables = randperm(num_pages, dev, 1).view(s, w).contiguous()
    lens = torch.tensor([512, 0, 1, 300, 511, 512, 17, 256], dtype=torch.int32, device=dev)
    tables[2, 0] = -1  # out-of-range entries never survive
    valid = (torch.rand(num_pages, generator=gen(dev, 2), device=dev) < 0.7).to(torch.int8)
    nt, nl, gi, gc = ops.page_compact(tables, lens, valid)
    out = ops.page_gather(pool, gi, gc, n=s * w)
    torch.cuda.synchronize()
    rt, rl, rg = P.compact(_np(tables), _np(lens), _np(valid))
    assert np.array_equal(_np(nt), rt)
    assert np.array_equal(_np(nl), rl)
    c = int(gc.item())
    assert c == len(rg)
    assert np.array_equal(_np(gi[:c]), rg)
    ref_bytes = P.gather_pages(_np(pool.view(num_pages, -1).view(torch.int16)), rg)
    assert np.array_equal(_np(out[:c].reshape(c, -1).view(torch.int16)), ref_bytes)


def test_valid_list_matches_get_layer_kv_order(dev):
    from kessie_amd import ops

    valid = (torch.rand(10000, generator=gen(dev, 3), device=dev) < 0.3).to(torch.int8)
    idx, cnt = ops.page_valid_list(valid)
    torch.cuda.synchronize()
    ref = P.valid_list(_np(valid))
    assert int(cnt.item()) == len(ref)
    assert np.array_equal(_np(idx[: len(ref)]), ref)


def test_score_evict_full_config(dev):
    """Config: 65,536-page pool (1,048,576 tokens), 64 sequences x 1,024 pages,
    scores ~ U(0,1), evict the lowest 25%, compact, gather survivors (3 GiB)."""
    from kessie_amd import ops

    num_pages, s, w = 65536, 64, 1024
    pool = paged_pool(num_pages, 16, 8, 128, torch.bfloat16, dev, 0)
    tables = randperm(num_pages, dev, 1).view(s, w).contiguous()
    scores = torch.rand(num_pages, generator=gen(dev, 2), device=dev)
    valid = torch.ones(num_pages, dtype=torch.int8, device=dev)
    lens = torch.full((s,), w, dtype=torch.int32, device=dev)
    lst, cnt = ops.page_select_evict(scores, valid, -1, 0.25)
    nt, nl, gi, gc = ops.page_compact(tables, lens, valid)
    out = ops.page_gather(pool, gi, gc, n=s * w)
    torch.cuda.synchronize()
    rv, rlist = P.select_evict(_np(scores), np.ones(num_pages, np.int8), -1, 0.25)
    assert len(rlist) == 16384
    assert int(cnt.item()) == 16384 and np.array_equal(_np(lst[:16384]), rlist)
    assert np.array_equal(_np(valid), rv)
    rt, rl, rg = P.compact(_np(tables), _np(lens), rv)
    assert np.array_equal(_np(nt), rt) and np.array_equal(_np(nl), rl)
    c = int(gc.item())
    assert c == 49152 and np.array_equal(_np(gi[:c]), rg)
    # Gathered bytes: every gathered page compared with its source page, on the
    # device, 4,096 pages (256 MiB) at a time.
    ref_idx = torch.from_numpy(rg).to(dev).long()
    for i in range(0, c, 4096):
        assert torch.equal(out[i:i + 4096], pool[ref_idx[i:i + 4096]]), f"pages {i}.."


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_insert_matches_oracle(dev, dtype):
    from kessie_amd import ops

    num_pages, p, h, d = 64, 16, 8, 128
    pool = paged_pool(num_pages, p, h, d, dtype, dev, 0)
    t = 70
    nk = torch.randn(t, h, d, generator=gen(dev, 1), device=dev).to(dtype)
    nv = torch.randn(t, h, d, generator=gen(dev, 2), device=dev).to(dtype)
    target = torch.tensor([5, -1, 63, 64, 9], dtype=torch.int32, device=dev)
    valid = torch.zeros(num_pages, dtype=torch.int8, device=dev)
    posn = torch.zeros(num_pages, dtype=torch.int32, device=dev)
    ref_pool, ref_valid, ref_pos = (x.cpu().numpy().copy() for x in (pool.view(torch.int16) if dtype != torch.float32 else pool, valid, posn))
    P.page_insert(ref_pool, (nk.view(torch.int16) if dtype != torch.float32 else nk).cpu().numpy(),
                  (nv.view(torch.int16) if dtype != torch.float32 else nv).cpu().numpy(), target.cpu().numpy(),
                  ref_valid, ref_pos, 1000)
    ops.page_insert(pool, nk, nv, target, valid, posn, 1000)
    torch.cuda.synchronize()
    got = (pool.view(torch.int16) if dtype != torch.float32 else pool).cpu().numpy()
    assert np.array_equal(got, ref_pool)
    assert np.array_equal(_np(valid), ref_valid)
    assert np.array_equal(_np(posn), ref_pos)


def test_insert_with_remap_matches_insert_then_remap(dev):
    from kessie_amd import ops

    num_pages, p, h, d = 32, 16, 8, 128
    pool_a = paged_pool(num_pages, p, h, d, torch.bfloat16, dev, 0)
    pool_b = pool_a.clone()
    t = 48
    nk = torch.randn(t, h, d, generator=gen(dev, 1), device=dev).bfloat16()
    nv = torch.randn(t, h, d, generator=gen(dev, 2), device=dev).bfloat16()
    target = torch.tensor([3, 7, 11], dtype=torch.int32, device=dev)
    orig = torch.randint(0, 1_000_000, (t,), generator=gen(dev, 3), device=dev, dtype=torch.int32)
    tgt = (5000 + torch.arange(t, device=dev)).to(torch.int32)
    va, pa = torch.zeros(num_pages, dtype=torch.int8, device=dev), torch.zeros(num_pages, dtype=torch.int32, device=dev)
    vb, pb = va.clone(), pa.clone()
    ops.page_insert(pool_a, nk, nv, target, va, pa, 0, orig_pos=orig, tgt_pos=tgt, rope_theta=500000.0)
    ops.page_insert(pool_b, nk, nv, target, vb, pb, 0)
    ops.rope_remap_paged(pool_b, orig, tgt, 500000.0, page_list=target)
    torch.cuda.synchronize()
    assert torch.equal(pool_a, pool_b)  # same kernels' arithmetic, same bits
    assert torch.equal(va, vb) and torch.equal(pa, pb)


def test_legacy_page_insert_fp16(dev):
    from kessie_amd import _lib

    num_pages, p, h, d = 16, 8, 4, 64
    pool = torch.zeros(num_pages, p, 2, h, d, dtype=torch.float16, device=dev)
    t = 20
    nk = torch.randn(t, h, d, generator=gen(dev, 5), device=dev).half()
    nv = torch.randn(t, h, d, generator=gen(dev, 6), device=dev).half()
    target = torch.tensor([2, 40, 9], dtype=torch.int32, device=dev)
    valid = torch.zeros(num_pages, dtype=torch.int8, device=dev)
    posn = torch.zeros(num_pages, dtype=torch.int32, device=dev)
    rp, rv, rpos = pool.cpu().numpy().copy(), valid.cpu().numpy().copy(), posn.cpu().numpy().copy()
    P.page_insert(rp, nk.cpu().numpy(), nv.cpu().numpy(), target.cpu().numpy(), rv, rpos, 77)
    ptr = lambda x: ctypes.c_void_p(x.data_ptr())
    _lib.call_legacy("launch_kessie_page_insert", ptr(pool), ptr(nk), ptr(nv), ptr(target), ptr(valid), ptr(posn),
                     77, t, h, d, p, num_pages, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy(), rp)
    assert np.array_equal(_np(valid), rv) and np.array_equal(_np(posn), rpos)


@pytest.mark.parametrize("n,s,w,frac,k,distinct", [
    (65536, 64, 1024, 0.25, -1, 0),       # the full config's shape
    (1000, 3, 700, 0.25, -1, 0),
    (5000, 8, 600, 0.5, -1, 40),          # many tied scores at the threshold
    (65536, 2, 30000, 0.25, -1, 1),       # one score for every page (candidates overflow LDS)
    (20000, 100, 150, 0.0, 17, 0),        # explicit k
    (3000, 5, 500, 0.0, -1, 0),           # nothing evicted
    (70000, 300, 200, 0.999, -1, 0),      # more tiles than workgroups' first pass; nearly all evicted
])
def test_evict_compact_matches_oracle(dev, n, s, w, frac, k, distinct):
    """The fused call equals select_evict followed by compact (the oracle),
    bit for bit: evict list and count, valid flags, compacted tables, lengths,
    gather indices and count."""
    from kessie_amd import ops

    g = torch.Generator().manual_seed(n + s)
    if distinct:
        values = torch.rand(distinct, generator=g)
        scores = values[torch.randint(0, distinct, (n,), generator=g)]
    else:
        scores = torch.rand(n, generator=g)
        scores[5] = -0.0
        scores[6] = 0.0
        scores[7] = -2.0
    valid = (torch.rand(n, generator=g) < 0.9).to(torch.int8)
    tables = torch.randint(-3, n + 3, (s, w), generator=g, dtype=torch.int32)  # incl. out-of-range ids
    lens = torch.randint(0, w + 1, (s,), generator=g, dtype=torch.int32)
    lens[0] = w
    rv, rlist = P.select_evict(scores.numpy(), valid.numpy(), k, frac)
    rt, rl, rg = P.compact(tables.numpy(), lens.numpy(), rv)
    dv = valid.to(dev)
    lst, cnt, nt, nl, gi, gc = ops.page_evict_compact(scores.to(dev), dv, tables.to(dev), lens.to(dev), k, frac)
    torch.cuda.synchronize()
    c = int(cnt.item())
    assert c == len(rlist) and np.array_equal(_np(lst[:c]), rlist)
    assert np.array_equal(_np(dv), rv)
    assert np.array_equal(_np(nt), rt) and np.array_equal(_np(nl), rl)
    m = int(gc.item())
    assert m == len(rg) and np.array_equal(_np(gi[:m]), rg)


@pytest.mark.parametrize("n,s,w", [(4099, 3, 1500), (1, 2, 4), (4096, 5, 1024)])
def test_evict_compact_edge_values(dev, n, s, w):
    """Edge values through the fused call, against the oracle bit for bit:
    lengths below 0 and past the row width (clamped), page ids at the int32
    limits and just outside [0, n), valid flags other than 0 and 1 (only 1 is
    valid), a page count one past a 4,096-key tile or a single page, and rows
    wider than 1,024 entries (more than one chunk per row)."""
    from kessie_amd import ops

    g = torch.Generator().manual_seed(n * 7 + w)
    scores = torch.rand(n, generator=g)
    valid = torch.randint(-1, 3, (n,), generator=g, dtype=torch.int8)
    valid[: max(1, n // 2)] = 1
    tables = torch.randint(0, n, (s, w), generator=g, dtype=torch.int32)
    specials = torch.tensor([-(2 ** 31), 2 ** 31 - 1, -1, n, n - 1, 0, 2 ** 30 + 1, -(2 ** 30)], dtype=torch.int32)
    for r in range(s):
        pos = torch.randint(0, w, (min(w, 8),), generator=g)
        tables[r, pos] = specials[: len(pos)]
    lens = torch.tensor([(-5, w + 7, w // 2, w, 0)[r % 5] for r in range(s)], dtype=torch.int32)
    rv, rlist = P.select_evict(scores.numpy(), valid.numpy(), -1, 0.25)
    rt, rl, rg = P.compact(tables.numpy(), lens.numpy(), rv)
    dv = valid.to(dev)
    lst, cnt, nt, nl, gi, gc = ops.page_evict_compact(scores.to(dev), dv, tables.to(dev), lens.to(dev), -1, 0.25)
    torch.cuda.synchronize()
    c = int(cnt.item())
    assert c == len(rlist) and np.array_equal(_np(lst[:c]), rlist)
    assert np.array_equal(_np(dv), rv)
    assert np.array_equal(_np(nt), rt) and np.array_equal(_np(nl), rl)
    m = int(gc.item())
    assert m == len(rg) and np.array_equal(_np(gi[:m]), rg)
    # the standalone compaction (look-back kernel) on the post-eviction flags
    nt2, nl2, gi2, gc2 = ops.page_compact(tables.to(dev), lens.to(dev), dv)
    torch.cuda.synchronize()
    assert np.array_equal(_np(nt2), rt) and np.array_equal(_np(nl2), rl)
    m2 = int(gc2.item())
    assert m2 == len(rg) and np.array_equal(_np(gi2[:m2]), rg)


def test_evict_compact_rejects_too_many_rows(dev):
    from kessie_amd import _lib, ops

    n = 100
    tables = torch.zeros(8193, 1, dtype=torch.int32, device=dev)
    lens = torch.ones(8193, dtype=torch.int32, device=dev)
    with pytest.raises(_lib.KeSSieError) as e:
        ops.page_evict_compact(torch.rand(n, device=dev), torch.ones(n, dtype=torch.int8, device=dev), tables, lens)
    assert e.value.status == _lib.ERR_UNSUPPORTED


def test_evict_compact_full_config_then_gather(dev):
    """Config: 65,536-page pool, 64 x 1,024 tables, evict the lowest 25%, fused
    evict + compact, gather every survivor; every gathered page compared."""
    from kessie_amd import ops

    num_pages, s, w = 65536, 64, 1024
    pool = paged_pool(num_pages, 16, 8, 128, torch.bfloat16, dev, 0)
    tables = randperm(num_pages, dev, 1).view(s, w).contiguous()
    scores = torch.rand(num_pages, generator=gen(dev, 2), device=dev)
    valid = torch.ones(num_pages, dtype=torch.int8, device=dev)
    lens = torch.full((s,), w, dtype=torch.int32, device=dev)
    lst, cnt, nt, nl, gi, gc = ops.page_evict_compact(scores, valid, tables, lens, -1, 0.25)
    out = ops.page_gather(pool, gi, gc, n=s * w)
    torch.cuda.synchronize()
    rv, rlist = P.select_evict(_np(scores), np.ones(num_pages, np.int8), -1, 0.25)
    rt, rl, rg = P.compact(_np(tables), _np(lens), rv)
    assert int(cnt.item()) == 16384 and np.array_equal(_np(lst[:16384]), rlist)
    assert np.array_equal(_np(valid), rv)
    assert np.array_equal(_np(nt), rt) and np.array_equal(_np(nl), rl)
    c = int(gc.item())
    assert c == 49152 and np.array_equal(_np(gi[:c]), rg)
    ref_idx = torch.from_numpy(rg).to(dev).long()
    for i in range(0, c, 4096):
        assert torch.equal(out[i:i + 4096], pool[ref_idx[i:i + 4096]]), f"pages {i}.."


def test_select_evict_needs_an_initialised_workspace(dev):
    """Through the C ABI with a caller-owned workspace: a workspace that was
    never prepared by kessie_page_workspace_init is refused (count -2, flags
    untouched); once prepared, repeated calls on it (each restoring the
    scratch for the next) all match the oracle."""
    from kessie_amd import _lib

    lib = _lib.load()
    n = 5000
    g = torch.Generator().manual_seed(11)
    scores = torch.rand(n, generator=g)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nbytes = lib.kessie_page_workspace_bytes(n)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    sc = scores.to(dev)
    valid = torch.ones(n, dtype=torch.int8, device=dev)
    lst = torch.empty(n, dtype=torch.int32, device=dev)
    cnt = torch.zeros(1, dtype=torch.int32, device=dev)

    def call():
        _lib.check("kessie_page_select_evict", lib.kessie_page_select_evict(
            ptr(sc), ptr(valid), n, -1, 0.25, ptr(lst), ptr(cnt), ptr(ws), nbytes, stream))
        torch.cuda.synchronize()

    call()
    assert int(cnt.item()) == -2 and bool((valid == 1).all())
    _lib.check("kessie_page_workspace_init", lib.kessie_page_workspace_init(ptr(ws), nbytes, stream))
    ref_valid, ref_list = P.select_evict(scores.numpy(), np.ones(n, np.int8), -1, 0.25)
    for _ in range(3):
        valid.fill_(1)
        call()
        c = int(cnt.item())
        assert c == len(ref_list) and np.array_equal(_np(lst[:c]), ref_list)
        assert np.array_equal(_np(valid), ref_valid)


def test_evict_compact_barrier_failure_leaves_outputs_untouched(dev, monkeypatch):
    """A grid-barrier wait that runs out fails the whole call: both counts read
    -1 and page_valid, the evict list, the tables and the gather indices keep
    their previous contents.  The condition is forced from the host
    (KESSIE_GRID_TEST_TIMEOUT: the first barrier waits for one arrival more
    than the grid has and gives up after a few polls, so every workgroup still
    exits normally).  The scratch is restored, so the next call on the same
    workspace matches the oracle bit for bit."""
    from kessie_amd import ops

    for n, s, w in [(262144, 64, 4096), (65536, 64, 1024), (5000, 3, 700)]:  # 64, 16 and 2 workgroups
        g = torch.Generator().manual_seed(n)
        scores = torch.rand(n, generator=g)
        valid = (torch.rand(n, generator=g) < 0.9).to(torch.int8)
        tables = torch.randint(0, n, (s, w), generator=g, dtype=torch.int32)
        lens = torch.randint(0, w + 1, (s,), generator=g, dtype=torch.int32)
        dsc, dtab, dlens = scores.to(dev), tables.to(dev), lens.to(dev)
        sentinel = -7
        for polls in ("0", "100"):
            dv = valid.to(dev)
            lst = torch.full((n,), sentinel, dtype=torch.int32, device=dev)
            nt = torch.full((s, w), sentinel, dtype=torch.int32, device=dev)
            nl = torch.full((s,), sentinel, dtype=torch.int32, device=dev)
            gi = torch.full((s * w,), sentinel, dtype=torch.int32, device=dev)
            cnt = torch.zeros(1, dtype=torch.int32, device=dev)
            gc = torch.zeros(1, dtype=torch.int32, device=dev)
            monkeypatch.setenv("KESSIE_GRID_TEST_TIMEOUT", polls)
            ops.page_evict_compact(dsc, dv, dtab, dlens, -1, 0.25, evict_list=lst, evict_count=cnt,
                                   new_tables=nt, new_lens=nl, gather_idx=gi, gather_count=gc)
            torch.cuda.synchronize()
            monkeypatch.delenv("KESSIE_GRID_TEST_TIMEOUT")
            assert int(cnt.item()) == -1 and int(gc.item()) == -1, (n, polls)
            assert torch.equal(dv.cpu(), valid)
            for t in (lst, nt, nl, gi):
                assert bool((t == sentinel).all())
        rv, rlist = P.select_evict(scores.numpy(), valid.numpy(), -1, 0.25)
        rt, rl, rg = P.compact(tables.numpy(), lens.numpy(), rv)
        dv = valid.to(dev)
        lst, cnt, nt, nl, gi, gc = ops.page_evict_compact(dsc, dv, dtab, dlens, -1, 0.25)
        torch.cuda.synchronize()
        c = int(cnt.item())
        assert c == len(rlist) and np.array_equal(_np(lst[:c]), rlist)
        assert np.array_equal(_np(dv), rv)
        assert np.array_equal(_np(nt), rt) and np.array_equal(_np(nl), rl)
        m = int(gc.item())
        assert m == len(rg) and np.array_equal(_np(gi[:m]), rg)
