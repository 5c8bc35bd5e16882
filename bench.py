#!/usr/bin/env python3
"""KeSSie hot path on one MI355X: fog-attention decode GB/s (primary) and RoPE
remap Mtok/s, with the kernels' roofline and the CPU oracle timed beside them.

Primary workload (the JSON ``value``): fog-attention decode, bf16, Llama-3-8B
attention shape -- batch 16, 32 query / 8 KV heads, head_dim 128, 131,072-token
context per sequence in 16-token pages (random page tables), V-fog weights
alpha 0.5 / fog_start 0.5, window 0.  A step is one decode of the batch
through the serving entry point (kessie_fog_decode_paged: the streaming kernel
plus the split-combine kernel).  ``value`` = algorithmic bytes of one decode /
step time.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu] [--no-secondary]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fog-attn decode GB/s (% HBM peak) @128K ctx; RoPE-remap Mtok/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def events(n):
    import torch

    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def backlog(ms: float = 5.0) -> None:
    """Queue a GPU spin of ~ms before a timed loop, so the launches behind it
    pile up and per-launch events time the kernels, not host launch gaps."""
    import torch

    torch.cuda._sleep(int(ms * 1e-3 * 2.4e9))


PREHEAT = True  # off for the counter passes, whose launch sequences must repeat exactly


def preheat(fn, ms: float = 150.0, cycle: int = 0) -> int:
    """Untimed calls of ``fn`` until ~ms of GPU time has passed, before a
    timed loop.  The device raises its clocks over the first tens of
    milliseconds of load: the first timed pass of the headline decode after 3
    warm-up steps ran 1.7 % slower than the passes after it (1,279 against
    1,257 us per step), so every timed loop starts from steady clocks.  Calls
    go in doubling batches, each timed with an event pair.  With cycle > 0,
    ``fn(j)`` is called with j = 0, 1, ... modulo cycle (the input sets the
    timed loop rotates through), else ``fn()``.  Returns the number of calls
    made (they are not steps of the measurement)."""
    import torch

    if not PREHEAT:
        return 0
    e0, e1 = events(2)
    total, n, calls = 0.0, 1, 0
    while total < ms and calls < 4096:
        e0.record()
        for j in range(calls, calls + n):
            if cycle > 0:
                fn(j % cycle)
            else:
                fn()
        e1.record()
        torch.cuda.synchronize()
        total += e0.elapsed_time(e1)
        calls += n
        n = min(2 * n, 256)
    return calls


def time_back_to_back(fn, reps):
    """ms per call of ``reps`` calls issued back to back between two events
    (behind a backlog, so the queue never drains).  For kernels of tens of
    microseconds an event pair around every launch adds the dispatch and
    completion of that launch (~2-3 us on MI355X); back to back, the time per
    call matches rocprofv3's kernel duration to ~1 %.  ``fn(i)`` makes call i.
    A pre-heat of the same calls (rotating i) brings the clocks up first."""
    preheat(fn, 100.0, cycle=reps)
    start, end = events(2)
    backlog()
    start.record()
    for i in range(reps):
        fn(i)
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps


def decode_bytes(b, ctx, hq, hkv, d, es, page_size, fog=True):
    pages = (ctx + page_size - 1) // page_size
    kv = b * ctx * hkv * d * 2 * es
    return kv + 2 * b * hq * d * es + b * pages * 4 + (ctx * 4 if fog else 0)


def read_traffic(kernel: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE/WRITE_SIZE),
    scaled by the copy-kernel calibration; from profiles/hbm_traffic.txt."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for ln in open(path):
        parts = ln.split()
        if len(parts) >= 2 and parts[0] == kernel and not ln.startswith("#"):
            try:
                return float(parts[1])
            except ValueError:
                return None
    return None


# ---------------------------------------------------------------------------
# Primary: bf16 decode @128K
# ---------------------------------------------------------------------------
def setup_decode(dev, b=16, hq=32, hkv=8, d=128, ctx=131072, page_size=16, dtype=None, seed=0):
    import torch

    from kessie_amd import ops

    dtype = dtype or torch.bfloat16
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn(b, hq, d, generator=g, device=dev, dtype=torch.float32).to(dtype)
    pages = (ctx + page_size - 1) // page_size
    n_pages = b * pages
    pool = torch.empty(n_pages, page_size, 2, hkv, d, device=dev, dtype=dtype)
    chunk = 4096
    for p0 in range(0, n_pages, chunk):  # K and V ~ N(0,1), generated chunk by chunk
        p1 = min(n_pages, p0 + chunk)
        pool[p0:p1] = torch.randn(p1 - p0, page_size, 2, hkv, d, generator=g, device=dev).to(dtype)
    g1 = torch.Generator(device=dev)
    g1.manual_seed(seed + 1)
    table = torch.randperm(n_pages, generator=g1, device=dev).to(torch.int32).view(b, pages).contiguous()
    lens = torch.full((b,), ctx, dtype=torch.int32, device=dev)
    # Fog weights: the reference's kessie_build_fog_weights(ctx, 0.5, 0.5), built on the device.
    c = int(ctx * 0.5)
    fog = torch.ones(ctx, dtype=torch.float32, device=dev)
    fog[:c] = (torch.arange(c, dtype=torch.float32, device=dev) / max(c - 1, 1)).pow(0.5)
    nbytes = ws_bytes = 0
    from kessie_amd import _lib

    ws_bytes = _lib.load().kessie_fog_decode_workspace_bytes(b, hq, hkv, d, ctx, page_size, ops.dtype_code(dtype))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)
    nbytes = decode_bytes(b, ctx, hq, hkv, d, q.element_size(), page_size)
    return dict(q=q, pool=pool, table=table, lens=lens, fog=fog, ws=ws, out=out, ctx=ctx, hkv=hkv,
                page_size=page_size, bytes=nbytes, b=b, hq=hq, d=d)


def run_decode_step(s):
    """One decode step through the serving entry point (ops.fog_decode ->
    kessie_fog_decode_paged: the streaming kernel, with the split layout it
    chooses for the batch, then the split combine)."""
    from kessie_amd import ops

    ops.fog_decode(s["q"], s["pool"], s["table"], s["lens"], s["ctx"], fog_vscale=s["fog"], out=s["out"], ws=s["ws"])


def run_partials_combine(s):
    """The same decode as the two halves of the C ABI (kessie_fog_decode_partials
    + kessie_fog_decode_combine: the plain split layout)."""
    from kessie_amd import ops

    ops.fog_decode_partials(s["q"], s["pool"], s["table"], s["lens"], s["ctx"], s["ws"], fog_vscale=s["fog"])
    ops.fog_decode_combine(s["ws"], s["out"], s["hkv"], s["ctx"], s["page_size"])


def time_decode(s, steps, warmup):
    """(ms per serving step, ms of the streaming kernel alone, ms per
    partials + combine step)."""
    import torch

    from kessie_amd import ops

    preheat(lambda: run_decode_step(s))
    for _ in range(warmup):
        run_decode_step(s)
        run_partials_combine(s)
    torch.cuda.synchronize()
    # The steps: K decodes back to back between two events, nothing else in
    # the stream (an event pair around each launch would add its dispatch and
    # completion, ~2-3 us, to every step).
    start, end = events(2)
    backlog()
    start.record()
    for _ in range(steps):
        run_decode_step(s)
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    # The streaming kernel alone: K launches of the partials half, an event
    # pair around each, on the stream they run on.
    e0, e1 = events(steps), events(steps)
    backlog()
    for i in range(steps):
        e0[i].record()
        ops.fog_decode_partials(s["q"], s["pool"], s["table"], s["lens"], s["ctx"], s["ws"], fog_vscale=s["fog"])
        e1[i].record()
        ops.fog_decode_combine(s["ws"], s["out"], s["hkv"], s["ctx"], s["page_size"])
    torch.cuda.synchronize()
    kern = [a.elapsed_time(b) for a, b in zip(e0, e1)]
    # The two-call form back to back, for comparison with the serving entry.
    start, end = events(2)
    backlog()
    start.record()
    for _ in range(steps):
        run_partials_combine(s)
    end.record()
    torch.cuda.synchronize()
    return total_ms / steps, sum(kern) / len(kern), start.elapsed_time(end) / steps


def _cpu_median(fn, reps=3):
    """1 warm-up, then the median of ``reps`` timed calls (seconds)."""
    fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return sorted(ts)[len(ts) // 2]


def _cpu_threads():
    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def cpu_decode_baseline(s, budget_s=12.0):
    """The CPU oracle (oracle.attention.paged_decode_blockwise) on the host
    cores of the machine the bench runs on: whole sequences of the same
    workload until ~budget_s seconds."""
    import torch

    from oracle.attention import paged_decode_blockwise

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    fog = s["fog"].cpu()
    q = s["q"].cpu()
    table = s["table"]
    per_seq_bytes = s["bytes"] / s["b"]

    def seq_inputs(i):
        sub_pool = s["pool"][table[i].long()].cpu()
        sub_table = torch.arange(table.shape[1], dtype=torch.int32).view(1, -1)
        return sub_pool, sub_table

    p0, t0 = seq_inputs(0)
    paged_decode_blockwise(q[0:1], p0, t0, s["lens"][0:1].cpu(), fog)  # warm-up
    done, elapsed = 0, 0.0
    for i in range(1, s["b"]):
        pool_i, table_i = seq_inputs(i)
        t = time.perf_counter()
        paged_decode_blockwise(q[i:i + 1], pool_i, table_i, s["lens"][i:i + 1].cpu(), fog)
        elapsed += time.perf_counter() - t
        done += 1
        if elapsed >= budget_s:
            break
    return {
        "value": round(per_seq_bytes * done / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{done} of {s['b']} sequences x {s['ctx']} tokens (bf16 pages upcast to fp32, blockwise "
                  f"online softmax, torch {torch.__version__}, {platform.processor() or platform.machine()})",
        "seconds": round(elapsed, 2),
    }


# ---------------------------------------------------------------------------
# Secondary workloads
# ---------------------------------------------------------------------------
def bench_remap(dev, reps=20, sets=4, n_tok=65536, page_size=16, hkv=8, d=128, theta=500000.0, cpu=False,
                layout="native"):
    """RoPE remap, bf16, 65,536 tokens, 8 KV heads, D=128, theta 5e5, only K
    rotated.  ``layout``: "native" -- 16-token pages of interleaved K/V token
    rows [pages][16][2][8][128] (K is the first half of every 4 KiB row);
    "kv_first" -- 16-token K-only pages of vLLM's [2][blocks][16][8][128];
    "dense" -- the reference operator's own K tensor [T][8][128]
    (kessie_hip_kernels.py:443).  ``sets`` disjoint page sets (or tensors)
    rotate across reps so the 256 MB MALL cannot serve the next rep."""
    import torch

    from kessie_amd import ops

    pages = n_tok // page_size
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    if layout == "native":
        pool = torch.randn(pages * sets, page_size, 2, hkv, d, generator=g, device=dev).bfloat16()
    elif layout == "kv_first":
        pool = torch.randn(2, pages * sets, page_size, hkv, d, generator=g, device=dev).bfloat16()
    elif layout == "dense":
        dense = [torch.randn(n_tok, hkv, d, generator=g, device=dev).bfloat16() for _ in range(sets)]
    else:
        raise ValueError(layout)
    g1 = torch.Generator(device=dev)
    g1.manual_seed(1)
    perm = torch.randperm(pages * sets, generator=g1, device=dev).to(torch.int32)
    lists = [perm[i * pages:(i + 1) * pages].contiguous() for i in range(sets)]
    g2 = torch.Generator(device=dev)
    g2.manual_seed(2)
    orig = torch.randint(0, 1_000_000, (n_tok,), generator=g2, device=dev, dtype=torch.int32)
    g3 = torch.Generator(device=dev)
    g3.manual_seed(3)
    base = int(torch.randint(0, 1_000_000, (1,), generator=g3, device=dev).item())
    tgt = (base + torch.arange(n_tok, device=dev)).to(torch.int32)

    def run(i):
        if layout == "dense":
            ops.rope_remap_paged(dense[i % sets], orig, tgt, theta)
        else:
            ops.rope_remap_paged(pool, orig, tgt, theta, page_list=lists[i % sets], layout=layout)

    for i in range(3):
        run(i)
    torch.cuda.synchronize()
    mean_ms = time_back_to_back(run, reps)
    nbytes = 2 * n_tok * hkv * d * 2 + 2 * n_tok * 4 + (0 if layout == "dense" else pages * 4)
    achieved = nbytes / (mean_ms * 1e-3) / 1e9
    res_cpu = None
    if cpu:
        from oracle.rope import rope_remap_ref

        cores = _cpu_threads()
        if layout == "dense":
            k0 = dense[0].cpu()
        elif layout == "kv_first":
            k0 = pool[0][lists[0].long()].cpu().reshape(n_tok, hkv, d)
        else:
            k0 = pool[lists[0].long(), :, 0].cpu().reshape(n_tok, hkv, d)
        o_c, t_c = orig.cpu(), tgt.cpu()
        k = k0.clone()
        sec = _cpu_median(lambda: rope_remap_ref(k, o_c, t_c, theta))
        res_cpu = {"value": round(n_tok / sec / 1e6, 2), "unit": "Mtok/s", "cores": cores, "kind": "port",
                   "sample": f"the full workload ({n_tok} tokens, K [T, {hkv}, {d}] bf16"
                             + ("" if layout == "dense" else " gathered from the pages")
                             + f"), torch {torch.__version__}, 1 warm-up + median of 3"}
    where = {"native": f"in {page_size}-token pages of interleaved K/V rows",
             "kv_first": f"in {page_size}-token K-only pages ([2][blocks][{page_size}][{hkv}][{d}])",
             "dense": f"as one dense K tensor [{n_tok}][{hkv}][{d}]"}[layout]
    return {
        "cpu_baseline": res_cpu,
        "workload": f"RoPE remap bf16, {n_tok} tokens {where}, {hkv} KV heads, D={d}, theta {theta:g}, K only, "
                    f"{sets} rotating {'tensors' if layout == 'dense' else 'page sets'}",
        "mtok_s": round(n_tok / (mean_ms * 1e-3) / 1e6, 1),
        "kernel_ms_mean": round(mean_ms, 5),
        "timing": f"{reps} launches back to back between two events",
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": {"native": read_traffic("rope_remap_vec"),
                                 "dense": read_traffic("rope_remap_vec_dense_k")}.get(layout),
                     "algorithmic_bytes": nbytes},
    }


def bench_gather_evict(dev, reps=5, cpu=False):
    """Paged-KV gather + eviction: 65,536-page pool (1,048,576 tokens, 16-token
    pages, 8 KV heads x D=128 bf16), 64 sequences x 1,024 pages (random
    tables), per-page scores ~ U(0,1); evict the lowest 25%, compact the
    tables, gather the survivors' pages."""
    import torch

    from kessie_amd import ops

    num_pages, s, w = 65536, 64, 1024
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    pool = torch.randn(num_pages, 16, 2, 8, 128, generator=g, device=dev).bfloat16()
    g1 = torch.Generator(device=dev)
    g1.manual_seed(1)
    tables = torch.randperm(num_pages, generator=g1, device=dev).to(torch.int32).view(s, w).contiguous()
    g2 = torch.Generator(device=dev)
    g2.manual_seed(2)
    scores = torch.rand(num_pages, generator=g2, device=dev)
    lens = torch.full((s,), w, dtype=torch.int32, device=dev)
    valid = torch.ones(num_pages, dtype=torch.int8, device=dev)
    out = torch.empty(s * w, 16, 2, 8, 128, dtype=torch.bfloat16, device=dev)
    ev_list = torch.empty(num_pages, dtype=torch.int32, device=dev)
    ev_cnt = torch.zeros(1, dtype=torch.int32, device=dev)
    nt = torch.empty_like(tables)
    nl = torch.empty(s, dtype=torch.int32, device=dev)
    gi = torch.empty(s * w, dtype=torch.int32, device=dev)
    gc = torch.zeros(1, dtype=torch.int32, device=dev)

    def pipeline(e_sel=None, e_gat=None):
        # Score eviction + table compaction fused (clear + one launch), then the gather.
        ops.page_evict_compact(scores, valid, tables, lens, -1, 0.25, ev_list, ev_cnt, nt, nl, gi, gc)
        if e_sel is not None:
            e_sel.record()
        ops.page_gather(pool, gi, gc, out=out, n=s * w)
        if e_gat is not None:
            e_gat.record()

    for _ in range(2):
        valid.fill_(1)
        pipeline()
    torch.cuda.synchronize()

    def heat():
        valid.fill_(1)
        pipeline()

    preheat(heat)
    e0, e1, e2 = events(reps), events(reps), events(reps)
    backlog()
    for i in range(reps):
        valid.fill_(1)
        e0[i].record()
        pipeline(e1[i], e2[i])
    torch.cuda.synchronize()
    tot = sum(a.elapsed_time(c) for a, c in zip(e0, e2)) / reps
    gat = sum(b.elapsed_time(c) for b, c in zip(e1, e2)) / reps
    survivors = int(gc.item())
    page_bytes = 16 * 2 * 8 * 128 * 2
    gather_bytes = 2 * survivors * page_bytes
    alg = gather_bytes + num_pages * 4 * 2 + s * w * 4 + survivors * 4 + int(ev_cnt.item()) * 4
    ach = gather_bytes / (gat * 1e-3) / 1e9
    res_cpu = None
    if cpu:
        import numpy as np

        from oracle.pages import compact, gather_pages, select_evict

        cores = _cpu_threads()
        sc, tb, ln = scores.cpu().numpy(), tables.cpu().numpy(), lens.cpu().numpy()
        pool_bytes = pool.view(torch.uint8).reshape(num_pages, -1).cpu().numpy()
        ones = np.ones(num_pages, dtype=np.int8)

        def cpu_pipeline():
            v, _ = select_evict(sc, ones, -1, 0.25)
            _, _, gidx = compact(tb, ln, v)
            gather_pages(pool_bytes, gidx)

        sec = _cpu_median(cpu_pipeline)
        res_cpu = {"value": round(gather_bytes / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
                   "sample": "the full workload (numpy select + compact + fancy-index gather of the survivors), "
                             "1 warm-up + median of 3; GB/s of gathered bytes over the whole pipeline",
                   "pipeline_ms": round(1000 * sec, 1)}
        del pool_bytes
    return {
        "cpu_baseline": res_cpu,
        "workload": "score evict 25% of 65,536 pages + compact 64x1024 tables (fused: 1 launch) + gather "
                    "survivors (bf16 pages)",
        "pipeline_ms": round(tot, 4),
        "gather_kernel_ms": round(gat, 4),
        "select_compact_ms": round(tot - gat, 4),
        "pipeline_gbs": round(alg / (tot * 1e-3) / 1e9, 1),
        "survivor_pages": survivors,
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": read_traffic("gather_kernel"),
                     "algorithmic_bytes": gather_bytes},
    }


def bench_prefill(dev, reps=3, c=2048, L=1 << 20, hq=32, hkv=8, d=128, cpu=False, cpu_L=8192):
    """Chunked prefill, bf16 on MFMA: a 2,048-query chunk appended to a
    1,048,576-token paged KV (65,664 pages, random table), 32 q / 8 kv heads,
    D=128, causal, V-fog over the full context."""
    import torch

    from kessie_amd import ops

    ctx = L + c
    n_pages = ctx // 16
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    q = torch.randn(1, c, hq, d, generator=g, device=dev).bfloat16()
    pool = torch.empty(n_pages, 16, 2, hkv, d, device=dev, dtype=torch.bfloat16)
    for p0 in range(0, n_pages, 8192):
        p1 = min(n_pages, p0 + 8192)
        pool[p0:p1] = torch.randn(p1 - p0, 16, 2, hkv, d, generator=g, device=dev).bfloat16()
    g1 = torch.Generator(device=dev)
    g1.manual_seed(1)
    table = torch.randperm(n_pages, generator=g1, device=dev).to(torch.int32).view(1, n_pages).contiguous()
    lens = torch.tensor([ctx], dtype=torch.int32, device=dev)
    cf = int(ctx * 0.5)
    fog = torch.ones(ctx, dtype=torch.float32, device=dev)
    fog[:cf] = (torch.arange(cf, dtype=torch.float32, device=dev) / max(cf - 1, 1)).pow(0.5)
    out = torch.empty_like(q)
    ops.fog_prefill(q, pool, table, lens, ctx, fog_vscale=fog, out=out)
    torch.cuda.synchronize()
    preheat(lambda: ops.fog_prefill(q, pool, table, lens, ctx, fog_vscale=fog, out=out))
    e0, e1 = events(reps), events(reps)
    backlog()
    for i in range(reps):
        e0[i].record()
        ops.fog_prefill(q, pool, table, lens, ctx, fog_vscale=fog, out=out)
        e1[i].record()
    torch.cuda.synchronize()
    ms = sum(a.elapsed_time(b) for a, b in zip(e0, e1)) / reps
    flops = 4 * d * hq * (c * L + c * (c + 1) // 2)
    tf = flops / (ms * 1e-3) / 1e12
    res_cpu = None
    if cpu:
        # The full context's score matrix does not fit host memory: the oracle
        # (blockwise online softmax) runs the same chunk on the last cpu_L
        # prior tokens, and the time is extrapolated linearly in FLOPs.
        from oracle.attention import paged_prefill_blockwise

        cores = _cpu_threads()
        ctx_s = cpu_L + c
        pages_s = ctx_s // 16
        tab_s = table[:, n_pages - pages_s:].contiguous()
        lens_s = torch.tensor([ctx_s], dtype=torch.int32)
        fog_s = fog[ctx - ctx_s:].cpu()
        q_c = q.cpu()
        rows = torch.arange(c)
        t = time.perf_counter()
        paged_prefill_blockwise(q_c, pool, tab_s.cpu(), lens_s, rows, fog_vscale=fog_s, block_pages=256)
        sec = time.perf_counter() - t
        flops_s = 4 * d * hq * (c * cpu_L + c * (c + 1) // 2)
        res_cpu = {"value": round(flops_s / sec / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
                   "sample": f"the same 2,048-query chunk over the last {cpu_L:,} prior tokens (fp32 blockwise "
                             f"online softmax, pages copied from the device per block), one timed call",
                   "seconds": round(sec, 2),
                   "extrapolated_full_ms": round(1000 * sec * flops / flops_s, 0)}
    return {"workload": "chunked prefill bf16: 2048 queries on a 1,048,576-token paged context, 32q/8kv, D=128, "
                        "causal, V-fog", "ms": round(ms, 3), "tflops": round(tf, 1), "cpu_baseline": res_cpu,
            "roofline": {"bound": "mfma", "kernel": "prefill_mfma_kernel", "achieved": round(tf, 1),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                         "traffic": read_traffic("prefill_mfma_kernel"), "algorithmic_flops": flops}}


def bench_dense(dev, reps=3, b=1, h=32, n=8192, d=128, cpu=False, cpu_heads=4):
    """The reference's dense launcher launch_kessie_fused_fog_attn through
    KeSSieKernels.fused_fog_attention: fp16 [B, H, N, D] with every position a
    query, causal, V rows scaled by fog weights.  D=128 or 64 with H*N a
    multiple of 16 runs on the MFMA prefill kernel with table-less pages."""
    import torch

    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    g = torch.Generator(device=dev)
    g.manual_seed(3)
    q, k, v = (torch.randn(b, h, n, d, generator=g, device=dev).half() for _ in range(3))
    cf = n // 2
    w = torch.ones(n, dtype=torch.float32, device=dev)
    w[:cf] = (torch.arange(cf, dtype=torch.float32, device=dev) / max(cf - 1, 1)).pow(0.5)
    kk = KeSSieKernels()
    s = torch.cuda.current_stream()
    kk.fused_fog_attention(q, k, v, w, stream=s)
    torch.cuda.synchronize()
    preheat(lambda: kk.fused_fog_attention(q, k, v, w, stream=s))
    e0, e1 = events(reps), events(reps)
    backlog()
    for i in range(reps):
        e0[i].record()
        kk.fused_fog_attention(q, k, v, w, stream=s)
        e1[i].record()
    torch.cuda.synchronize()
    ms = sum(a.elapsed_time(b_) for a, b_ in zip(e0, e1)) / reps
    flops = b * h * 4 * d * (n * (n + 1) // 2)
    tf = flops / (ms * 1e-3) / 1e12
    res_cpu = None
    if cpu:
        from oracle.attention import fused_fog_attention_ref

        cores = _cpu_threads()
        qc, kc, vc = (x[:1, :cpu_heads].float().cpu() for x in (q, k, v))
        wc = w.cpu()
        t = time.perf_counter()
        fused_fog_attention_ref(qc, kc, vc, wc)
        sec = time.perf_counter() - t
        flops_s = cpu_heads * 4 * d * (n * (n + 1) // 2)
        res_cpu = {"value": round(flops_s / sec / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
                   "sample": f"{cpu_heads} of the {h} heads (fp32 dense oracle: scores, causal mask, softmax, "
                             f"@ V*w), one timed call", "seconds": round(sec, 2)}
    return {"workload": f"dense fused fog attention fp16 (reference launcher), B={b} H={h} N={n:,} D={d}, causal",
            "ms": round(ms, 3), "tflops": round(tf, 1), "cpu_baseline": res_cpu,
            "roofline": {"bound": "mfma", "kernel": "prefill_mfma_kernel (table-less pages)", "achieved": round(tf, 1),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                         "traffic": None, "algorithmic_flops": flops}}


def bench_dense_reference_sweep(dev, reps=20, cpu=False):
    """The reference's own benchmark of its dense launcher
    (kessie_kernels_v2.hip:961-1004): launch_kessie_windowed_attn, fp16,
    B=1, H=8, D=128, N = 512 ... 8,192, causal, full and W=1024.  Calls back
    to back between two events (the reference times 20 calls between host
    clocks).  FLOPs = 4 * D * H * (query, visible key) pairs."""
    import ctypes

    import torch

    from kessie_amd import _lib

    lib = _lib.load()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    rows = []
    for n in (512, 1024, 2048, 4096, 8192):
        q, k, v = (torch.randn(1, 8, n, 128, generator=g, device=dev).half() for _ in range(3))
        o = torch.empty_like(q)
        ptr = lambda t: ctypes.c_void_p(t.data_ptr())
        entry = {"N": n}
        for w in (0, 1024):
            call = lambda i: lib.launch_kessie_windowed_attn(ptr(q), ptr(k), ptr(v), ptr(o), ctypes.c_float(128 ** -0.5),
                                                             1, 8, n, 128, w, 1, st)
            for _ in range(3):
                call(0)
            torch.cuda.synchronize()
            status, msg = _lib.last_error()
            if status != _lib.OK:
                raise RuntimeError(msg)
            ms = time_back_to_back(call, reps)
            pairs = sum(min(i + 1, w) if w else i + 1 for i in range(n))
            tf = 4.0 * 128 * 8 * pairs / (ms * 1e-3) / 1e12
            key = "full" if w == 0 else "w1024"
            entry[f"{key}_us"] = round(1000 * ms, 1)
            entry[f"{key}_tflops"] = round(tf, 1)
        rows.append(entry)
    big = rows[-1]
    pairs8k = 8192 * 8193 // 2
    res_cpu = None
    if cpu:
        from oracle.attention import windowed_attention_ref

        cores = _cpu_threads()
        qc, kc, vc = (torch.randn(1, 8, 2048, 128, generator=torch.Generator().manual_seed(5)) for _ in range(3))
        sec = _cpu_median(lambda: windowed_attention_ref(qc, kc, vc, 0, True))
        res_cpu = {"value": round(4.0 * 128 * 8 * (2048 * 2049 // 2) / sec / 1e12, 4), "unit": "TFLOP/s",
                   "cores": cores, "kind": "port",
                   "sample": "N=2,048 of the sweep (fp32 dense oracle: scores, causal mask, softmax, @ V), "
                             "1 warm-up + median of 3", "seconds": round(sec, 3)}
    return {"workload": "reference dense-launcher benchmark: launch_kessie_windowed_attn fp16, B=1 H=8 D=128, "
                        "causal, full and W=1024, N=512..8192",
            "sweep": rows, "cpu_baseline": res_cpu,
            "roofline": {"bound": "mfma", "kernel": "prefill_mfma_kernel (table-less pages, key splits) + combine",
                         "shape": "N=8192 full", "achieved": big["full_tflops"], "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(big["full_tflops"] / BF16_PEAK_TFLOPS, 4), "traffic": None,
                         "algorithmic_flops": 4 * 128 * 8 * pairs8k}}


def bench_decode_fp32(dev, reps=20, cpu=False):
    """Fog decode on the reference CPU path's shape, fp32: B=1, 32q/8kv, D=128,
    4,096-token context in 16-token pages."""
    import torch

    from kessie_amd import ops

    s = setup_decode(dev, b=1, ctx=4096, dtype=torch.float32)
    for _ in range(3):
        run_decode_step(s)
    torch.cuda.synchronize()
    ms = time_back_to_back(lambda i: run_decode_step(s), reps)  # steps back to back, as the headline's
    # The streaming kernel alone (decode_f32_4x4_kernel), K launches back to
    # back: at ~16 us an event pair around each launch would add its dispatch.
    ms_kern = time_back_to_back(lambda i: ops.fog_decode_partials(s["q"], s["pool"], s["table"], s["lens"], s["ctx"],
                                                                   s["ws"], fog_vscale=s["fog"]), reps)
    res_cpu = None
    if cpu:
        from oracle.attention import paged_decode_ref

        cores = _cpu_threads()
        q_c, pool_c, tab_c, lens_c, fog_c = (s["q"].cpu(), s["pool"].cpu(), s["table"].cpu(), s["lens"].cpu(),
                                             s["fog"].cpu())
        sec = _cpu_median(lambda: paged_decode_ref(q_c, pool_c, tab_c, lens_c, fog_c))
        res_cpu = {"value": round(s["bytes"] / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
                   "sample": "the full workload (fp32 paged decode oracle), 1 warm-up + median of 3",
                   "ms": round(1000 * sec, 3)}
    ach = s["bytes"] / (ms_kern * 1e-3) / 1e9
    return {"workload": "fog decode fp32, B=1, 32q/8kv, D=128, 4096-token context",
            "ms": round(ms, 5), "gbs": round(s["bytes"] / (ms * 1e-3) / 1e9, 1), "cpu_baseline": res_cpu,
            "kernel_ms": round(ms_kern, 5),
            "roofline": {"bound": "hbm", "kernel": "decode_f32_4x4_kernel", "achieved": round(ach, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                         "traffic": read_traffic("decode_f32_4x4_kernel"), "algorithmic_bytes": s["bytes"],
                         "timing": "20 launches of the streaming kernel back to back between two events"}}


def bench_decode_ragged(dev, reps=20, cpu=False, lens=None):
    """Fog decode over a ragged batch through the fused entry point
    (kessie_fog_decode_paged: split kernel + combine): B=16, 32q/8kv, D=128,
    bf16, two 131,072-token and fourteen 4,096-token sequences in 16-token
    pages, V-fog over the longest context.  Bytes: every sequence's K and V,
    q and out, its page-table entries and the shared fog vector once."""
    import torch

    from kessie_amd import _lib, ops

    lens = lens or [131072] * 2 + [4096] * 14
    b, hq, hkv, d, ps = len(lens), 32, 8, 128, 16
    max_ctx = max(lens)
    width = (max_ctx + ps - 1) // ps
    pages = [(c + ps - 1) // ps for c in lens]
    n_pages = sum(pages)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    q = torch.randn(b, hq, d, generator=g, device=dev).to(torch.bfloat16)
    pool = torch.empty(n_pages, ps, 2, hkv, d, device=dev, dtype=torch.bfloat16)
    for p0 in range(0, n_pages, 4096):
        p1 = min(n_pages, p0 + 4096)
        pool[p0:p1] = torch.randn(p1 - p0, ps, 2, hkv, d, generator=g, device=dev).to(torch.bfloat16)
    perm = torch.randperm(n_pages, generator=g, device=dev).to(torch.int32)
    table = torch.full((b, width), -1, dtype=torch.int32, device=dev)
    off = 0
    for i, n in enumerate(pages):
        table[i, :n] = perm[off:off + n]
        off += n
    ctx_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
    c = int(max_ctx * 0.5)
    fog = torch.ones(max_ctx, dtype=torch.float32, device=dev)
    fog[:c] = (torch.arange(c, dtype=torch.float32, device=dev) / max(c - 1, 1)).pow(0.5)
    out = torch.empty_like(q)
    need = _lib.load().kessie_fog_decode_workspace_bytes(b, hq, hkv, d, max_ctx, ps, ops.dtype_code(q.dtype))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    for _ in range(3):
        ops.fog_decode(q, pool, table, ctx_lens, max_ctx, fog_vscale=fog, out=out, ws=ws)
    torch.cuda.synchronize()
    # steps back to back, as the headline's
    ms = time_back_to_back(lambda i: ops.fog_decode(q, pool, table, ctx_lens, max_ctx, fog_vscale=fog, out=out, ws=ws),
                           reps)
    nbytes = sum(lens) * hkv * d * 2 * 2 + 2 * b * hq * d * 2 + n_pages * 4 + max_ctx * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    res_cpu = None
    if cpu:
        from oracle.attention import paged_decode_blockwise

        cores = _cpu_threads()
        q_c, fog_c = q.cpu(), fog.cpu()
        sec = 0.0
        for i in range(b):  # each sequence's pages gathered to host memory first, outside the timing
            sub = pool[table[i, :pages[i]].long()].cpu()
            sub_table = torch.arange(pages[i], dtype=torch.int32).view(1, -1)
            t = time.perf_counter()
            paged_decode_blockwise(q_c[i:i + 1], sub, sub_table, ctx_lens[i:i + 1].cpu(), fog_c)
            sec += time.perf_counter() - t
            del sub
        res_cpu = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
                   "sample": "the full batch once (paged_decode_blockwise per sequence)", "seconds": round(sec, 2)}
    return {"workload": f"fog decode bf16 ragged batch {b}: " + ", ".join(
                f"{lens.count(v)} x {v}" for v in sorted(set(lens), reverse=True)) + " tokens, 32q/8kv, D=128",
            "ms": round(ms, 5), "gbs": round(gbs, 1), "algorithmic_bytes": nbytes,
            "roofline": {"bound": "hbm", "kernel": "decode_mfma_kernel + combine_kernel (step)",
                         "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
            "cpu_baseline": res_cpu}


def bench_fog_bias(dev, reps=50, kv_len=131072, n_recall=1000):
    """Fog logit bias of the serving path, bf16 over a 131,072-token context
    with 1,000 recalled positions (alpha 0.5, fog_start 0.5, boost 0.1): the
    device producer, and the reference's torch op sequence with its
    per-position recall writes on the host cores as the CPU baseline."""
    import torch

    from kessie_amd import ops

    g = torch.Generator().manual_seed(5)
    recall = torch.randperm(kv_len, generator=g)[:n_recall].to(torch.int32)
    rec_dev = recall.to(dev)
    buf = torch.empty(kv_len, dtype=torch.bfloat16, device=dev)
    ops.fog_bias_fill(buf, kv_len, 0.5, 0.5, rec_dev, 0.1)
    torch.cuda.synchronize()
    e0, e1 = events(reps), events(reps)
    backlog()
    for i in range(reps):
        e0[i].record()
        ops.fog_bias_fill(buf, kv_len, 0.5, 0.5, rec_dev, 0.1)
        e1[i].record()
    torch.cuda.synchronize()
    us = 1000.0 * sum(a.elapsed_time(b) for a, b in zip(e0, e1)) / reps
    from oracle.fog import fog_bias

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rl = recall.tolist()
    fog_bias(kv_len, 0.5, 0.5, rl, 0.1, dtype=torch.bfloat16)
    t0 = time.perf_counter()
    cpu_reps = 3
    for _ in range(cpu_reps):
        fog_bias(kv_len, 0.5, 0.5, rl, 0.1, dtype=torch.bfloat16)
    cpu_ms = 1000.0 * (time.perf_counter() - t0) / cpu_reps
    return {"workload": "fog bias bf16, 131,072 positions, 1,000 recalled positions", "us": round(us, 2),
            "launches": 1, "cpu_baseline": {"value": round(cpu_ms, 3), "unit": "ms", "cores": cores,
                                            "kind": "port", "sample": "the full vector, 3 reps"}}


def bench_recall_inject(dev, reps=20, n_tok=65536, hkv=8, d=128, theta=500000.0, cpu=False):
    """Recall-inject: 65,536 recalled tokens (K and V, bf16, 8 kv heads,
    head_dim 128) already staged in HBM written into 4,096 random pages of an
    8,192-page pool with K re-rotated from its original to its new positions
    (fused insert + RoPE remap); also the pinned host-to-device rate of the
    staging copy that precedes it."""
    import torch

    from kessie_amd import ops

    n_pages = 2 * n_tok // 16
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    pool = torch.randn(n_pages, 16, 2, hkv, d, generator=g, device=dev).bfloat16()
    new_k = torch.randn(n_tok, hkv, d, generator=g, device=dev).bfloat16()
    new_v = torch.randn(n_tok, hkv, d, generator=g, device=dev).bfloat16()
    g.manual_seed(1)
    tgt_pages = torch.randperm(n_pages, generator=g, device=dev)[: n_tok // 16].to(torch.int32)
    orig = torch.randint(0, 1_000_000, (n_tok,), generator=g, device=dev, dtype=torch.int32)
    tgt = torch.arange(n_tok, dtype=torch.int32, device=dev)
    valid = torch.zeros(n_pages, dtype=torch.int8, device=dev)
    positions = torch.zeros(n_pages, dtype=torch.int32, device=dev)

    def run():
        ops.page_insert(pool, new_k, new_v, tgt_pages, valid, positions, 0, orig_pos=orig, tgt_pos=tgt,
                        rope_theta=theta)

    run()
    torch.cuda.synchronize()
    ms = time_back_to_back(lambda i: run(), reps)
    kv_bytes = n_tok * hkv * d * 2
    nbytes = 4 * kv_bytes + 2 * 4 * n_tok + 4 * (n_tok // 16)
    gbs = nbytes / (ms * 1e-3) / 1e9
    host = torch.empty(2, n_tok, hkv, d, dtype=torch.bfloat16, pin_memory=True)
    stage = torch.empty(2, n_tok, hkv, d, dtype=torch.bfloat16, device=dev)
    stage.copy_(host, non_blocking=True)
    torch.cuda.synchronize()
    h0, h1 = events(1)[0], events(1)[0]
    h0.record()
    for _ in range(5):
        stage.copy_(host, non_blocking=True)
    h1.record()
    torch.cuda.synchronize()
    h2d = 5 * 2 * kv_bytes / (h0.elapsed_time(h1) * 1e-3) / 1e9
    res_cpu = None
    if cpu:
        from oracle.pages import page_insert
        from oracle.rope import rope_remap_ref

        cores = _cpu_threads()
        pool_c = pool.cpu().view(torch.int16).numpy()
        k_c, v_c = new_k.cpu(), new_v.cpu().view(torch.int16).numpy()
        o_c, t_c, pages_c = orig.cpu(), tgt.cpu(), tgt_pages.cpu().numpy()
        valid_c, pos_c = valid.cpu().numpy(), positions.cpu().numpy()

        def cpu_inject():
            k = k_c.clone()
            rope_remap_ref(k, o_c, t_c, theta)
            page_insert(pool_c, k.view(torch.int16).numpy(), v_c, pages_c, valid_c, pos_c, 0)

        sec = _cpu_median(cpu_inject)
        res_cpu = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
                   "sample": "the full workload (torch remap of K, then the per-token page insert), 1 warm-up + "
                             "median of 3", "ms": round(1000 * sec, 1)}
    return {"workload": "recall-inject: 65,536 tokens K+V bf16 into 4,096 random pages with fused RoPE remap "
                        "(theta 5e5)", "ms": round(ms, 4), "gbs": round(gbs, 1),
            "roofline": {"bound": "hbm", "kernel": "insert_vec_kernel", "achieved": round(gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": read_traffic("insert_vec_kernel"), "algorithmic_bytes": nbytes},
            "h2d_pinned_gbs": round(h2d, 1), "cpu_baseline": res_cpu}


def bench_index_query(dev, reps=50, n=78125, d=256, k=5):
    """Semantic index query: cosine scan of 78,125 fp32 embeddings of width
    256 (10M tokens at 128-token granularity) plus the exact top-5, matrix
    resident in HBM; the CPU baseline is the reference's numpy search step
    (matrix-vector product + argsort) on the host cores."""
    import torch

    from kessie_amd import ops

    g = torch.Generator(device=dev)
    g.manual_seed(0)
    # Four 80 MB matrices, one per rep in turn: 320 MB, more than the 256 MB
    # MALL, so no rep finds the matrix left in it by the previous one.
    mats = [torch.randn(n, d, generator=g, device=dev) for _ in range(4)]
    mat = mats[0]
    q = torch.randn(d, generator=g, device=dev)

    def timed(top_k):
        ops.index_query(mat, q, top_k=top_k, norm_mode=2)
        torch.cuda.synchronize()
        return 1000.0 * time_back_to_back(lambda i: ops.index_query(mats[i % 4], q, top_k=top_k, norm_mode=2), reps)

    us = timed(k)  # scan with each wave's top-k + one merge launch
    scan_us = timed(0)  # the similarities alone (cosine_scan_kernel, no top-k)
    nbytes = n * d * 4 + n * 4
    from oracle.index import numpy_search_step

    m = mat.cpu().numpy()
    m = m / np.maximum(np.linalg.norm(m, axis=1, keepdims=True), 1e-8)
    qn = q.cpu().numpy()
    qn = qn / np.linalg.norm(qn)
    numpy_search_step(m, qn, k)
    t0 = time.perf_counter()
    cpu_reps = 20
    for _ in range(cpu_reps):
        numpy_search_step(m, qn, k)
    cpu_ms = 1000.0 * (time.perf_counter() - t0) / cpu_reps
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"workload": "index query: 78,125 x 256 fp32 embeddings, cosine scan + top-5", "us": round(us, 2),
            "launches": 2, "scan_only_us": round(scan_us, 2),
            "roofline": {"bound": "hbm", "kernel": "scan_topk_kernel + topk_merge_kernel (the whole query)",
                         "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": read_traffic("scan_topk_kernel"),
                         "algorithmic_bytes": nbytes},
            "cpu_baseline": {"value": round(cpu_ms, 3), "unit": "ms", "cores": len(os.sched_getaffinity(0)),
                             "kind": "port", "sample": "numpy matrix-vector product + argsort, 20 reps"}}


def bench_hf_cache(dev, layers=32, heads=8, d=128, window=4096, prefill=8000, steps=50):
    """HF tiered cache (KeSSieCache) decode steps: 32 layers x (append one
    token, return K and the fog-weighted V over the ~8K-token window), bf16, 8
    kv heads, head_dim 128, window_size 4096 (no eviction in the timed steps);
    plus the fused append + fog launch alone over an 8,192-token window (its
    HBM roofline).  CPU baseline: the reference's torch.cat / fog op sequence on
    the host cores for 2 steps."""
    import torch

    from kessie_amd import ops
    from kessie_amd.hf_cache import KeSSieCache

    g = torch.Generator(device=dev)
    g.manual_seed(0)
    cache = KeSSieCache(window_size=window)
    kv0 = torch.randn(1, heads, prefill, d, generator=g, device=dev).bfloat16()
    for li in range(layers):
        cache.update(kv0, kv0, li)
    tok = torch.randn(1, heads, 1, d, generator=g, device=dev).bfloat16()
    for li in range(layers):
        cache.update(tok, tok, li)
    torch.cuda.synchronize()
    e0, e1 = events(1)[0], events(1)[0]
    e0.record()
    for _ in range(steps):
        for li in range(layers):
            cache.update(tok, tok, li)
    e1.record()
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    # The fused per-layer launch alone: append one token to an 8,191-token
    # window and write the fogged V of all 8,192 tokens.
    # Eight arenas in turn (8 x ~50 MB, more than the 256 MB MALL), so no
    # launch finds its window left in the MALL by the previous one.
    n, sets = 8192, 8
    arenas = [(torch.randn(1, heads, n + 64, d, generator=g, device=dev).bfloat16(),
               torch.randn(1, heads, n + 64, d, generator=g, device=dev).bfloat16(),
               torch.empty(1, heads, n, d, dtype=torch.bfloat16, device=dev)) for _ in range(sets)]

    def fused(i):
        k_ar, v_ar, vf = arenas[i % sets]
        ops.hf_append_fog(k_ar, v_ar, 0, n - 1, tok, tok, vf, 0.5, 0.5)

    for i in range(sets):
        fused(i)
    torch.cuda.synchronize()
    reps = 48
    fog_us = 1000.0 * time_back_to_back(fused, reps)
    row = heads * d * 2
    fog_bytes = (n - 1) * row + 2 * row + 2 * row + n * row  # read V window + new K/V, write new K/V + V'
    fog_gbs = fog_bytes / (fog_us * 1e-6) / 1e9
    from oracle.hf_cache import HFCacheModel

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    model = HFCacheModel(window_size=window)
    kc = kv0.cpu()
    for li in range(layers):
        model.update(kc, kc, li)
    tc = tok.cpu()
    t0 = time.perf_counter()
    for _ in range(2):
        for li in range(layers):
            model.update(tc, tc, li)
    cpu_ms = 1000.0 * (time.perf_counter() - t0) / 2
    return {"workload": "HF tiered cache decode step: 32 layers, bf16, 8 kv heads, D=128, ~8K-token window "
                        "(window_size 4096), K + fog-weighted V returned per layer",
            "step_ms": round(step_ms, 4), "per_layer_us": round(1000.0 * step_ms / layers, 2),
            "append_fog_8k_us": round(fog_us, 2),
            "roofline": {"bound": "hbm", "kernel": "hf_append_fog_kernel", "achieved": round(fog_gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(fog_gbs / HBM_PEAK_GBS, 4),
                         "traffic": read_traffic("hf_append_fog_kernel"), "algorithmic_bytes": fog_bytes},
            "cpu_baseline": {"value": round(cpu_ms, 2), "unit": "ms per step", "cores": cores, "kind": "port",
                             "sample": "2 decode steps of the reference's torch.cat / fog op sequence"}}


def load_probes():
    """libkessie_probes.so (measurement-only HBM ceiling probes, built beside
    the product library by kessie_amd.build; declared in include/kessie_probes.h)."""
    import ctypes as C

    from kessie_amd import build as kbuild

    if not os.path.exists(kbuild.PROBES_LIB_PATH):
        raise FileNotFoundError(f"{kbuild.PROBES_LIB_PATH} is not built (python -m kessie_amd.build)")
    lib = C.CDLL(kbuild.PROBES_LIB_PATH)
    P, I, I64 = C.c_void_p, C.c_int, C.c_int64
    lib.kessie_probe_stream_read.argtypes = [P, I64, P, P]
    lib.kessie_probe_copy.argtypes = [P, P, I64, P]
    lib.kessie_probe_page_rows.argtypes = [P, P, I64, I64, I, I, P, I, I, I, P, P]
    for fn in (lib.kessie_probe_stream_read, lib.kessie_probe_copy, lib.kessie_probe_page_rows):
        fn.restype = I
    return lib


def bench_hbm_ceilings(dev, reps=10):
    """Practical HBM ceilings of the hot path's access patterns on this device
    (libkessie_probes.so): a 4 GiB read-only stream (the decode kernel's
    pattern at its best), a 2 GiB copy (gather, insert), and a matrix of page
    patterns around the RoPE remap's (read and rewrite the 2 KiB K half of
    every 4 KiB token row of 4,096 random 64 KiB pages, 4 rotating page sets
    so the 256 MB MALL does not serve it): whole rows instead of half rows,
    out of place instead of in place, pages in ascending id order, the V half
    instead of the K half, whole pages copied out of place, and half / whole
    rows only read; each at 1, 2, 4 and 8 sixteen-byte chunks per thread (8 =
    one page's K half per workgroup, all read before any write).  GB/s count
    the bytes read plus the bytes written."""
    import ctypes as C

    import torch

    lib = load_probes()
    s = C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def check(name, st):
        if st != 0:
            raise RuntimeError(f"{name} returned {st}")

    def timed(fn, n):
        fn(0)
        torch.cuda.synchronize()
        a, b = events(n), events(n)
        backlog()
        for i in range(n):
            a[i].record()
            fn(i)
            b[i].record()
        torch.cuda.synchronize()
        return sum(x.elapsed_time(y) for x, y in zip(a, b)) / n

    out = {}
    big = torch.empty(4 << 30, dtype=torch.uint8, device=dev)
    big.fill_(1)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    ms = timed(lambda i: check("stream_read", lib.kessie_probe_stream_read(
        C.c_void_p(big.data_ptr()), big.numel(), C.c_void_p(sink.data_ptr()), s)), reps)
    out["stream_read_gbs"] = round(big.numel() / (ms * 1e-3) / 1e9, 1)
    half = big.numel() // 2
    ms = timed(lambda i: check("copy", lib.kessie_probe_copy(
        C.c_void_p(big.data_ptr() + half), C.c_void_p(big.data_ptr()), half, s)), reps)
    out["copy_gbs"] = round(2 * half / (ms * 1e-3) / 1e9, 1)
    del big
    torch.cuda.empty_cache()
    n_pages, sets = 4096, 4
    pool = torch.zeros(n_pages * sets * 2, 16, 2, 8, 128, dtype=torch.bfloat16, device=dev)
    dst = torch.zeros_like(pool)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    lists = [torch.randperm(pool.shape[0], generator=g, device=dev)[:n_pages].to(torch.int32) for _ in range(sets)]
    sorted_lists = [torch.sort(x)[0].contiguous() for x in lists]
    page_bytes = pool[0].numel() * 2
    # name -> (byte offset in the page, destination (None: read only), row stride, rows per page,
    #          bytes per row, page lists)
    variants = {
        "remap_pattern_rmw": (0, pool, 4096, 16, 2048, lists),
        "full_row_rmw": (0, pool, 4096, 16, 4096, lists),
        "half_row_out_of_place": (0, dst, 4096, 16, 2048, lists),
        "half_row_rmw_sorted_pages": (0, pool, 4096, 16, 2048, sorted_lists),
        "v_half_row_rmw": (2048, pool, 4096, 16, 2048, lists),
        "whole_page_out_of_place": (0, dst, page_bytes, 1, page_bytes, lists),
        "half_row_read_only": (0, None, 4096, 16, 2048, lists),
        "full_row_read_only": (0, None, 4096, 16, 4096, lists),
    }
    matrix = {}
    for name, (off, target, stride, rows, row_bytes, pl) in variants.items():
        moved = (2 if target is not None else 1) * n_pages * rows * row_bytes
        row = {}
        for u in (1, 2, 4, 8):
            ms = timed(lambda i: check("page_rows", lib.kessie_probe_page_rows(
                C.c_void_p(pool.data_ptr() + off), None if target is None else C.c_void_p(target.data_ptr() + off),
                page_bytes, stride, rows, row_bytes, C.c_void_p(pl[i % sets].data_ptr()), n_pages, pool.shape[0], u,
                C.c_void_p(sink.data_ptr()), s)), 4 * reps)
            row[f"u{u}"] = round(moved / (ms * 1e-3) / 1e9, 1)
        row["best_gbs"] = max(row.values())
        matrix[name] = row
        log(f"ceilings: {name} {row}")
    out["remap_pattern_rmw_gbs"] = matrix["remap_pattern_rmw"]["best_gbs"]
    out["page_pattern_matrix_gbs"] = matrix
    out["note"] = ("bandwidth of the access pattern alone, no arithmetic (bytes read + written per second); "
                   "spec peak 8000 GB/s")
    return out


def pmc_run(dev) -> None:
    """A short fixed sequence of launches for hardware-counter passes
    (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE): a 1 GiB device copy of
    known size (the calibration kernel), then one decode (bf16 B=16 128K, then
    fp32 B=1 4K, each as partials + combine), one remap in
    interleaved pages and one on a dense K tensor, one gather + evict
    pipeline, one recall-inject, one index query, one HF append + fog launch
    and one chunked prefill of the bench workloads."""
    import torch

    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    src.fill_(3)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    s = setup_decode(dev)
    run_partials_combine(s)
    torch.cuda.synchronize()
    del s
    torch.cuda.empty_cache()
    s = setup_decode(dev, b=1, ctx=4096, dtype=torch.float32)
    run_partials_combine(s)
    torch.cuda.synchronize()
    del s
    torch.cuda.empty_cache()
    bench_remap(dev, reps=1, sets=1)
    torch.cuda.empty_cache()
    bench_remap(dev, reps=1, sets=1, layout="dense")
    torch.cuda.empty_cache()
    bench_gather_evict(dev, reps=1)
    torch.cuda.empty_cache()
    bench_recall_inject(dev, reps=1)
    torch.cuda.empty_cache()
    bench_index_query(dev, reps=1)
    from kessie_amd import ops

    v = torch.randn(1, 8, 8192 + 64, 128, device=dev).bfloat16()
    k = torch.randn_like(v)
    tok = torch.randn(1, 8, 1, 128, device=dev).bfloat16()
    ops.hf_append_fog(k, v, 0, 8191, tok, tok, torch.empty(1, 8, 8192, 128, dtype=v.dtype, device=dev), 0.5, 0.5)
    del v, k
    torch.cuda.empty_cache()
    bench_prefill(dev, reps=1)
    torch.cuda.synchronize()
    log("pmc run done")


# ---------------------------------------------------------------------------
SECONDARY = {
    "remap": bench_remap,
    "remap_dense": lambda dev, cpu=False: bench_remap(dev, cpu=cpu, layout="dense"),
    "remap_kv_first": lambda dev, cpu=False: bench_remap(dev, cpu=cpu, layout="kv_first"),
    "gather": bench_gather_evict,
    "fp32": bench_decode_fp32,
    "ragged": bench_decode_ragged,
    "prefill": bench_prefill,
    "dense": bench_dense,
    "dense64": lambda dev, cpu=False: bench_dense(dev, d=64, cpu=cpu),
    "dense_ref": bench_dense_reference_sweep,
    "fog_bias": bench_fog_bias,
    "recall": bench_recall_inject,
    "index": bench_index_query,
    "hf_cache": bench_hf_cache,
    "ceilings": bench_hbm_ceilings,
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-secondary", action="store_true", help="skip remap / gather / fp32 lines")
    ap.add_argument("--pmc-run", action="store_true",
                    help="only run the launch sequence used for rocprofv3 --pmc traffic passes")
    ap.add_argument("--only", choices=sorted(SECONDARY),
                    help="run one secondary workload and print its JSON (for profiling it alone)")
    args = ap.parse_args()
    if args.pmc_run:
        import torch

        global PREHEAT
        PREHEAT = False
        pmc_run(torch.device("cuda:0"))
        return
    if args.only:
        import torch

        print(json.dumps(SECONDARY[args.only](torch.device("cuda:0"))), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the hot path is built and measured on a single MI355X); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    import torch

    from kessie_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} CUs={props.multi_processor_count} lib={_lib.lib_path()}")

    log("setting up decode: B=16, 131072-token context, bf16")
    s = setup_decode(dev)
    torch.cuda.synchronize()
    log(f"timing decode: warmup {args.warmup}, steps {args.steps}")
    ms_step, ms_kern, ms_two = time_decode(s, args.steps, args.warmup)
    value = s["bytes"] / (ms_step * 1e-3) / 1e9
    achieved = s["bytes"] / (ms_kern * 1e-3) / 1e9
    log(f"decode: {ms_step:.4f} ms/step, partials kernel {ms_kern:.4f} ms, partials + combine {ms_two:.4f} ms, "
        f"{value:.1f} GB/s")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: q, K, V ~ N(0,1) (seed 0), random page tables (seed 1)",
        "config": {
            "workload": "fog-attention decode, bf16, batch 16, 32 query / 8 KV heads, head_dim 128, "
                        "131072-token context per sequence in 16-token pages, V-fog alpha 0.5 fog_start 0.5, "
                        "window 0; step = one kessie_fog_decode_paged call (streaming kernel + split combine)",
            "batch": 16, "ctx": 131072, "q_heads": 32, "kv_heads": 8, "head_dim": 128, "page_size": 16,
            "splits": _lib.load().kessie_fog_decode_num_splits(16, 8, 131072, 16),
            "algorithmic_bytes": s["bytes"],
        },
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic("decode_mfma_kernel"),
            "kernel": "decode_mfma_kernel", "kernel_ms": round(ms_kern, 5),
            "kernel_timing": "event pair around each of K launches of kessie_fog_decode_partials (the streaming "
                             "kernel alone, plain split layout), on the stream it runs on",
        },
        "partials_combine_ms_per_step": round(ms_two, 5),
        "device": {"name": props.name, "cus": props.multi_processor_count},
    }
    if not args.no_cpu:
        log("CPU baseline (oracle, host cores)")
        result["cpu_baseline"] = cpu_decode_baseline(s)
    else:
        result["cpu_baseline"] = None
    del s
    torch.cuda.empty_cache()
    if not args.no_secondary:
        sec = {}
        log("secondary: RoPE remap")
        sec["rope_remap"] = bench_remap(dev, cpu=not args.no_cpu)
        result["rope_remap_mtok_s"] = sec["rope_remap"]["mtok_s"]
        torch.cuda.empty_cache()
        log("secondary: RoPE remap, dense K tensor and K-only pages")
        sec["rope_remap_dense_k"] = bench_remap(dev, cpu=False, layout="dense")
        sec["rope_remap_dense_k"]["cpu_baseline"] = sec["rope_remap"]["cpu_baseline"]
        result["rope_remap_dense_k_mtok_s"] = sec["rope_remap_dense_k"]["mtok_s"]
        torch.cuda.empty_cache()
        sec["rope_remap_k_only_pages"] = bench_remap(dev, cpu=False, layout="kv_first")
        sec["rope_remap_k_only_pages"]["cpu_baseline"] = sec["rope_remap"]["cpu_baseline"]
        torch.cuda.empty_cache()
        log("secondary: gather + evict")
        sec["gather_evict"] = bench_gather_evict(dev, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        log("secondary: fp32 decode 4K")
        sec["decode_fp32_4k"] = bench_decode_fp32(dev, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        log("secondary: ragged-batch decode")
        sec["decode_ragged_2x128k_14x4k"] = bench_decode_ragged(dev, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        log("secondary: chunked prefill 2048 x 1M")
        sec["prefill_1m"] = bench_prefill(dev, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        log("secondary: dense fused fog attention (reference launcher)")
        sec["dense_fused_fog_8k"] = bench_dense(dev, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        log("secondary: dense fused fog attention, head_dim 64 (reference launcher)")
        sec["dense_fused_fog_8k_d64"] = bench_dense(dev, d=64, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        log("secondary: the reference's dense-launcher benchmark (B=1 H=8 D=128, N=512..8192)")
        sec["dense_reference_sweep"] = bench_dense_reference_sweep(dev, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        log("secondary: fog bias producer")
        sec["fog_bias_131k"] = bench_fog_bias(dev)
        log("secondary: recall inject")
        sec["recall_inject_65k"] = bench_recall_inject(dev, cpu=not args.no_cpu)
        log("secondary: index query")
        sec["index_query_78k"] = bench_index_query(dev)
        log("secondary: HF tiered cache")
        sec["hf_cache_step"] = bench_hf_cache(dev)
        torch.cuda.empty_cache()
        log("secondary: HBM ceilings of the access patterns")
        sec["hbm_ceilings"] = bench_hbm_ceilings(dev)
        result["secondary"] = sec
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
