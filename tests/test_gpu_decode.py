"""GPU parity: paged fog decode vs the CPU oracle.

Tolerances (the path's parity requirement): bf16/fp16 outputs with fp32 accumulation
|gpu - ref| <= 2e-2 + 1e-2*|ref|; fp32 configs 1e-5 (atol and rtol).
"""
import math

import pytest
import torch

from oracle.attention import paged_decode_blockwise, paged_decode_ref
from oracle.fog import build_fog_weights, fog_bias
from tests.inputs import decode_case, gen

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float16: (2e-2, 1e-2), torch.float32: (1e-5, 1e-5)}


def _check(got, ref, dtype):
    atol, rtol = TOL[dtype]
    g = got.float().cpu()
    diff = (g - ref).abs()
    bad = diff > atol + rtol * ref.abs()
    assert not bad.any(), f"{int(bad.sum())}/{bad.numel()} outside tol, max diff {diff.max().item():.3e}"


def _run(dev, b, hq, hkv, ctx, dtype, fog="vscale", window=0, ctx_lens=None, layout="native", seed=0, page_size=16):
    from kessie_amd import ops

    d, p = 128, page_size
    q, pool, table, lens = decode_case(b, hq, hkv, d, ctx, p, dtype, dev, seed=seed, ctx_lens=ctx_lens)
    vs = bias = None
    if fog == "vscale":
        vs = build_fog_weights(ctx, 0.5, 0.5).to(dev)
    elif fog == "bias":
        bias = fog_bias(ctx, 0.5, 0.5, {3, 17, ctx - 2}, 0.1).to(dev)
    elif fog == "vscale_batched":
        vs = torch.rand(b, ctx, generator=gen(dev, 77), device=dev)
    elif fog == "both":
        vs = torch.rand(b, ctx, generator=gen(dev, 77), device=dev)
        bias = fog_bias(ctx, 0.5, 0.5, {3, 17, ctx - 2}, 0.1).to(dev)
    pool_arg = pool
    if layout == "kv_first":
        pool_arg = pool.permute(2, 0, 1, 3, 4).contiguous()
    elif layout == "block_kv":
        pool_arg = pool.permute(0, 2, 1, 3, 4).contiguous()
    out = ops.fog_decode(q, pool_arg, table, lens, max_ctx=ctx, fog_vscale=vs, fog_bias=bias, window=window,
                         layout=layout)
    torch.cuda.synchronize()
    ref = paged_decode_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(),
                           None if vs is None else vs.cpu(), None if bias is None else bias.cpu(), window)
    return out, ref


@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (16, 8), (64, 8), (8, 1), (12, 3), (32, 4),
                                     (16, 1), (128, 8)])
def test_decode_bf16_gqa(dev, hq, hkv):
    out, ref = _run(dev, 2, hq, hkv, 1000, torch.bfloat16)
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("page_size,dtype,fog,window,ctx_lens,layout", [
    (32, torch.bfloat16, "vscale", 0, [1000, 37, 777], "native"),
    (64, torch.bfloat16, "both", 100, [530, 301, 17], "native"),
    (32, torch.float32, "vscale", 0, [1000, 0, 513], "native"),
    (32, torch.bfloat16, "bias", 0, [640, 33, 1], "kv_first"),
    (128, torch.bfloat16, "vscale", 0, [1000, 129, 128], "native"),
])
def test_decode_larger_pages(dev, page_size, dtype, fog, window, ctx_lens, layout):
    """Pages of 32, 64 and 128 tokens (vLLM block sizes) on the MFMA kernels,
    which read them as 16-token blocks: against the oracle, ragged and empty
    sequences, windows and vLLM's K/V-first layout included."""
    out, ref = _run(dev, len(ctx_lens), 32, 8, max(ctx_lens), dtype, fog=fog, window=window, ctx_lens=ctx_lens,
                    layout=layout, page_size=page_size)
    _check(out, ref, dtype)
    for i, n in enumerate(ctx_lens):
        if n == 0:
            assert not out[i].any()


def test_decode_larger_pages_balanced(dev):
    """32-token pages through the balanced split (a ragged batch whose K/V
    bound passes its threshold): every sequence against the oracle."""
    from kessie_amd import ops

    ctx, p = 32768, 32
    ctx_lens = [ctx, 5, 20000, 0]
    q, pool, table, lens = decode_case(len(ctx_lens), 32, 8, 128, ctx, p, torch.bfloat16, dev, seed=97,
                                       ctx_lens=ctx_lens)
    vs = build_fog_weights(ctx).to(dev)
    out = ops.fog_decode(q, pool, table, lens, ctx, fog_vscale=vs)
    torch.cuda.synchronize()
    for i, n in enumerate(ctx_lens):
        if n == 0:
            assert not out[i].any()
            continue
        sub_pool = pool[table[i].long()].cpu()
        sub_table = torch.arange(table.shape[1], dtype=torch.int32).view(1, -1)
        ref = paged_decode_blockwise(q[i:i + 1].cpu(), sub_pool, sub_table, lens[i:i + 1].cpu(), vs.cpu())
        _check(out[i:i + 1], ref, torch.bfloat16)


def test_decode_fp16(dev):
    out, ref = _run(dev, 2, 32, 8, 777, torch.float16)
    _check(out, ref, torch.float16)


def test_decode_fp32_cpu_path_shape(dev):
    """Config: fp32, B=1, 32q/8kv, D=128, 4096-token context, V-fog defaults."""
    out, ref = _run(dev, 1, 32, 8, 4096, torch.float32)
    _check(out, ref, torch.float32)


def test_decode_fp32_config_inputs_with_rope(dev):
    """The configuration's inputs as specified: fp32, B=1, 32q/8kv, D=128,
    4,096 tokens in 16-token pages (table randperm(256), seed 1), Q, K, V ~
    N(0,1) from seed 0 in that order, K stored after rotate-half RoPE (theta
    1e4) at positions 0..4095 and q rotated at position 4095, fog weights
    build_fog_weights(4096, 0.5, 0.5), window 0: within 1e-5 of the oracle."""
    from kessie_amd import ops

    n, hq, hkv, d, p = 4096, 32, 8, 128, 16
    g = gen(dev, 0)
    q = torch.randn(1, hq, d, generator=g, device=dev)
    k = torch.randn(n, hkv, d, generator=g, device=dev)
    v = torch.randn(n, hkv, d, generator=g, device=dev)

    def rope(x, pos):  # rotate-half RoPE in float64; x [T, H, D], pos [T]
        inv = 1.0 / (1e4 ** (torch.arange(d // 2, dtype=torch.float64, device=dev) / (d // 2)))
        ang = pos.double()[:, None] * inv[None, :]
        c, s = ang.cos()[:, None, :], ang.sin()[:, None, :]
        x1, x2 = x[..., :d // 2].double(), x[..., d // 2:].double()
        return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], -1).float()

    k = rope(k, torch.arange(n, device=dev))
    q = rope(q, torch.tensor([n - 1], device=dev))
    table = torch.randperm(n // p, generator=gen(dev, 1), device=dev).to(torch.int32).view(1, -1)
    pool = torch.empty(n // p, p, 2, hkv, d, device=dev)
    pool[table[0].long()] = torch.stack([k, v], 1).view(n // p, p, 2, hkv, d)
    lens = torch.tensor([n], dtype=torch.int32, device=dev)
    vs = build_fog_weights(n, 0.5, 0.5).to(dev)
    out = ops.fog_decode(q, pool, table, lens, max_ctx=n, fog_vscale=vs)
    torch.cuda.synchronize()
    ref = paged_decode_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), vs.cpu(), None, 0)
    _check(out, ref, torch.float32)


@pytest.mark.parametrize("fog", ["none", "bias", "vscale_batched", "both"])
def test_decode_fog_modes(dev, fog):
    out, ref = _run(dev, 3, 32, 8, 530, torch.bfloat16, fog=fog)
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("fog", ["bias", "both"])
@pytest.mark.parametrize("window", [15, 100])
def test_decode_fog_modes_windowed_ragged(dev, fog, window):
    """Per-token fog values on the window's first page and the last, partial
    page of ragged sequences (both edges read only the visible tokens)."""
    out, ref = _run(dev, 3, 32, 8, 530, torch.bfloat16, fog=fog, window=window,
                    ctx_lens=[530, 301, 17])
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("window", [1, 15, 16, 100, 5000])
def test_decode_window(dev, window):
    out, ref = _run(dev, 2, 32, 8, 1200, torch.bfloat16, window=window)
    _check(out, ref, torch.bfloat16)


def test_decode_ragged_and_empty(dev):
    lens = [0, 1, 15, 16, 17, 999]
    out, ref = _run(dev, 6, 32, 8, 1000, torch.bfloat16, ctx_lens=lens)
    _check(out, ref, torch.bfloat16)
    assert torch.count_nonzero(out[0]) == 0


@pytest.mark.parametrize("layout", ["kv_first", "block_kv"])
def test_decode_vllm_layouts(dev, layout):
    out, ref = _run(dev, 2, 32, 8, 640, torch.bfloat16, layout=layout)
    _check(out, ref, torch.bfloat16)


def test_decode_invalid_page_ids_are_masked(dev):
    from kessie_amd import ops

    q, pool, table, lens = decode_case(1, 32, 8, 128, 256, 16, torch.bfloat16, dev, seed=3)
    table[0, 5] = -1
    table[0, 9] = 1 << 20
    out = ops.fog_decode(q, pool, table, lens, max_ctx=256)
    torch.cuda.synchronize()
    # Oracle: the same attention without the tokens of logical pages 5 and 9.
    keep = [i for i in range(16) if i not in (5, 9)]
    pool_c = pool.cpu()
    t2 = table.cpu()[:, keep].contiguous()
    ref = paged_decode_ref(q.cpu(), pool_c, t2, torch.tensor([len(keep) * 16]))
    _check(out, ref, torch.bfloat16)


def test_decode_generic_path_matches_mfma_path(dev, monkeypatch):
    """The VALU fallback kernel (any shape) and the MFMA kernel agree."""
    from kessie_amd import ops

    q, pool, table, lens = decode_case(2, 32, 8, 128, 900, 16, torch.bfloat16, dev, seed=4)
    vs = build_fog_weights(900).to(dev)
    a = ops.fog_decode(q, pool, table, lens, 900, fog_vscale=vs)
    monkeypatch.setenv("KESSIE_FORCE_GENERIC", "1")
    b = ops.fog_decode(q, pool, table, lens, 900, fog_vscale=vs)
    torch.cuda.synchronize()
    assert (a.float() - b.float()).abs().max().item() < 2e-2


def test_decode_llama8b_128k_all_sequences(dev):
    """Config: bf16, B=16, 32q/8kv, D=128, 131,072-token context in 16-token pages,
    V-fog defaults.  Full-size run; every sequence checked against the oracle."""
    from kessie_amd import ops

    b, ctx = 16, 131072
    q, pool, table, lens = decode_case(b, 32, 8, 128, ctx, 16, torch.bfloat16, dev, seed=0)
    vs = build_fog_weights(ctx).to(dev)
    out = ops.fog_decode(q, pool, table, lens, ctx, fog_vscale=vs)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    for s in range(b):
        # Gather the sequence's pages on the device first (8192 pages), then run
        # the blockwise oracle on the CPU copy of just those pages.
        sub_pool = pool[table[s].long()].cpu()
        sub_table = torch.arange(table.shape[1], dtype=torch.int32).view(1, -1)
        ref = paged_decode_blockwise(q[s:s + 1].cpu(), sub_pool, sub_table, lens[s:s + 1].cpu(), vs.cpu())
        _check(out[s:s + 1], ref, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kind", ["bimodal", "spread", "empty", "window"])
def test_decode_ragged_batch(dev, dtype, kind):
    """Ragged batches, whose split workgroups go to the batch's pages (a long
    context gets many more than a short one): two long contexts among
    fourteen short ones, a spread of lengths, empty sequences between long
    ones, and a window.  Every sequence matches the oracle (V-fog)."""
    from kessie_amd import ops

    ctx = 32768
    lens_by_kind = {
        "bimodal": [ctx, ctx] + [2048] * 14,
        "spread": [2048 * (i + 1) for i in range(16)],
        "empty": [ctx, 0, 0, 5000, 0, ctx - 1, 17, 0],
        "window": [ctx, 300, 9000, ctx, 1, 16384],
    }
    ctx_lens = lens_by_kind[kind]
    window = 3000 if kind == "window" else 0
    b = len(ctx_lens)
    q, pool, table, lens = decode_case(b, 32, 8, 128, ctx, 16, dtype, dev, seed=91, ctx_lens=ctx_lens)
    vs = build_fog_weights(ctx).to(dev)
    out = ops.fog_decode(q, pool, table, lens, ctx, fog_vscale=vs, window=window)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    for i in range(b):
        if ctx_lens[i] == 0:  # no keys: the kernels write zeros (the oracle's 0/0 is NaN)
            assert not out[i].any()
            continue
        sub_pool = pool[table[i].long()].cpu()
        sub_table = torch.arange(table.shape[1], dtype=torch.int32).view(1, -1)
        ref = paged_decode_blockwise(q[i:i + 1].cpu(), sub_pool, sub_table, lens[i:i + 1].cpu(), vs.cpu(), window)
        _check(out[i:i + 1], ref, dtype)


@pytest.mark.parametrize("hq,hkv,ctx", [(16, 1, 65536), (64, 8, 32768)])
def test_decode_ragged_batch_gqa(dev, hq, hkv, ctx):
    """Ragged batches through the balanced split at other GQA shapes (MQA and
    8 q heads per kv head): every sequence against the oracle."""
    from kessie_amd import ops

    ctx_lens = [ctx, 17, ctx // 3, 0, 4097, ctx - 5, 1, 2048]
    b = len(ctx_lens)
    q, pool, table, lens = decode_case(b, hq, hkv, 128, ctx, 16, torch.bfloat16, dev, seed=95, ctx_lens=ctx_lens)
    vs = build_fog_weights(ctx).to(dev)
    out = ops.fog_decode(q, pool, table, lens, ctx, fog_vscale=vs)
    torch.cuda.synchronize()
    for i in range(b):
        if ctx_lens[i] == 0:
            assert not out[i].any()
            continue
        sub_pool = pool[table[i].long()].cpu()
        sub_table = torch.arange(table.shape[1], dtype=torch.int32).view(1, -1)
        ref = paged_decode_blockwise(q[i:i + 1].cpu(), sub_pool, sub_table, lens[i:i + 1].cpu(), vs.cpu())
        _check(out[i:i + 1], ref, torch.bfloat16)


@pytest.mark.parametrize("b", [64, 65])
def test_decode_ragged_batch_at_the_balanced_limit(dev, b):
    """64 sequences (the most the balanced split takes: one per lane) and 65
    (the plain split), lengths spread over 0..4096 with empty ones among them;
    every sequence against the oracle."""
    from kessie_amd import ops

    ctx = 4096
    ctx_lens = [(i * 997) % (ctx + 1) if i % 9 else 0 for i in range(b)]
    ctx_lens[b - 1] = ctx  # the last lane holds a full-length sequence
    q, pool, table, lens = decode_case(b, 32, 8, 128, ctx, 16, torch.bfloat16, dev, seed=93, ctx_lens=ctx_lens)
    vs = build_fog_weights(ctx).to(dev)
    out = ops.fog_decode(q, pool, table, lens, ctx, fog_vscale=vs)
    torch.cuda.synchronize()
    for i in range(b):
        if ctx_lens[i] == 0:
            assert not out[i].any()
            continue
        sub_pool = pool[table[i].long()].cpu()
        sub_table = torch.arange(table.shape[1], dtype=torch.int32).view(1, -1)
        ref = paged_decode_blockwise(q[i:i + 1].cpu(), sub_pool, sub_table, lens[i:i + 1].cpu(), vs.cpu())
        _check(out[i:i + 1], ref, torch.bfloat16)


@pytest.mark.parametrize("hq,hkv,fog,window,ctx_lens", [
    (32, 8, "vscale", 0, None),
    (32, 8, "both", 100, [4096, 1000, 17]),
    (16, 16, "bias", 0, [333, 0, 4096]),
    (16, 8, "vscale", 0, [4096, 2500]),
    (64, 8, "both", 0, None),
    (64, 4, "none", 5000, None),
])
def test_decode_fp32_mfma_matches_oracle_and_generic(dev, monkeypatch, hq, hkv, fog, window, ctx_lens):
    """fp32 decode on the MFMA kernels (v_mfma_f32_4x4x1_16b_f32 for GQA ratios
    up to 4, v_mfma_f32_16x16x4_f32 for 8 and 16; probabilities in fp32):
    within the fp32 tolerance of the oracle and of the VALU kernel."""
    from kessie_amd import ops

    b = len(ctx_lens) if ctx_lens else 2
    ctx = 4096
    q, pool, table, lens = decode_case(b, hq, hkv, 128, ctx, 16, torch.float32, dev, seed=71, ctx_lens=ctx_lens)
    vs = build_fog_weights(ctx).to(dev) if fog in ("vscale", "both") else None
    bias = fog_bias(ctx, 0.5, 0.5, [3, 900], 0.1, dtype=torch.float32, device=dev) if fog in ("bias", "both") else None
    a = ops.fog_decode(q, pool, table, lens, ctx, fog_vscale=vs, fog_bias=bias, window=window)
    monkeypatch.setenv("KESSIE_FORCE_GENERIC", "1")
    g = ops.fog_decode(q, pool, table, lens, ctx, fog_vscale=vs, fog_bias=bias, window=window)
    torch.cuda.synchronize()
    ref = paged_decode_ref(q.cpu(), pool.cpu(), table.cpu(), lens.cpu(), None if vs is None else vs.cpu(),
                           None if bias is None else bias.cpu(), window=window)
    _check(a, ref, torch.float32)
    _check(g, ref, torch.float32)


@pytest.mark.parametrize("hq,hkv,ctx_lens", [(16, 8, [20000, 3000]), (32, 8, [30000]), (8, 8, [12345, 1, 9000])])
def test_decode_fp32_long_contexts(dev, hq, hkv, ctx_lens):
    """fp32 decode with more than two 16-token blocks per split (the
    two-blocks-in-flight instance of the 4x4x1 kernel), GQA 2, 4 and 1,
    ragged lengths incl. a one-token sequence, V-fog: against the oracle at
    1e-5."""
    out, ref = _run(dev, len(ctx_lens), hq, hkv, max(ctx_lens), torch.float32, ctx_lens=ctx_lens)
    _check(out, ref, torch.float32)


def test_decode_fp32_invalid_page_ids_are_masked(dev):
    """An invalid page id (negative, or past the pool) on the fp32 4x4x1
    kernel: its 16 tokens are left out, as the bf16 kernel does."""
    from kessie_amd import ops

    q, pool, table, lens = decode_case(1, 32, 8, 128, 256, 16, torch.float32, dev, seed=4)
    table[0, 2] = -1
    table[0, 11] = 1 << 20
    out = ops.fog_decode(q, pool, table, lens, max_ctx=256)
    torch.cuda.synchronize()
    keep = [i for i in range(16) if i not in (2, 11)]
    ref = paged_decode_ref(q.cpu(), pool.cpu(), table.cpu()[:, keep].contiguous(), torch.tensor([len(keep) * 16]))
    _check(out, ref, torch.float32)
