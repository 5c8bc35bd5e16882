"""GPU parity: RoPE remap (paged and dense) vs the CPU oracle.

Tolerance (floating point, bf16/fp16 storage): |gpu - ref| <= 2e-2 + 1e-2*|ref|,
and the fraction of elements that differ at all must stay below 1e-3: the
angle is bit-identical (host inv_freq table, one fp32 multiply) and every
product is rounded separately, so differences come only from cos/sin values
that differ by an ulp between the GPU math library and torch's CPU one.
"""
import numpy as np
import pytest
import torch

from oracle.rope import rope_remap_pages_ref, rope_remap_ref
from tests.inputs import gen, paged_pool, randperm

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _assert_close_rare(got: torch.Tensor, ref: torch.Tensor, max_frac=1e-3):
    """bf16/fp16: tolerance plus rare flips.  fp32 storage shows every ulp of
    cos/sin difference, so there the fp32 tolerance (1e-5) applies instead."""
    g, r = got.float().cpu(), ref.float().cpu()
    diff = (g - r).abs()
    if got.dtype == torch.float32:
        bad = diff > 1e-5 + 1e-5 * r.abs()
        assert not bad.any(), f"{int(bad.sum())} elements outside fp32 tolerance, max diff {diff.max().item()}"
        return
    bad = diff > ATOL + RTOL * r.abs()
    assert not bad.any(), f"{int(bad.sum())} elements outside tolerance, max diff {diff.max().item()}"
    frac = (g != r).float().mean().item()
    assert frac <= max_frac, f"{frac:.2e} of elements differ (expected rare ulp flips)"


def _remap_case(dev, n_tok, num_pages, theta, dtype, seed=0, base_seed=3):
    from kessie_amd import ops

    p = 16
    pool = paged_pool(num_pages, p, 8, 128, dtype, dev, seed)
    page_list = randperm(num_pages, dev, seed + 1)[: (n_tok + p - 1) // p].contiguous()
    orig = torch.randint(0, 1_000_000, (n_tok,), generator=gen(dev, seed + 2), device=dev, dtype=torch.int32)
    base = int(torch.randint(0, 1_000_000, (1,), generator=gen(dev, base_seed), device=dev).item())
    tgt = (base + torch.arange(n_tok, device=dev)).to(torch.int32)
    ref = pool.cpu()
    rope_remap_pages_ref(ref, page_list.cpu(), orig.cpu(), tgt.cpu(), theta)
    ops.rope_remap_paged(pool, orig, tgt, theta, page_list=page_list)
    torch.cuda.synchronize()
    return pool, ref


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_remap_paged_matches_oracle(dev, dtype):
    pool, ref = _remap_case(dev, n_tok=2000, num_pages=160, theta=500000.0, dtype=dtype)
    # K of the listed pages rotated, V and unlisted pages untouched (bit-exact).
    _assert_close_rare(pool, ref)
    assert torch.equal(pool[:, :, 1].cpu(), ref[:, :, 1])


def test_remap_full_size_every_token(dev):
    """Config: 65,536 tokens in 16-token pages, 8 KV heads, D=128, bf16, theta 5e5;
    every token's K checked against the oracle, V and unlisted pages untouched."""
    from kessie_amd import ops

    n_tok, p = 65536, 16
    num_pages = n_tok // p
    pool = paged_pool(num_pages + 64, p, 8, 128, torch.bfloat16, dev, 0)
    page_list = randperm(num_pages + 64, dev, 1)[:num_pages].contiguous()
    orig = torch.randint(0, 1_000_000, (n_tok,), generator=gen(dev, 2), device=dev, dtype=torch.int32)
    base = int(torch.randint(0, 1_000_000, (1,), generator=gen(dev, 3), device=dev).item())
    tgt = (base + torch.arange(n_tok, device=dev)).to(torch.int32)
    before = pool.clone()
    ref = pool.cpu()
    rope_remap_pages_ref(ref, page_list.cpu(), orig.cpu(), tgt.cpu(), 500000.0)
    ops.rope_remap_paged(pool, orig, tgt, 500000.0, page_list=page_list)
    torch.cuda.synchronize()
    _assert_close_rare(pool[:, :, 0], ref[:, :, 0])
    assert torch.equal(pool[:, :, 1], before[:, :, 1])  # V untouched everywhere
    listed = torch.zeros(num_pages + 64, dtype=torch.bool, device=dev)
    listed[page_list.long()] = True
    assert torch.equal(pool[~listed], before[~listed])  # pages not in the list untouched
    # Remapping back to the original positions: per-pair norm preserved (bf16 rounding bound).
    ops.rope_remap_paged(pool, tgt, orig, 500000.0, page_list=page_list)
    torch.cuda.synchronize()
    k0 = before[:, :, 0].float()
    k2 = pool[:, :, 0].float()
    assert (k2 - k0).abs().max().item() < 0.1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", ["kv_first", "block_kv"])
def test_remap_k_only_page_layouts(dev, layout, dtype):
    """Pools whose pages hold K rows contiguously (vLLM's [2][blocks][P][H][D]
    and [blocks][2][P][H][D]) take the contiguous-row tile; 2,003 tokens leave
    a partial last page and a partial last tile.  Checked through a native
    view of the same storage against the oracle; V untouched."""
    from kessie_amd import ops

    n_tok, p, num_pages = 2003, 16, 160
    g = gen(dev, 21)
    if layout == "kv_first":
        pool = torch.randn(2, num_pages, p, 8, 128, generator=g, device=dev).to(dtype)
        native = lambda t: t.permute(1, 2, 0, 3, 4)  # noqa: E731
    else:
        pool = torch.randn(num_pages, 2, p, 8, 128, generator=g, device=dev).to(dtype)
        native = lambda t: t.permute(0, 2, 1, 3, 4)  # noqa: E731
    page_list = randperm(num_pages, dev, 22)[: (n_tok + p - 1) // p].contiguous()
    orig = torch.randint(0, 1_000_000, (n_tok,), generator=gen(dev, 23), device=dev, dtype=torch.int32)
    tgt = (777 + torch.arange(n_tok, device=dev)).to(torch.int32)
    before = pool.clone()
    ref = pool.cpu()
    rope_remap_pages_ref(native(ref), page_list.cpu(), orig.cpu(), tgt.cpu(), 500000.0)
    ops.rope_remap_paged(pool, orig, tgt, 500000.0, page_list=page_list, layout=layout)
    torch.cuda.synchronize()
    _assert_close_rare(native(pool)[:, :, 0], native(ref)[:, :, 0])
    assert torch.equal(native(pool)[:, :, 1], native(before)[:, :, 1])


@pytest.mark.parametrize("n_tok", [65536, 1005])
def test_remap_dense_k_tensor(dev, n_tok):
    """The reference operator's own form, K [T, 8, 128] bf16 (kessie_hip_kernels.py:443-476),
    at the full 65,536 tokens and at a count that leaves a partial tile: every
    element against the oracle."""
    from kessie_amd import ops

    k = torch.randn(n_tok, 8, 128, generator=gen(dev, 31), device=dev).bfloat16()
    orig = torch.randint(0, 1_000_000, (n_tok,), generator=gen(dev, 32), device=dev, dtype=torch.int32)
    base = int(torch.randint(0, 1_000_000, (1,), generator=gen(dev, 33), device=dev).item())
    tgt = (base + torch.arange(n_tok, device=dev)).to(torch.int32)
    ref = rope_remap_ref(k.cpu().clone(), orig.cpu(), tgt.cpu(), 500000.0)
    ops.rope_remap_paged(k, orig, tgt, 500000.0)
    torch.cuda.synchronize()
    _assert_close_rare(k, ref)


def test_remap_identity_is_bit_exact(dev):
    from kessie_amd import ops

    pool = paged_pool(64, 16, 8, 128, torch.bfloat16, dev, 5)
    before = pool.clone()
    pos = torch.randint(0, 1_000_000, (1024,), generator=gen(dev, 6), device=dev, dtype=torch.int32)
    ops.rope_remap_paged(pool, pos, pos, 500000.0, page_list=torch.arange(64, device=dev, dtype=torch.int32))
    torch.cuda.synchronize()
    assert torch.equal(pool, before)


def test_remap_skips_bad_page_ids(dev):
    from kessie_amd import ops

    pool = paged_pool(8, 16, 8, 128, torch.bfloat16, dev, 9)
    before = pool.clone()
    page_list = torch.tensor([-1, 8, 100, 3], dtype=torch.int32, device=dev)
    orig = torch.zeros(64, dtype=torch.int32, device=dev)
    tgt = torch.full((64,), 1000, dtype=torch.int32, device=dev)
    ops.rope_remap_paged(pool, orig, tgt, 10000.0, page_list=page_list)
    torch.cuda.synchronize()
    untouched = [0, 1, 2, 4, 5, 6, 7]
    assert torch.equal(pool[untouched], before[untouched])
    assert not torch.equal(pool[3, :, 0], before[3, :, 0])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_ctypes_rope_remap_dense(dev, dtype):
    """KeSSieKernels.rope_remap on [T,H,D] (the reference's method) vs the oracle,
    plus the reference's own round-trip (<0.05) and identity (<1e-5) checks."""
    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    kk = KeSSieKernels()
    L, H, D = 64, 8, 128
    k = torch.randn(L, H, D, generator=gen(dev, 11), device=dev).to(dtype)
    k_orig = k.clone()
    orig = torch.arange(100, 100 + L, dtype=torch.int32, device=dev)
    tgt = torch.arange(5000, 5000 + L, dtype=torch.int32, device=dev)
    ref = rope_remap_ref(k.cpu().clone(), orig.cpu(), tgt.cpu(), 10000.0)
    kk.rope_remap(k, orig, tgt)
    _assert_close_rare(k, ref)
    k_back = k.clone()
    kk.rope_remap(k_back, tgt, orig)
    assert (k_orig.float() - k_back.float()).abs().max().item() < 0.05
    k2 = torch.randn(L, H, D, generator=gen(dev, 12), device=dev).to(dtype)
    k2o = k2.clone()
    kk.rope_remap(k2, orig, orig)
    assert (k2o.float() - k2.float()).abs().max().item() < 1e-5


def test_legacy_launcher_rope_fp16(dev):
    """launch_kessie_rope_remap (reference signature, fp16, device-side table)."""
    import ctypes

    from kessie_amd import _lib

    L, H, D = 96, 4, 64
    k = torch.randn(L, H, D, generator=gen(dev, 13), device=dev).half()
    orig = torch.randint(0, 100000, (L,), generator=gen(dev, 14), device=dev, dtype=torch.int32)
    tgt = torch.randint(0, 100000, (L,), generator=gen(dev, 15), device=dev, dtype=torch.int32)
    ref = rope_remap_ref(k.cpu().clone(), orig.cpu(), tgt.cpu(), 10000.0)
    _lib.call_legacy("launch_kessie_rope_remap", ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(orig.data_ptr()),
                     ctypes.c_void_p(tgt.data_ptr()), ctypes.c_float(10000.0), L, H, D // 2,
                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    # The device-side frequency table may differ from the host one by an ulp,
    # so only the tolerance applies here.
    diff = (k.float().cpu() - ref.float()).abs()
    assert (diff <= ATOL + RTOL * ref.float().abs()).all(), diff.max().item()
    assert np.isfinite(k.float().cpu().numpy()).all()
