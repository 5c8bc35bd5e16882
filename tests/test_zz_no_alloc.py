"""GPU: kessie_fog_decode_paged_noalloc (split partials in the library's static
device scratch, no workspace argument) against kessie_fog_decode_paged with a
caller workspace, both called through the C ABI.  Same kernels and split
count, so the outputs must be identical bit for bit; two calls in a row, the
second smaller (the scratch keeps the first call's partials, which the
second must not read), and a shape whose partials exceed the scratch."""
import ctypes

import pytest
import torch

from oracle.fog import build_fog_weights
from tests.inputs import decode_case

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _args(q, pool, table, lens, max_ctx, vs, out, dtype_code):
    b, hq, d = q.shape
    n, p, _, hkv, _ = pool.shape
    s = pool.stride()
    return [_ptr(q), _ptr(pool), n, s[0], s[1], s[2], s[3], _ptr(table), table.stride(0), _ptr(lens), _ptr(vs), 0,
            None, 0, _ptr(out), b, hq, hkv, d, p, int(max_ctx), 0, float(d) ** -0.5, dtype_code]


def _both(dev, q, pool, table, lens, max_ctx, vs):
    from kessie_amd import _lib

    lib = _lib.load()
    dt = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}[q.dtype]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    b, hq, d = q.shape
    need = lib.kessie_fog_decode_workspace_bytes(b, hq, pool.shape[3], d, int(max_ctx), pool.shape[1], dt)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    ref = torch.full_like(q, float("nan"))
    got = torch.full_like(q, float("nan"))
    _lib.check("kessie_fog_decode_paged", lib.kessie_fog_decode_paged(
        *_args(q, pool, table, lens, max_ctx, vs, ref, dt), _ptr(ws), ws.numel(), stream))
    _lib.check("kessie_fog_decode_paged_noalloc", lib.kessie_fog_decode_paged_noalloc(
        *_args(q, pool, table, lens, max_ctx, vs, got, dt), stream))
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_decode_equals_workspace_decode_twice(dev, dtype):
    from kessie_amd import _lib

    lib = _lib.load()
    # First call: 2 x 3,000 tokens (several splits), V-fog.
    q, pool, table, lens = decode_case(2, 32, 8, 128, 3000, 16, dtype, dev, seed=61)
    assert lib.kessie_fog_decode_num_splits(2, 8, 3000, 16) > 1
    vs = build_fog_weights(3000).to(dev)
    ref, got = _both(dev, q, pool, table, lens, 3000, vs)
    assert torch.isfinite(ref.float()).all()
    assert torch.equal(got, ref)
    # Second call, smaller: one ragged 700-token sequence, another kv/q shape.
    q, pool, table, lens = decode_case(1, 16, 4, 128, 700, 16, dtype, dev, seed=62, ctx_lens=[613])
    ref, got = _both(dev, q, pool, table, lens, 700, None)
    assert torch.isfinite(ref.float()).all()
    assert torch.equal(got, ref)


def test_noalloc_decode_rejects_partials_beyond_the_scratch(dev):
    from kessie_amd import _lib

    lib = _lib.load()
    # 128 sequences x 128 q heads (GQA 16) x 2 splits x 130 floats: 17 MB > 16 MiB.
    b, hq, hkv, d, ctx = 128, 128, 8, 128, 64
    assert lib.kessie_fog_decode_num_splits(b, hkv, ctx, 16) == 2
    q, pool, table, lens = decode_case(b, hq, hkv, d, ctx, 16, torch.bfloat16, dev, seed=63)
    out = torch.zeros_like(q)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = lib.kessie_fog_decode_paged_noalloc(*_args(q, pool, table, lens, ctx, None, out, _lib.DTYPE_BF16), stream)
    torch.cuda.synchronize()
    assert st == _lib.ERR_WORKSPACE
    status, msg = _lib.last_error()
    assert status == _lib.ERR_WORKSPACE and "static scratch" in msg
    assert bool((out == 0).all())  # nothing launched
