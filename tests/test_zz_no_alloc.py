"""GPU: kessie_fog_decode_paged_noalloc (split partials in the library's static
device scratch, no workspace argument) against kessie_fog_decode_paged with a
caller workspace, both called through the C ABI.  Same kernels and split
count, so the outputs must be identical bit for bit; two calls in a row, the
second smaller (the scratch keeps the first call's partials, which the
second must not read), the balanced split layout, a capture in a HIP graph,
and a shape whose partials exceed the scratch."""
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


def test_noalloc_decode_balanced_layout_equals_workspace_decode(dev):
    """A ragged batch whose K/V (1 GiB) takes the balanced split layout (a
    sequence's partials at h * S * B + unit) through the static scratch: 2
    sequences of 131,072 and 9,000 tokens, 32 q / 8 kv heads, ~4.3 MB of
    partials; bit for bit against the workspace call, then a smaller call."""
    ctx = 131072
    q, pool, table, lens = decode_case(2, 32, 8, 128, ctx, 16, torch.bfloat16, dev, seed=64, ctx_lens=[ctx, 9000])
    vs = build_fog_weights(ctx).to(dev)
    ref, got = _both(dev, q, pool, table, lens, ctx, vs)
    assert torch.isfinite(ref.float()).all()
    assert torch.equal(got, ref)
    del pool
    q, pool, table, lens = decode_case(1, 32, 8, 128, 2000, 16, torch.bfloat16, dev, seed=65)
    ref, got = _both(dev, q, pool, table, lens, 2000, None)
    assert torch.equal(got, ref)


def test_noalloc_decode_under_graph_capture(dev):
    """The no-alloc call captured in a HIP graph (after one eager call on the
    device, which resolves the scratch address) and replayed with new query
    values and new lengths between replays: every replay equals the eager call
    on the same inputs bit for bit."""
    from kessie_amd import _lib

    lib = _lib.load()
    ctx = 6000
    q, pool, table, lens = decode_case(3, 32, 8, 128, ctx, 16, torch.bfloat16, dev, seed=66,
                                       ctx_lens=[ctx, 4000, 77])
    vs = build_fog_weights(ctx).to(dev)
    out = torch.empty_like(q)
    stream = torch.cuda.Stream()

    def call(o):
        st = lib.kessie_fog_decode_paged_noalloc(*_args(q, pool, table, lens, ctx, vs, o, _lib.DTYPE_BF16),
                                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        _lib.check("kessie_fog_decode_paged_noalloc", st)

    call(out)  # eager, outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        call(out)
    torch.cuda.synchronize()
    for i, new_lens in enumerate(([ctx, 4000, 77], [100, ctx, 5999], [0, 1, ctx])):
        q.copy_(torch.randn(q.shape, generator=torch.Generator(device=dev).manual_seed(300 + i), device=dev)
                .to(torch.bfloat16))
        lens.copy_(torch.tensor(new_lens, dtype=torch.int32, device=dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = torch.empty_like(q)
        call(want)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"
