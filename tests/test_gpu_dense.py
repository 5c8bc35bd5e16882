"""GPU parity: the reference's dense launchers (launch_kessie_windowed_attn,
launch_kessie_fused_fog_attn: fp16 [B, H, N, D], every position a query)
through KeSSieKernels vs the CPU oracle (fp32 on upcast inputs).  head_dim 128
or 64 with H*N a multiple of 16 runs on the MFMA prefill kernel (table-less
pages), other shapes on the generic kernel.  Tolerance |gpu - ref| <= 2e-2 +
1e-2*|ref|."""
import pytest
import torch

from oracle.attention import fused_fog_attention_ref, windowed_attention_ref
from tests.inputs import gen

pytestmark = pytest.mark.gpu


def _check(got, ref):
    g = got.float().cpu()
    diff = (g - ref).abs()
    bad = diff > 2e-2 + 1e-2 * ref.abs()
    assert not bad.any(), f"{int(bad.sum())}/{bad.numel()} outside tol, max diff {diff.max().item():.3e}"


def _qkv(dev, b, h, n, d, seed):
    return [torch.randn(b, h, n, d, generator=gen(dev, seed + i), device=dev).to(torch.float16) for i in range(3)]


# MFMA route: D = 128 or 64 and H*N a multiple of 16 (N itself need not be:
# the last page of every head ends inside it); the rest (here (2, 2, 100, *)
# and (1, 3, 50, 64)) run on the generic kernel.
SHAPES = [(2, 4, 256, 128), (1, 3, 1024, 128), (2, 32, 100, 128), (1, 4, 1000, 128), (3, 16, 37, 128),
          (2, 2, 100, 128), (2, 3, 64, 64), (1, 2, 48, 64), (2, 4, 256, 64), (1, 4, 1000, 64), (3, 16, 37, 64),
          (2, 2, 100, 64), (1, 3, 50, 64)]
MFMA_ROUTE = {s for s in SHAPES if (s[1] * s[2]) % 16 == 0}


@pytest.mark.parametrize("b,h,n,d", SHAPES)
@pytest.mark.parametrize("window,causal", [(0, True), (37, True), (0, False), (1, True)])
def test_windowed_attention(dev, monkeypatch, b, h, n, d, window, causal):
    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    if (b, h, n, d) in MFMA_ROUTE:
        monkeypatch.setenv("KESSIE_REQUIRE_MFMA", "1")  # the launcher errors if it would use the generic kernel
    q, k, v = _qkv(dev, b, h, n, d, seed=n + d + window)
    out = KeSSieKernels().windowed_attention(q, k, v, window_size=window, causal=causal)
    ref = windowed_attention_ref(q.float().cpu(), k.float().cpu(), v.float().cpu(), window, causal)
    _check(out, ref)


@pytest.mark.parametrize("b,h,n,d", SHAPES)
@pytest.mark.parametrize("window", [0, 200])
def test_fused_fog_attention(dev, monkeypatch, b, h, n, d, window):
    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    if (b, h, n, d) in MFMA_ROUTE:
        monkeypatch.setenv("KESSIE_REQUIRE_MFMA", "1")
    q, k, v = _qkv(dev, b, h, n, d, seed=2 * n + d)
    w = torch.rand(n, generator=gen(dev, 7), device=dev)
    out = KeSSieKernels().fused_fog_attention(q, k, v, w, window_size=window)
    ref = fused_fog_attention_ref(q.float().cpu(), k.float().cpu(), v.float().cpu(), w.cpu(), window)
    _check(out, ref)


@pytest.mark.parametrize("d", [128, 64])
def test_dense_mfma_matches_generic(dev, monkeypatch, d):
    """The MFMA route (table-less pages) and the generic kernel agree on a
    2,048-token causal fog case, both within tolerance of the oracle."""
    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    q, k, v = _qkv(dev, 1, 8, 2048, d, seed=11)
    w = torch.rand(2048, generator=gen(dev, 12), device=dev)
    kk = KeSSieKernels()
    monkeypatch.setenv("KESSIE_REQUIRE_MFMA", "1")
    fast = kk.fused_fog_attention(q, k, v, w)
    monkeypatch.delenv("KESSIE_REQUIRE_MFMA")
    monkeypatch.setenv("KESSIE_FORCE_GENERIC", "1")
    slow = kk.fused_fog_attention(q, k, v, w)
    ref = fused_fog_attention_ref(q.float().cpu(), k.float().cpu(), v.float().cpu(), w.cpu())
    _check(fast, ref)
    _check(slow, ref)
    assert not torch.equal(fast, slow)  # two different kernels ran


def test_require_mfma_switch_rejects_a_generic_shape(dev, monkeypatch):
    """H*N not a multiple of 16 has no MFMA route: with the switch set the
    launcher reports it instead of running the generic kernel."""
    from kessie_amd import _lib
    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    monkeypatch.setenv("KESSIE_REQUIRE_MFMA", "1")
    q, k, v = _qkv(dev, 1, 3, 50, 64, seed=13)
    with pytest.raises(_lib.KeSSieError, match="generic kernel"):
        KeSSieKernels().windowed_attention(q, k, v)


@pytest.mark.parametrize("n", [512, 2048, 4096])
@pytest.mark.parametrize("window", [0, 1024])
def test_reference_benchmark_shapes(dev, monkeypatch, n, window):
    """The reference's own benchmark of launch_kessie_windowed_attn
    (kessie_kernels_v2.hip:961-1004: B=1, H=8, D=128, causal, full and
    W=1024) on the MFMA route, where the key splits fill the chip: within
    tolerance of the oracle, and so is the same call held to one split."""
    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    monkeypatch.setenv("KESSIE_REQUIRE_MFMA", "1")
    q, k, v = _qkv(dev, 1, 8, n, 128, seed=n + window)
    kk = KeSSieKernels()
    out = kk.windowed_attention(q, k, v, window_size=window, causal=True)
    monkeypatch.setenv("KESSIE_DENSE_SPLITS", "1")
    one = kk.windowed_attention(q, k, v, window_size=window, causal=True)
    ref = windowed_attention_ref(q.float().cpu(), k.float().cpu(), v.float().cpu(), window, True)
    _check(out, ref)
    _check(one, ref)


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("splits", [2, 5])
def test_dense_forced_splits_fused_fog(dev, monkeypatch, d, splits):
    """Forced key splits (partials + combine) of the fused fog launcher,
    causal and windowed, with N not a multiple of the 64-key tile: within
    tolerance of the oracle, and not the bits of the unsplit launch (the split
    route ran)."""
    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    monkeypatch.setenv("KESSIE_REQUIRE_MFMA", "1")
    n = 1000
    q, k, v = _qkv(dev, 2, 4, n, d, seed=21 + splits)
    w = torch.rand(n, generator=gen(dev, 22), device=dev)
    kk = KeSSieKernels()
    for window in (0, 300):
        monkeypatch.setenv("KESSIE_DENSE_SPLITS", str(splits))
        out = kk.fused_fog_attention(q, k, v, w, window_size=window)
        monkeypatch.setenv("KESSIE_DENSE_SPLITS", "1")
        one = kk.fused_fog_attention(q, k, v, w, window_size=window)
        ref = fused_fog_attention_ref(q.float().cpu(), k.float().cpu(), v.float().cpu(), w.cpu(), window)
        _check(out, ref)
        _check(one, ref)
        assert not torch.equal(out, one)


def test_dense_split_under_graph_capture(dev):
    """The split dense launcher (through the C ABI, on an explicit stream)
    captured in a HIP graph on a stream whose partial buffer exists (an eager
    call on that stream first) and replayed with new inputs between replays:
    every replay equals the eager call bit for bit.  A first call under
    capture on a fresh stream (no buffer, nothing allocated) runs unsplit and
    is still correct."""
    import ctypes

    from kessie_amd import _lib

    q, k, v = _qkv(dev, 1, 8, 2048, 128, seed=31)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())

    def call(o, st):
        _lib.call_legacy("launch_kessie_windowed_attn", ptr(q), ptr(k), ptr(v), ptr(o), ctypes.c_float(128 ** -0.5),
                         1, 8, 2048, 128, 0, 1, ctypes.c_void_p(st.cuda_stream))

    out = torch.empty_like(q)
    stream = torch.cuda.Stream()
    call(out, stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        call(out, stream)
    torch.cuda.synchronize()
    for i in range(3):
        q.copy_(torch.randn(q.shape, generator=gen(dev, 40 + i), device=dev).to(torch.float16))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = torch.empty_like(q)
        call(want, stream)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"
    ref = windowed_attention_ref(q.float().cpu(), k.float().cpu(), v.float().cpu(), 0, True)
    _check(got, ref)
    fresh = torch.cuda.Stream()
    out2 = torch.empty_like(q)
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=fresh):
        call(out2, fresh)
    g2.replay()
    torch.cuda.synchronize()
    _check(out2, ref)
