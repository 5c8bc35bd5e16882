"""CPU: pin the fog oracles against the closed forms the reference's own tests
assert (kessie_attention.py:355-436, kessie_niah_test.py:514-542)."""
import pytest
import torch

from oracle.fog import build_fog_weights, fog_bias


@pytest.mark.parametrize("n,alpha,fs", [(4096, 0.5, 0.5), (131072, 0.5, 0.5), (1000, 0.8, 0.3), (7, 0.5, 0.5)])
def test_fog_weights_closed_form(n, alpha, fs):
    w = build_fog_weights(n, alpha, fs)
    c = int(n * (1.0 - fs))
    assert w.shape == (n,) and w.dtype == torch.float32
    assert w[0].item() == 0.0
    assert w[c - 1].item() == pytest.approx(1.0, abs=1e-6)
    assert torch.all(w[c:] == 1.0)
    assert torch.all(w[1:] >= w[:-1])
    t = torch.arange(c, dtype=torch.float64) / max(c - 1, 1)
    assert torch.allclose(w[:c].double(), t ** alpha, atol=1e-6)


def test_fog_weights_degenerate():
    assert torch.all(build_fog_weights(100, 0.0, 0.5) == 1.0)
    assert torch.all(build_fog_weights(1, 0.5, 0.5) == 1.0)  # c = 0
    w = build_fog_weights(2, 0.5, 0.5)  # c = 1: t = 0/max(0,1)
    assert w.tolist() == [0.0, 1.0]


def test_fog_bias_reference_assertions():
    """kessie_attention.py:355-405: shape, -alpha at 0, zero clear zone, recall boost."""
    b = fog_bias(128, 0.5, 0.5)
    boundary = 64
    assert b.shape == (128,)
    assert b[0].item() == pytest.approx(-0.5)
    assert b[0] < b[32] < 0
    assert b[boundary - 1] < 0
    assert torch.all(b[boundary:] == 0)
    assert b.max().item() <= 0
    b2 = fog_bias(128, 0.5, 0.5, {10, 50, 100}, 0.1)
    assert b2[10].item() == pytest.approx(0.1, abs=1e-7)
    assert b2[100].item() == pytest.approx(0.1, abs=1e-7)
    assert b2[11] < 0
    assert b2[10] > b2[70]
    b3 = fog_bias(256, 0.8, 0.3, {5}, 0.1)
    assert torch.all(b3[int(256 * 0.7):].abs() < 1e-5)
    assert b3[0] < b[0]
    assert torch.all(fog_bias(128, 0.0, 0.5) == 0)


def test_fog_bias_closed_form_values():
    n, alpha, fs = 131072, 0.5, 0.5
    recall = {7, 1000, 65535, 131071, 200000}
    b = fog_bias(n, alpha, fs, recall, 0.1)
    bd = int(n * (1 - fs))
    p = torch.arange(bd, dtype=torch.float64)
    want = -alpha * (1 - p / bd) ** 2
    for r in recall:
        if r < bd:
            want[r] = 0.1
    assert torch.allclose(b[:bd].double(), want, atol=1e-6)
    assert torch.all(b[bd:][[i - bd for i in range(bd, n) if i not in recall][:10]] == 0)
    assert b[131071].item() == pytest.approx(0.1, abs=1e-7)
    # kessie_niah_test.py:538-542 ordering: recalled > clear > fogged.
    assert b[1000] > b[bd + 1] > b[1001]


def test_fog_bias_bf16_follows_dtype_ops():
    """In bf16 the reference computes arange and the decay in bf16; the
    restatement stays within bf16 rounding of the fp32 closed form, and its
    positions are the bf16-rounded integers."""
    n = 8192
    b16 = fog_bias(n, 0.5, 0.5, (), 0.1, dtype=torch.bfloat16)
    assert b16.dtype == torch.bfloat16
    b32 = fog_bias(n, 0.5, 0.5)
    assert (b16.float() - b32).abs().max().item() < 0.02
    # arange(4096) in bf16 is not exact past 256: the step pattern must show it.
    assert len(torch.unique(b16[:4096])) < 4096
