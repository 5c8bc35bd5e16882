"""CPU: pin the RoPE-remap oracle (oracle/rope.py) against the mathematics and
the reference's own checks (kessie_hip_kernels.py:662-683)."""
import numpy as np
import pytest
import torch

from oracle.rope import inv_freq_table, rope_apply_f64, rope_remap_pages_ref, rope_remap_ref


def _k(t, h, d, seed=0, dtype=torch.float32):
    return torch.randn(t, h, d, generator=torch.Generator().manual_seed(seed)).to(dtype)


def test_inv_freq_table_closed_form():
    for d, theta in ((128, 10000.0), (128, 500000.0), (64, 10000.0)):
        inv = inv_freq_table(d, theta).double().numpy()
        exact = theta ** (-np.arange(d // 2) / (d // 2))
        assert inv[0] == 1.0
        assert np.allclose(inv, exact, rtol=3e-7, atol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_identity_is_bit_exact(dtype):
    k = _k(32, 4, 128, 1, dtype)
    pos = torch.randint(0, 1_000_000, (32,), dtype=torch.int32)
    out = rope_remap_ref(k.clone(), pos, pos, 500000.0)
    assert torch.equal(out, k)


def test_reference_round_trip_bound():
    """The reference's round-trip test: fp16, 100.. -> 5000.. and back, < 0.05."""
    k = _k(64, 8, 128, 2, torch.float16)
    orig = torch.arange(100, 164, dtype=torch.int32)
    tgt = torch.arange(5000, 5064, dtype=torch.int32)
    back = rope_remap_ref(rope_remap_ref(k.clone(), orig, tgt), tgt, orig)
    assert (back.float() - k.float()).abs().max().item() < 0.05


def test_composition_with_full_rope():
    """remap(rope(x, p), p -> q) == rope(x, q): the check that catches a wrong
    pairing, sign, frequency index or partial coverage (which identity and
    round trip cannot)."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((40, 4, 128))
    p = rng.integers(0, 4000, 40)
    q = rng.integers(0, 4000, 40)
    k = torch.from_numpy(rope_apply_f64(x, p, 10000.0)).float()
    got = rope_remap_ref(k, torch.from_numpy(p).int(), torch.from_numpy(q).int(), 10000.0).double().numpy()
    want = rope_apply_f64(x, q, 10000.0)
    assert np.abs(got - want).max() < 5e-3


def test_large_delta_matches_fp32_angle_closed_form():
    """At |delta| ~ 1e6 with theta 5e5 the fp32 angle is what the reference
    computes; rotating by exactly that angle in float64 must agree."""
    rng = np.random.default_rng(1)
    t, h, d = 64, 2, 128
    x = rng.standard_normal((t, h, d)).astype(np.float32)
    orig = rng.integers(0, 1_000_000, t).astype(np.int32)
    tgt = (rng.integers(0, 1_000_000) + np.arange(t)).astype(np.int32)
    got = rope_remap_ref(torch.from_numpy(x.copy()), torch.from_numpy(orig), torch.from_numpy(tgt),
                         500000.0).numpy()
    inv = inv_freq_table(d, 500000.0).numpy()
    ang = (np.float32(1) * (tgt - orig).astype(np.float32))[:, None] * inv[None, :]  # fp32 products
    ang = ang.astype(np.float32).astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = x[:, :, :64].astype(np.float64), x[:, :, 64:].astype(np.float64)
    want = np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], -1)
    assert np.abs(got - want).max() < 2e-6


def test_planted_sign_mistake_is_caught():
    """A remap with the sine's sign flipped (a plausible slip) fails the
    composition check, so that check pins the oracle."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((8, 2, 64))
    p, q = rng.integers(0, 1000, 8), rng.integers(0, 1000, 8)
    k = torch.from_numpy(rope_apply_f64(x, p, 10000.0)).float()
    wrong = rope_remap_ref(k.clone(), torch.from_numpy(q).int(), torch.from_numpy(p).int(), 10000.0)  # p<->q
    want = rope_apply_f64(x, q, 10000.0)
    assert np.abs(wrong.double().numpy() - want).max() > 0.1


def test_paged_form_equals_dense_form():
    pool = torch.randn(6, 4, 2, 2, 16, generator=torch.Generator().manual_seed(3))
    page_list = torch.tensor([4, 1, 5], dtype=torch.int32)
    t = 10
    orig = torch.arange(t, dtype=torch.int32) * 7
    tgt = torch.arange(t, dtype=torch.int32) + 100
    dense = torch.stack([pool[page_list[i // 4], i % 4, 0] for i in range(t)]).clone()
    rope_remap_ref(dense, orig, tgt, 10000.0)
    paged = rope_remap_pages_ref(pool.clone(), page_list, orig, tgt, 10000.0)
    for i in range(t):
        assert torch.equal(paged[page_list[i // 4], i % 4, 0], dense[i])
    # V and slots beyond the token count are untouched.
    assert torch.equal(paged[:, :, 1], pool[:, :, 1])
    assert torch.equal(paged[5, 2:, 0], pool[5, 2:, 0])
