"""RoPE remap oracle (test infrastructure only).

Restates ``_rope_remap_ref`` (kessie_hip_kernels.py:596-606) with the same
torch CPU operations in the same order, so the result is what the reference
function returns on the same torch build.
"""
from __future__ import annotations

import numpy as np
import torch


def inv_freq_table(head_dim: int, rope_theta: float) -> torch.Tensor:
    """fp32 [head_dim/2]: 1/(theta ** (arange(half)/half)) (kessie_hip_kernels.py:600)."""
    half = head_dim // 2
    return 1.0 / (rope_theta ** (torch.arange(half, dtype=torch.float32) / half))


def rope_remap_ref(k_tensor: torch.Tensor, orig_positions: torch.Tensor,
                   target_positions: torch.Tensor, rope_theta: float = 10000.0) -> torch.Tensor:
    """In place on k [T,H,D] (any float dtype); returns k.

    kessie_hip_kernels.py:596-606: delta = outer((tgt-orig).float(), freqs);
    k1*cos - k2*sin and k1*sin + k2*cos in fp32, then cast back.

    One deliberate difference: for an fp32 tensor the reference's ``.float()``
    returns the tensor's own storage, so its first assignment overwrites k1
    before the second line reads it (the second half is then computed from
    the rotated first half).  The reference's HIP kernel rotates both halves
    from the original pair (kessie_kernels_v2.hip:697-706); so does this
    oracle, by cloning.  For bf16/fp16 the clone changes nothing.
    """
    num_tokens, num_heads, head_dim = k_tensor.shape
    half = head_dim // 2
    freqs = inv_freq_table(head_dim, rope_theta).to(k_tensor.device)
    delta = torch.outer((target_positions - orig_positions).float(), freqs)
    cos_d, sin_d = delta.cos()[:, None, :], delta.sin()[:, None, :]
    k1, k2 = k_tensor[:, :, :half].float().clone(), k_tensor[:, :, half:].float().clone()
    k_tensor[:, :, :half] = (k1 * cos_d - k2 * sin_d).to(k_tensor.dtype)
    k_tensor[:, :, half:] = (k1 * sin_d + k2 * cos_d).to(k_tensor.dtype)
    return k_tensor


def rope_apply_f64(x: np.ndarray, positions: np.ndarray, rope_theta: float) -> np.ndarray:
    """Full rotate-half RoPE at absolute positions, float64 (closed-form check).

    Used to pin the remap against the identity remap(rope(k,p), p->q) == rope(k,q).
    x: [T,H,D] float64, positions: [T] int.
    """
    t, h, d = x.shape
    half = d // 2
    inv = 1.0 / (rope_theta ** (np.arange(half, dtype=np.float64) / half))
    ang = positions.astype(np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = x[:, :, :half], x[:, :, half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


def rope_remap_pages_ref(pool: torch.Tensor, page_list: torch.Tensor, orig: torch.Tensor,
                         tgt: torch.Tensor, rope_theta: float) -> torch.Tensor:
    """Paged form: remap K of tokens t -> (page_list[t//P], t%P) in a native pool
    [pages, P, 2, H, D]; in place on a CPU pool, returns it."""
    p = pool.shape[1]
    t = orig.shape[0]
    idx = torch.arange(t)
    pages = page_list.long()[idx // p]
    slots = idx % p
    k = pool[pages, slots, 0].clone()
    rope_remap_ref(k, orig, tgt, rope_theta)
    pool[pages, slots, 0] = k
    return pool

