"""Fog oracles (test infrastructure only).

Two fog definitions exist in the reference and both are on the path:
  * V-mode weights  w[pos] scaling V rows  (kessie_hip_kernels.py:403-413)
  * bias-mode logit bias b[pos] added to scores (kessie_attention.py:114-139)
Fog index = KV position, 0 = oldest.
"""
from __future__ import annotations

from typing import Iterable

import torch


def build_fog_weights(seq_len: int, fog_alpha: float = 0.5, fog_start: float = 0.5,
                      device=None) -> torch.Tensor:
    """kessie_build_fog_weights (kessie_hip_kernels.py:403-413), restated op for op.

    w = 1; c = int(N*(1-fs)); if alpha > 0 and c > 0: w[:c] = (arange(c)/max(c-1,1))**alpha.
    """
    weights = torch.ones(seq_len, dtype=torch.float32, device=device)
    clear_start = int(seq_len * (1.0 - fog_start))
    if fog_alpha > 0 and clear_start > 0:
        t = torch.arange(clear_start, dtype=torch.float32, device=device) / max(clear_start - 1, 1)
        weights[:clear_start] = t.pow(fog_alpha)
    return weights


def fog_bias(kv_len: int, fog_alpha: float, fog_start: float,
             recall_positions: Iterable[int] = (), recall_boost: float = 0.1,
             dtype: torch.dtype = torch.float32, alloc_len: int | None = None,
             device=None) -> torch.Tensor:
    """_FogCache._compute_into (kessie_attention.py:114-139), restated op for op.

    Returns buf[:kv_len] computed in ``dtype`` exactly as the reference does it
    (arange in that dtype, in-place mul_ chain), including the per-position
    recall overwrite.  ``alloc_len`` mimics the reference's larger buffer.
    ``device`` runs the same ops where the reference runs them in serving (on
    the query's device); torch's CPU kernel divides by the boundary where its
    device kernel multiplies by the fp32 reciprocal, so the two can differ in
    the last place.
    """
    n = max(kv_len, alloc_len or 0)
    buf = torch.zeros(n, dtype=dtype, device=device)
    fog_boundary = int(kv_len * (1.0 - fog_start))
    buf[:kv_len].zero_()
    if fog_boundary > 0:
        pos = torch.arange(fog_boundary, dtype=buf.dtype, device=buf.device)
        decay = (1.0 - pos / fog_boundary)
        decay.mul_(decay)
        decay.mul_(-fog_alpha)
        buf[:fog_boundary].copy_(decay)
    for p in recall_positions:
        if 0 <= p < kv_len:
            buf[p] = recall_boost
    return buf[:kv_len]
