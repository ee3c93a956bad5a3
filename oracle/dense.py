"""Independent brute-force fp64 dense attention -- TEST INFRASTRUCTURE ONLY.

Used to pin ``reference_cpu.online_attention_statistics``: it materialises every
score at once and applies one masked softmax, so a mistake in the tiled online
recurrence (a dropped rescale, a wrong GQA head mapping, a transposed operand)
shows up as a mismatch. Mirrors the reference's own test oracle
(tests/unit/test_inference_online_attention.py:14-29): masked positions get
-inf, fully-masked rows produce 0.
"""

from __future__ import annotations

import numpy as np


def dense_attention(q, key, value, positions, *, key_positions=None, causal=True, window=None,
                    key_padding=None, query_padding=None, scale=None):
    """q ``[B, Hq, Q, D]``, key ``[B, Hkv, K, D]``, value ``[B, Hkv, K, Dv]`` (any float
    dtype, evaluated in float64); positions ``[B, Q]`` absolute; key positions
    default to ``0..K-1``. Returns ``[B, Hq, Q, Dv]`` float64."""
    q = np.asarray(q, dtype=np.float64)
    key = np.asarray(key, dtype=np.float64)
    value = np.asarray(value, dtype=np.float64)
    b, hq, nq, d = q.shape
    hkv, nk = key.shape[1], key.shape[2]
    groups = hq // hkv
    scale = d**-0.5 if scale is None else float(scale)
    k_full = np.repeat(key, groups, axis=1)
    v_full = np.repeat(value, groups, axis=1)
    scores = np.einsum("bhqd,bhkd->bhqk", q, k_full) * scale
    kpos = np.arange(nk) if key_positions is None else np.asarray(key_positions)
    positions = np.asarray(positions)
    mask = np.ones((b, nq, nk), dtype=bool)
    if causal:
        mask &= kpos[None, None, :] <= positions[:, :, None]
    if window is not None:
        mask &= kpos[None, None, :] > positions[:, :, None] - window
    if key_padding is not None:
        mask &= np.asarray(key_padding, dtype=bool)[:, None, :]
    if query_padding is not None:
        mask &= np.asarray(query_padding, dtype=bool)[:, :, None]
    mask = mask[:, None]
    scores = np.where(mask, scores, -np.inf)
    row_max = scores.max(-1, keepdims=True)
    row_max = np.where(np.isfinite(row_max), row_max, 0.0)
    weights = np.where(mask, np.exp(scores - row_max), 0.0)
    total = weights.sum(-1, keepdims=True)
    probs = np.where(total > 0, weights / np.where(total > 0, total, 1.0), 0.0)
    return probs @ v_full
