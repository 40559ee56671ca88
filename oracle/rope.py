"""Llama-class rotary embedding used to build the prefill inputs (oracle).

Restates the "norm" (adjacent-pair) style of the reference:
inverse frequencies ``freq_scale * base ** (-2 i / n_rot)`` in float32
(model.py:320-323), per-position cos/sin tables from
``arange(n_ctx) * inv_freq`` (model.py:866-874), and the batched rotation
``_rope_batch_np`` (model.py:1192-1210) with pairs ``(2i, 2i+1)``.
"""

from __future__ import annotations

import numpy as np


def rope_tables(n_ctx, n_rot, base, freq_scale=1.0):
    half = n_rot // 2
    inv_freq = (np.float32(freq_scale)
                * np.float32(base) ** (-2.0 * np.arange(half, dtype=np.float32) / n_rot)
                ).astype(np.float32)
    theta = np.arange(n_ctx, dtype=np.float32)[:, None] * inv_freq[None, :]
    return np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)


def rope_norm_batch(vecs, positions, cos, sin, n_rot=None):
    """Rotate ``vecs[t, head, :]`` at absolute ``positions[t]``; adjacent
    pairs ``(2i, 2i+1)`` for ``i < n_rot/2``; dims past ``n_rot`` untouched."""
    v = np.array(vecs, dtype=np.float32, copy=True)
    hd = v.shape[-1]
    n_rot = hd if n_rot is None else n_rot
    c = cos[positions][:, None, :]
    s = sin[positions][:, None, :]
    x0 = v[:, :, 0:n_rot:2].copy()
    x1 = v[:, :, 1:n_rot:2].copy()
    v[:, :, 0:n_rot:2] = x0 * c - x1 * s
    v[:, :, 1:n_rot:2] = x0 * s + x1 * c
    return v
