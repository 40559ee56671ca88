"""NumPy restatement of the reference gated delta-rule (GDN) recurrence.

Test oracle only.  State is row-major ``[value_dim, key_dim]`` per value
head (qwen35_ops.py:318-323; ``RecurrentState`` delta matrix
``[Hv, Dv, Dk]``, memory.py:477-585; ROCm workspace orientation
``batch,value_head,value,key``, qwen35_rocm_ops.py:68).
"""

from __future__ import annotations

import math

import numpy as np


def key_head_for_value_head(value_head, key_heads):
    """``qwen35_ops.key_head_for_value_head`` (qwen35_ops.py:275-285):
    value head ``v`` reads key/query head ``v % key_heads``."""
    return value_head % key_heads


def gdn_step(state, queries, keys, values, beta, log_decay, acc=np.float64):
    """``qwen35_gdn_step`` NumPy fallback (qwen35_kernels.py:322-331).

    state ``[Hv, Dv, Dk]`` is updated IN PLACE (as the reference mutates
    its state view); queries/keys ``[Hk, Dk]``; values ``[Hv, Dv]``;
    beta/log_decay ``[Hv]``.  Per value head ``h`` with ``kh = h % Hk``::

        S <- exp(g) * S
        p  = S @ k
        S <- S + beta * (v - p) outer k
        o  = (S @ q) / sqrt(Dk)

    Returns ``o`` ``[Hv, Dv]``.
    """
    hv, dv, dk = state.shape
    hk = keys.shape[0]
    out = np.empty((hv, dv), dtype=acc)
    inv = 1.0 / math.sqrt(dk)
    for h in range(hv):
        kh = key_head_for_value_head(h, hk)
        k = np.asarray(keys[kh], dtype=acc)
        q = np.asarray(queries[kh], dtype=acc)
        s = state[h].astype(acc) * math.exp(float(log_decay[h]))
        pred = s @ k
        corr = float(beta[h]) * (np.asarray(values[h], dtype=acc) - pred)
        s += corr[:, None] * k[None, :]
        out[h] = (s @ q) * inv
        state[h] = s
    return out


def gdn_scan(state, queries, keys, values, betas, log_decays, acc=np.float64):
    """Token-sequential scan of ``gdn_step`` over a chunk, the only form the
    reference implements (qwen35_ops.gated_delta_net_scan,
    qwen35_ops.py:373-403; per-token ``qwen35_gdn_step`` calls from
    ``Qwen35NumpyModel._recurrent``, qwen35_numpy.py:115).

    state ``[Hv, Dv, Dk]`` (updated in place, kept in ``acc`` precision);
    queries/keys ``[T, Hk, Dk]``; values ``[T, Hv, Dv]``; betas/log_decays
    ``[T, Hv]``.  Returns outputs ``[T, Hv, Dv]``.
    """
    t_count = queries.shape[0]
    out = np.empty((t_count, state.shape[0], state.shape[1]), dtype=acc)
    for t in range(t_count):
        out[t] = gdn_step(state, queries[t], keys[t], values[t], betas[t],
                          log_decays[t], acc)
    return out


def gdn_step_scalar(state, query, key, value, beta, log_decay):
    """Pure-Python restatement of ``qwen35_ops.gated_delta_net_step``
    (qwen35_ops.py:309-370) for one value head, with its validation
    (beta in [0, 1], log_decay <= 0) and exact ``math.fsum`` reductions.
    Returns ``(output, new_state)`` and does not mutate ``state``."""
    beta = float(beta)
    log_decay = float(log_decay)
    if not math.isfinite(beta) or beta < 0.0 or beta > 1.0:
        raise ValueError("GDN beta must be finite and in [0, 1]")
    if not math.isfinite(log_decay) or log_decay > 0.0:
        raise ValueError("GDN log_decay must be finite and non-positive")
    decay = math.exp(log_decay)
    dk = len(state[0])
    decayed = [[float(x) * decay for x in row] for row in state]
    pred = [math.fsum(row[c] * float(key[c]) for c in range(dk)) for row in decayed]
    delta = [beta * (float(value[r]) - pred[r]) for r in range(len(decayed))]
    new = [[decayed[r][c] + delta[r] * float(key[c]) for c in range(dk)]
           for r in range(len(decayed))]
    scale = 1.0 / math.sqrt(dk)
    out = [math.fsum(row[c] * float(query[c]) for c in range(dk)) * scale
           for row in new]
    return out, new


def normalize_qk(queries, keys, epsilon):
    """``qwen35_normalize_qk`` NumPy fallback (qwen35_kernels.py:277-287):
    each head row divided by ``max(||row||_2, epsilon)``."""
    queries = np.asarray(queries, dtype=np.float32)
    keys = np.asarray(keys, dtype=np.float32)
    qd = np.maximum(np.sqrt(np.sum(queries * queries, axis=-1)), epsilon)
    kd = np.maximum(np.sqrt(np.sum(keys * keys, axis=-1)), epsilon)
    return queries / qd[..., None], keys / kd[..., None]


def beta_decay(beta_logits, alpha_logits, dt_bias, ssm_a):
    """``qwen35_beta_decay`` NumPy fallback (qwen35_kernels.py:290-307):
    ``beta = sigmoid(b)`` (two-branch stable form) and
    ``log_decay = softplus(alpha + dt_bias) * ssm_a`` with converted
    (negative) ``ssm_a = -exp(A_log)``."""
    b = np.asarray(beta_logits, dtype=np.float64)
    beta = np.where(b >= 0, 1.0 / (1.0 + np.exp(-np.abs(b))),
                    np.exp(-np.abs(b)) / (1.0 + np.exp(-np.abs(b))))
    x = np.asarray(alpha_logits, dtype=np.float64) + np.asarray(dt_bias, dtype=np.float64)
    dt = np.maximum(x, 0.0) + np.log1p(np.exp(-np.abs(x)))
    return beta.astype(np.float32), (dt * np.asarray(ssm_a, dtype=np.float64)).astype(np.float32)
