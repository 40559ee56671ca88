"""Drop-in for the attention-path contracts of alpaccaroo's ``qwen35_ops``.

The reference module (alpaccaroo/qwen35_ops.py) states the Qwen3.5 hybrid
primitives as list-in / list-out scalar functions.  Three of them are on
this library's path, and this module serves them with the same names,
arguments, return values and error messages, computing on the GPU through
libalpx.so:

* ``gated_delta_net_step(state, query, key, value, *, beta, log_decay)``
  -> ``(output, new_state)`` for one value head, state row-major
  ``[value_dim][key_dim]`` (qwen35_ops.py:309-370);
* ``gated_delta_net_scan(state, queries, keys, values, betas, log_decays)``
  -> ``(outputs, final_state)``, the step applied token by token
  (qwen35_ops.py:373-403);
* ``causal_gqa_step(query_heads, key_cache, value_cache, *, scale=None)``
  -> ``[q_heads][value_dim]``, contiguous grouping ``h // (Hq / Hkv)``
  (qwen35_ops.py:406-472).

As in the reference, inputs are never mutated and every result is a fresh
list of Python floats.  The lists are validated here with the reference's
checks and messages, uploaded once as float32 device buffers, run by one
library call (the GDN step kernel, token after token for a scan; the
split-K decode for GQA), and downloaded.  The device arithmetic is float32
(the reference evaluates in Python floats with fsum), so results agree to
float32 accuracy, not bit for bit.  There is no host fallback: without the
library or a GPU the call raises.
"""

from __future__ import annotations

import math
from collections.abc import Sequence

import numpy as np

from . import _host, _ops


def _float_rows(rows) -> list[list[float]]:
    return [[float(item) for item in row] for row in rows]


def _floats(values) -> list[float]:
    return [float(item) for item in values]


def _check_gdn_scalars(beta: float, log_decay: float) -> None:
    # qwen35_ops.py:338-345
    if not math.isfinite(beta) or beta < 0.0 or beta > 1.0:
        raise ValueError(f"GDN beta must be finite and in [0, 1], got {beta!r}")
    if not math.isfinite(log_decay) or log_decay > 0.0:
        raise ValueError(
            "GDN log_decay must be finite and non-positive for converted ssm_a"
        )


def _check_gdn_token(matrix, q, k, v) -> None:
    # qwen35_ops.py:324-337
    value_dimension = len(matrix)
    key_dimension = len(matrix[0])
    if len(q) != key_dimension or len(k) != key_dimension:
        raise ValueError("GDN query/key lengths must equal the state key dimension")
    if len(v) != value_dimension:
        raise ValueError("GDN value length must equal the state value dimension")


def _state_matrix(state) -> list[list[float]]:
    matrix = _float_rows(state)
    if not matrix or not matrix[0]:
        raise ValueError("GDN state must have nonzero value and key dimensions")
    key_dimension = len(matrix[0])
    if any(len(row) != key_dimension for row in matrix):
        raise ValueError("GDN state rows must all have the same key dimension")
    return matrix


def _gdn_device(matrix, queries, keys, values, betas, log_decays):
    """Runs ``T`` GDN tokens of one value head on the device from a
    validated state; returns (outputs [T][Dv], state [Dv][Dk]) as lists."""
    torch = _host.torch_mod()
    dev = _host.device()
    tokens = len(queries)
    dv, dk = len(matrix), len(matrix[0])
    f32 = torch.float32

    def up(rows, shape):
        arr = np.asarray(rows, dtype=np.float32).reshape(shape)
        return torch.from_numpy(np.ascontiguousarray(arr)).to(dev)

    S = up(matrix, (1, 1, dv, dk))
    q = up(queries, (1, tokens, 1, dk))
    k = up(keys, (1, tokens, 1, dk))
    v = up(values, (1, tokens, 1, dv))
    beta = up(betas, (1, tokens, 1))
    g = up(log_decays, (1, tokens, 1))
    if tokens == 1:
        out = _ops.gdn_step(S, q[:, 0], k[:, 0], v[:, 0], beta[:, 0], g[:, 0], out_dtype=f32)
    else:
        out = _ops.gdn_chunk(S, q, k, v, beta, g, out_dtype=f32)
    outputs = out.reshape(tokens, dv).cpu().numpy().astype(np.float64)
    state = S.reshape(dv, dk).cpu().numpy().astype(np.float64)
    return outputs.tolist(), state.tolist()


def gated_delta_net_step(
    state: Sequence[Sequence[float]],
    query: Sequence[float],
    key: Sequence[float],
    value: Sequence[float],
    *,
    beta: float,
    log_decay: float,
) -> tuple[list[float], list[list[float]]]:
    """One Gated DeltaNet update of one value head (qwen35_ops.py:309-370):
    ``S <- e^g S``; ``S <- S + beta (v - S k) k^T``; output ``S q / sqrt(Dk)``.
    Returns ``(output, new_state)``; the prior state is not mutated."""
    matrix = _state_matrix(state)
    q, k, v = _floats(query), _floats(key), _floats(value)
    _check_gdn_token(matrix, q, k, v)
    beta, log_decay = float(beta), float(log_decay)
    _check_gdn_scalars(beta, log_decay)
    outputs, new_state = _gdn_device(matrix, [q], [k], [v], [beta], [log_decay])
    return outputs[0], new_state


def gated_delta_net_scan(
    state: Sequence[Sequence[float]],
    queries: Sequence[Sequence[float]],
    keys: Sequence[Sequence[float]],
    values: Sequence[Sequence[float]],
    betas: Sequence[float],
    log_decays: Sequence[float],
) -> tuple[list[list[float]], list[list[float]]]:
    """Causal scan of a token chunk through one value head's GDN state
    (qwen35_ops.py:373-403).  Returns ``(outputs, final_state)``."""
    count = len(queries)
    if not (len(keys) == count and len(values) == count and len(betas) == count
            and len(log_decays) == count):
        raise ValueError("GDN scan token-axis lengths must agree")
    if count == 0:
        # the reference returns the state unchanged without validating it
        return [], _float_rows(state)
    matrix = _state_matrix(state)
    qs, ks, vs = _float_rows(queries), _float_rows(keys), _float_rows(values)
    bs, gs = _floats(betas), _floats(log_decays)
    # the reference checks each token as it reaches it; all are checked
    # before anything runs, so a bad token raises the same error
    for index in range(count):
        _check_gdn_token(matrix, qs[index], ks[index], vs[index])
        _check_gdn_scalars(bs[index], gs[index])
    return _gdn_device(matrix, qs, ks, vs, bs, gs)


def causal_gqa_step(
    query_heads: Sequence[Sequence[float]],
    key_cache: Sequence[Sequence[Sequence[float]]],
    value_cache: Sequence[Sequence[Sequence[float]]],
    *,
    scale: float | None = None,
) -> list[list[float]]:
    """Causal GQA for one query token over an already-appended cache
    (qwen35_ops.py:406-472): query head ``h`` reads KV head ``h // group``;
    softmax over every cache token.  ``key_cache`` / ``value_cache`` are
    ``[tokens][kv_heads][dim]``."""
    queries = _float_rows(query_heads)
    keys = [_float_rows(token) for token in key_cache]
    values = [_float_rows(token) for token in value_cache]
    # validation and messages of qwen35_ops.py:436-460
    if not queries or not keys or len(keys) != len(values):
        raise ValueError("GQA requires queries and equal nonempty K/V caches")
    kv_heads = len(keys[0])
    if kv_heads <= 0 or len(queries) % kv_heads:
        raise ValueError("query heads must be a multiple of KV heads")
    if any(len(token) != kv_heads for token in keys + values):
        raise ValueError("every GQA cache token must have the same KV head count")
    key_dimension = len(queries[0])
    if key_dimension <= 0 or any(len(head) != key_dimension for head in queries):
        raise ValueError("GQA query heads must be nonempty and equally sized")
    if any(len(head) != key_dimension for token in keys for head in token):
        raise ValueError("GQA key heads must match the query head dimension")
    value_dimension = len(values[0][0])
    if value_dimension <= 0 or any(len(head) != value_dimension for token in values
                                   for head in token):
        raise ValueError("GQA value heads must be nonempty and equally sized")
    if scale is None:
        scale = 1.0 / math.sqrt(key_dimension)
    scale = float(scale)
    if not math.isfinite(scale) or scale <= 0.0:
        raise ValueError("GQA scale must be positive and finite")

    torch = _host.torch_mod()
    dev = _host.device()
    tokens, q_heads = len(keys), len(queries)

    def up(rows):
        return torch.from_numpy(np.ascontiguousarray(np.asarray(rows, dtype=np.float32))).to(dev)

    q = up(queries).reshape(1, q_heads, key_dimension)
    K = up(keys)    # [tokens, kv_heads, key_dim]: batch 1, llama layout
    V = up(values)
    out = _ops.decode(q, K, V, length=tokens, k_strides=(kv_heads * key_dimension, 0,
                                                          key_dimension),
                      v_strides=(kv_heads * value_dimension, 0, value_dimension), batch=1,
                      kv_heads=kv_heads, scale=scale)
    return out.reshape(q_heads, value_dimension).cpu().numpy().astype(np.float64).tolist()


__all__ = ["causal_gqa_step", "gated_delta_net_scan", "gated_delta_net_step"]
