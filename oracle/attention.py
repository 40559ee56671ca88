"""NumPy restatement of the reference attention path (test oracle only).

Every function cites the reference lines it restates.  Arithmetic defaults
to float64 on the exact (already rounded) input values, which is the
"fp64 accumulation" oracle: it differs from the reference's float32 BLAS
results by ~1e-6, far inside the parity tolerances (fp32 1e-4, fp16/bf16
2e-2).  Pass ``acc=np.float32`` to evaluate in the reference's own
precision (used by the CPU baseline timing).
"""

from __future__ import annotations

import math

import numpy as np


# ---------------------------------------------------------------- KV append

def attention_append(key_cache, value_cache, position, key, value):
    """``Qwen35RocmOps.attention_append_`` (qwen35_rocm_ops.py:475-500).

    Caches are ``[capacity, batch, kv_heads, dim]``; key/value are one token
    ``[batch, kv_heads, dim]``.  Writes row ``position`` in place and returns
    ``position + 1``.  Raises ``ValueError`` exactly where the reference does.
    """
    if isinstance(position, bool) or not isinstance(position, int) or position < 0:
        raise ValueError("attention cache position must be a non-negative integer")
    if key_cache.shape[0] != value_cache.shape[0]:
        raise ValueError("attention K/V cache capacities differ")
    if position >= key_cache.shape[0]:
        raise ValueError("attention cache position exceeds capacity")
    if key_cache.shape[1:3] != value_cache.shape[1:3]:
        raise ValueError("attention K/V cache batch and head axes differ")
    if tuple(key.shape) != tuple(key_cache.shape[1:]):
        raise ValueError("attention key does not match cache token shape")
    if tuple(value.shape) != tuple(value_cache.shape[1:]):
        raise ValueError("attention value does not match cache token shape")
    key_cache[position] = key
    value_cache[position] = value
    return position + 1


def ragged_append(key_cache, value_cache, positions, key, value):
    """Per-sequence append for a ragged batch: sequence ``b`` writes its
    ``key[t, b]`` rows at ``positions[b] + t`` of cache ``[C, B, Hkv, D]``.

    This is the ragged extension of ``attention_append_``
    (qwen35_rocm_ops.py:475-500), whose single ``position`` is the special
    case ``positions[b] == position`` for all ``b`` and ``T == 1``.
    """
    t_count = key.shape[0]
    for b, p in enumerate(positions):
        p = int(p)
        if p < 0 or p + t_count > key_cache.shape[0]:
            raise ValueError("attention cache position exceeds capacity")
        key_cache[p:p + t_count, b] = key[:, b]
        value_cache[p:p + t_count, b] = value[:, b]
    return key_cache, value_cache


# ---------------------------------------------------------------- decode

def attention_decode_twopass(q, K, V, group, inv_sqrt, acc=np.float64):
    """Llama-class single-token GQA, NumPy branch of ``Model._attention_np``
    (model.py:1246-1252); same contract as ``kernels.attention_decode``
    (kernels.py:1183-1200).

    q is flat ``(n_head*hd,)`` or ``(n_head, hd)``; K, V are ``(t, n_kv, hd)``.
    Returns ``(n_head, hd)``: ``softmax(q.K^T * inv_sqrt) . V`` with head ``h``
    reading kv head ``h // group``.
    """
    K = np.asarray(K, dtype=acc)
    V = np.asarray(V, dtype=acc)
    t, n_kv, hd = K.shape
    qg = np.asarray(q, dtype=acc).reshape(n_kv, group, hd)
    scores = np.matmul(qg, K.transpose(1, 2, 0)) * acc(inv_sqrt)
    scores = scores - scores.max(axis=2, keepdims=True)
    w = np.exp(scores)
    w = w / w.sum(axis=2, keepdims=True)
    out = np.matmul(w, V.transpose(1, 0, 2))
    return out.reshape(n_kv * group, V.shape[2])


def full_attention_decode_online(queries, keys, values, scale=None,
                                 acc=np.float64):
    """``qwen35_full_attention_decode`` NumPy fallback
    (qwen35_kernels.py:363-392): an online (running max / running sum)
    softmax over cache positions, one query head at a time.

    queries ``[Hq, D]``, keys ``[T, Hkv, D]``, values ``[T, Hkv, Dv]``.
    Contiguous grouping ``kv = h // (Hq // Hkv)``; scale ``1/sqrt(D)``.
    """
    queries = np.asarray(queries, dtype=acc)
    keys = np.asarray(keys, dtype=acc)
    values = np.asarray(values, dtype=acc)
    hq, d = queries.shape
    group = hq // keys.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = np.zeros((hq, values.shape[2]), dtype=acc)
    for h in range(hq):
        kv = h // group
        maximum = -math.inf
        denominator = 0.0
        row = out[h]
        for position in range(keys.shape[0]):
            score = float(queries[h] @ keys[position, kv]) * scale
            nxt = max(maximum, score)
            old = math.exp(maximum - nxt)
            new = math.exp(score - nxt)
            row *= old
            row += values[position, kv] * new
            denominator = denominator * old + new
            maximum = nxt
        row /= denominator
    return out


def online_attention(query, key_cache, value_cache, length, scale=None,
                     seq_lens=None, acc=np.float64):
    """``Qwen35RocmOps.online_attention`` (qwen35_rocm_ops.py:502-564).

    query ``[B, Hq, D]``; caches ``[C, B, Hkv, D|Dv]``; attends to cache rows
    ``0 .. length-1`` (all sequences) and returns ``[B, Hq, Dv]``.  The
    reference's per-position online recurrence is evaluated here in its
    closed two-pass form, which it equals exactly in real arithmetic
    (pinned by ``tests/test_oracle.py``).

    ``seq_lens`` (ragged extension): sequence ``b`` attends to its first
    ``seq_lens[b]`` rows instead of ``length``.
    """
    query = np.asarray(query)
    bsz, hq, d = query.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    kv_heads = key_cache.shape[2]
    group = hq // kv_heads
    out = np.empty((bsz, hq, value_cache.shape[3]), dtype=acc)
    for b in range(bsz):
        n = int(length if seq_lens is None else seq_lens[b])
        out[b] = attention_decode_twopass(
            query[b], key_cache[:n, b], value_cache[:n, b], group, scale, acc)
    return out


# ---------------------------------------------------------------- prefill

def attention_batch(q, K, V, positions, group, inv_sqrt, window=0, kv_start=0,
                    acc=np.float64):
    """Causal GQA of ``Model._attention_batch_np`` (model.py:1254-1272) and
    its windowed form ``_attention_batch_window_np`` (model.py:1567-1592):
    key index ``j`` sits at absolute position ``kv_start + j`` and query row
    ``t`` (absolute position ``positions[t]``) sees it iff
    ``kv_start + j <= positions[t]`` and, when ``window > 0``,
    ``kv_start + j > positions[t] - window``.  Allowed scores go through the
    usual max-subtracted softmax; disallowed ones get weight exactly 0.

    A row with no allowed key returns zeros, the convention of the device
    seam this path replaces (``cuda.attention_batch`` ->
    ``_attention_batch_gqa``, cuda.py:572-577).

    q ``(t_q, n_head, hd)``, K/V ``(t_kv, n_kv, hd)``; returns
    ``(t_q, n_head, hd)``.  Processed in query blocks so a 2048 x 4096
    problem never materialises the full score tensor at once.
    """
    q = np.asarray(q, dtype=acc)
    K = np.asarray(K, dtype=acc)
    V = np.asarray(V, dtype=acc)
    t_q, n_head, hd = q.shape
    n_kv = K.shape[1]
    positions = np.asarray(positions, dtype=np.int64)
    out = np.empty((t_q, n_head, V.shape[2]), dtype=acc)
    Kt = K.transpose(1, 2, 0)            # (kv, hd, s)
    Vt = V.transpose(1, 0, 2)            # (kv, s, hd)
    block = 128
    kv_pos = kv_start + np.arange(K.shape[0])
    for t0 in range(0, t_q, block):
        t1 = min(t_q, t0 + block)
        qg = q[t0:t1].reshape(t1 - t0, n_kv, group, hd).transpose(1, 0, 2, 3)
        scores = np.matmul(qg.reshape(n_kv, -1, hd), Kt) * acc(inv_sqrt)
        scores = scores.reshape(n_kv, t1 - t0, group, -1)
        allowed = kv_pos[None, :] <= positions[t0:t1, None]
        if window > 0:
            allowed &= kv_pos[None, :] > positions[t0:t1, None] - window
        scores = np.where(allowed[None, :, None, :], scores, -np.inf)
        m = scores.max(axis=-1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        w = np.exp(scores - m)
        den = w.sum(axis=-1, keepdims=True)
        w = w / np.where(den > 0, den, 1.0)
        o = np.matmul(w.reshape(n_kv, -1, K.shape[0]), Vt)
        o = o.reshape(n_kv, t1 - t0, group, -1).transpose(1, 0, 2, 3)
        out[t0:t1] = o.reshape(t1 - t0, n_head, -1)
    return out


def full_attention_prefill(queries, keys, values, prefix_length=0,
                           acc=np.float64):
    """``qwen35_full_attention_prefill`` (qwen35_kernels.py:395-411): token
    ``t`` of the chunk attends to cache rows ``0 .. prefix_length + t``."""
    positions = prefix_length + np.arange(np.asarray(queries).shape[0])
    group = queries.shape[1] // keys.shape[1]
    return attention_batch(queries, keys, values, positions, group,
                           1.0 / math.sqrt(queries.shape[2]), acc=acc)


# ---------------------------------------------------------------- gate

def stable_sigmoid(x):
    """Two-branch sigmoid of ``tensor.stable_sigmoid`` (tensor.py:123-129),
    vectorised; never overflows for large finite inputs."""
    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    pos = x >= 0.0
    z = np.exp(-x[pos])
    out[pos] = 1.0 / (1.0 + z)
    z = np.exp(x[~pos])
    out[~pos] = z / (1.0 + z)
    return out


def sigmoid_gate(values, gate):
    """``Qwen35RocmOps.sigmoid_gate`` (qwen35_rocm_ops.py:286-290) and the
    gating step of ``Qwen35Model._attention`` (qwen35_runtime.py:653-660):
    ``values * sigmoid(gate)`` elementwise."""
    return np.asarray(values, dtype=np.float64) * stable_sigmoid(gate)


# ---------------------------------------------------------------- scalar

def causal_gqa_step_scalar(query_heads, key_cache, value_cache, scale=None):
    """Pure-Python restatement of ``qwen35_ops.causal_gqa_step``
    (qwen35_ops.py:406-472): exact ``math.fsum`` reductions, for tiny
    brute-force cross-checks.  key/value caches are ``[T][Hkv][D]``."""
    queries = [[float(v) for v in h] for h in query_heads]
    kv_heads = len(key_cache[0])
    d = len(queries[0])
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    group = len(queries) // kv_heads
    result = []
    for qi, query in enumerate(queries):
        kv = qi // group
        scores = [math.fsum(a * float(b) for a, b in zip(query, tok[kv])) * scale
                  for tok in key_cache]
        m = max(scores)
        ex = [math.exp(s - m) for s in scores]
        den = math.fsum(ex)
        probs = [e / den for e in ex]
        dv = len(value_cache[0][0])
        result.append([
            math.fsum(probs[t] * float(value_cache[t][kv][c])
                      for t in range(len(value_cache)))
            for c in range(dv)
        ])
    return result


def paged_rows(pages, block_table, batch_index, length):
    """Logical rows ``0 .. length - 1`` of sequence ``batch_index`` of a paged
    cache ``pages [P, page_size, Hkv, D]`` under ``block_table [B, max_pages]``
    (row j = row j % page_size of page block_table[b, j // page_size]):
    the contiguous ``[length, Hkv, D]`` rows the same attention reads."""
    pages = np.asarray(pages)
    size = pages.shape[1]
    rows = [pages[block_table[batch_index][j // size], j % size] for j in range(length)]
    return np.stack(rows) if rows else pages[:0, 0]
