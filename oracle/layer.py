"""NumPy restatement of the Qwen3.5 layer primitives around the hot path.

Test oracle only.  These are the reference's decomposed operations that
sit on either side of the attention and GDN kernels in one decode step of a
Qwen3.5 layer:

* full-attention prologue (qwen35_runtime.py:597-650): the joint query/gate
  projection split per head (``split_query_gate``,
  qwen35_rocm_ops.py:298-318), per-head Q/K RMSNorm (``rms_norm``,
  qwen35_ops.py:46-76), IMROPE at the text position (``imrope_rotate``,
  qwen35_ops.py:138-215) and the cache append;
* recurrent (GDN) layer (qwen35_numpy.py:63-131): depthwise causal
  convolution step with SiLU (``qwen35_conv_step``, qwen35_kernels.py:
  261-274; ``depthwise_causal_conv_step``, qwen35_ops.py:218-258), Q/K L2
  normalisation, beta / log-decay, the GDN step and the gated RMSNorm
  (``qwen35_gated_rms``, qwen35_kernels.py:335-352).

Everything is evaluated in float64 from the given (already rounded) inputs.
"""

from __future__ import annotations

import numpy as np

from . import gdn


def silu(x):
    """``x * sigmoid(x)`` with the stable two-branch sigmoid
    (qwen35_ops.silu, qwen35_ops.py:26-31; tensor.stable_sigmoid,
    tensor.py:123-129)."""
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(-np.abs(x))
    sig = np.where(x >= 0, 1.0 / (1.0 + e), e / (1.0 + e))
    return x * sig


def l2_normalize(x, eps):
    """``tensor.l2_normalize`` (tensor.py:139-158) over the last axis:
    ``x / max(||x||_2, eps)``; also ``Qwen35RocmOps.l2_normalize``
    (qwen35_rocm_ops.py:260-268)."""
    x = np.asarray(x, dtype=np.float64)
    den = np.maximum(np.sqrt(np.sum(x * x, axis=-1, keepdims=True)), eps)
    return x / den


def rms_norm(x, weight, eps):
    """``qwen35_ops.rms_norm`` (qwen35_ops.py:46-76) over the last axis:
    ``x / sqrt(mean(x * x) + eps) * weight``."""
    x = np.asarray(x, dtype=np.float64)
    den = np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x / den * np.asarray(weight, dtype=np.float64)


def gated_rms_norm(x, weight, gate, eps):
    """``qwen35_ops.gated_rms_norm`` (qwen35_ops.py:79-98) and
    ``qwen35_gated_rms`` (qwen35_kernels.py:335-352): RMSNorm, then times
    ``silu(gate)``; ``Qwen35RocmOps.recurrent_gate``
    (qwen35_rocm_ops.py:292-296)."""
    return rms_norm(x, weight, eps) * silu(gate)


def conv_step(current, weights, history, *, layout="kc", apply_silu=False):
    """One depthwise causal convolution step.

    ``current [..., C]``, ``history [..., K-1, C]`` oldest first; weights
    ``[K, C]`` (``layout="kc"``, GGUF / ROCm order, qwen35_ops.py:218-258,
    qwen35_rocm_ops.py:320-341) or ``[C, K]`` (``layout="ck"``, the
    qwen35_kernels order, qwen35_kernels.py:53-68, :261-274).  Returns
    ``(out, new_history)``; ``out[c] = sum_t window[t, c] * w[t, c]`` over
    the window ``history + [current]``, then SiLU when ``apply_silu``
    (qwen35_conv_step applies it, the ROCm op leaves it to ``silu``)."""
    w = np.asarray(weights, dtype=np.float64)
    if layout == "ck":
        w = w.T
    cur = np.asarray(current, dtype=np.float64)
    hist = np.asarray(history, dtype=np.float64)
    window = np.concatenate((hist, cur[..., None, :]), axis=-2)
    if window.shape[-2] != w.shape[0]:
        raise ValueError("convolution history must hold kernel - 1 rows")
    out = np.sum(window * w, axis=-2)
    if apply_silu:
        out = silu(out)
    return out, window[..., 1:, :]


def recurrent_parameters(beta_logits, alpha_logits, dt_bias, ssm_a):
    """``Qwen35RocmOps.recurrent_parameters`` (qwen35_rocm_ops.py:343-360):
    ``beta = sigmoid(beta_logits)``, ``log_decay = softplus(alpha_logits +
    dt_bias) * ssm_a`` with per-head ``dt_bias`` / ``ssm_a`` broadcast over
    the leading (batch) axes; the batched form of ``qwen35_beta_decay``."""
    b = np.asarray(beta_logits, dtype=np.float64)
    e = np.exp(-np.abs(b))
    beta = np.where(b >= 0, 1.0 / (1.0 + e), e / (1.0 + e))
    x = np.asarray(alpha_logits, dtype=np.float64) + np.asarray(dt_bias, dtype=np.float64)
    dt = np.maximum(x, 0.0) + np.log1p(np.exp(-np.abs(x)))
    return beta, dt * np.asarray(ssm_a, dtype=np.float64)


def imrope_lane(pair, sections):
    """``qwen35_ops.imrope_lane_for_pair`` (qwen35_ops.py:138-157): the
    interleaved T/H/W/E position lane of rotary pair ``pair``."""
    s0, s1, s2, _ = sections
    sector = pair % sum(sections)
    if sector % 3 == 1 and sector < 3 * s1:
        return 1
    if sector % 3 == 2 and sector < 3 * s2:
        return 2
    if sector % 3 == 0 and sector < 3 * s0:
        return 0
    return 3


def imrope(values, lanes, sections, base, scale=1.0):
    """``qwen35_ops.imrope_rotate`` (qwen35_ops.py:159-215) over the last
    axis of ``values``: pair ``p < R = sum(sections)`` rotates coordinates
    ``(p, p + R)`` (NeoX half split) by ``theta = lanes[lane(p)] * scale *
    base ** (-2 p / (2 R))``; coordinates ``>= 2 R`` are copied.
    ``lanes`` is either one 4-vector or an array ``[..., 4]`` matching the
    leading axes of ``values`` (without the last one) or broadcastable to them."""
    v = np.array(values, dtype=np.float64, copy=True)
    rp = int(sum(sections))
    rd = 2 * rp
    if v.shape[-1] < rd:
        raise ValueError("IMROPE input is shorter than 2 * sum(sections)")
    lanes = np.asarray(lanes, dtype=np.float64)
    first = v[..., :rp].copy()
    second = v[..., rp:rd].copy()
    for p in range(rp):
        lane = imrope_lane(p, sections)
        pos = lanes[..., lane]
        theta = pos * scale * float(base) ** (-2.0 * p / rd)
        c, s = np.cos(theta), np.sin(theta)
        v[..., p] = first[..., p] * c - second[..., p] * s
        v[..., rp + p] = first[..., p] * s + second[..., p] * c
    return v


def text_lanes(position):
    """``qwen35_ops.imrope_text_position`` (qwen35_ops.py:102-108):
    lanes ``(p, p, p, 0)`` for a text token at ``position``."""
    p = np.asarray(position, dtype=np.float64)
    return np.stack([p, p, p, np.zeros_like(p)], axis=-1)


def split_query_gate(projected, heads, dim):
    """``Qwen35RocmOps.split_query_gate`` (qwen35_rocm_ops.py:298-318): the
    joint projection's last axis holds, per head, ``dim`` query values then
    ``dim`` gate values."""
    p = np.asarray(projected)
    r = p.reshape(p.shape[:-1] + (heads, 2 * dim))
    return r[..., :dim].copy(), r[..., dim:].copy()


def attention_prologue(query_gate, key, value, q_norm, k_norm, eps, positions, sections,
                       base):
    """Qwen3.5 full-attention decode prologue (qwen35_runtime.py:597-650)
    for a batch of sequences, one token each: split the joint projection
    ``query_gate [B, Hq * 2 D]``, RMSNorm every query head with ``q_norm``
    and every key head of ``key [B, Hkv * D]`` with ``k_norm``, rotate both
    with IMROPE at the text position ``positions[b]``.  Returns
    ``(query [B, Hq, D], gate [B, Hq, D], key_rot [B, Hkv, D],
    value [B, Hkv, Dv])``; the caller appends key_rot / value at
    ``positions[b]``."""
    key = np.asarray(key, dtype=np.float64)
    value = np.asarray(value, dtype=np.float64)
    b = key.shape[0]
    d = np.asarray(q_norm).shape[0]
    hq = np.asarray(query_gate).shape[-1] // (2 * d)
    q, g = split_query_gate(np.asarray(query_gate, dtype=np.float64), hq, d)
    k = key.reshape(b, -1, d)
    lanes = text_lanes(np.asarray(positions))[:, None, :]
    qn = imrope(rms_norm(q, q_norm, eps), lanes, sections, base)
    kn = imrope(rms_norm(k, k_norm, eps), lanes, sections, base)
    return qn, g, kn, value.reshape(b, k.shape[1], -1)


def recurrent_layer_step(mixed, conv_w, history, gate, beta_logits, alpha_logits, dt_bias,
                         ssm_a, norm_weight, state, *, key_heads, key_dim, value_heads,
                         value_dim, eps):
    """One token of the Qwen3.5 recurrent (GDN) layer for a batch,
    qwen35_numpy.py:63-131 after the projections: ``conv_step`` + SiLU of
    ``mixed [B, C]`` with ``conv_w [K, C]`` and ``history [B, K-1, C]``,
    split into q ``[Hk, Dk]``, k ``[Hk, Dk]``, v ``[Hv, Dv]``, L2-normalised
    q / k (``qwen35_normalize_qk``), ``recurrent_parameters``, the GDN step
    on ``state [B, Hv, Dv, Dk]`` (updated in place), and the gated RMSNorm
    with ``gate [B, Hv * Dv]`` and ``norm_weight [Dv]``.  Returns
    ``(out [B, Hv * Dv], new_history)``."""
    mixed = np.asarray(mixed, dtype=np.float64)
    bsz = mixed.shape[0]
    act, new_hist = conv_step(mixed, conv_w, history, apply_silu=True)
    w = key_heads * key_dim
    out = np.empty((bsz, value_heads * value_dim))
    beta, g = recurrent_parameters(beta_logits, alpha_logits, dt_bias, ssm_a)
    for b in range(bsz):
        q = act[b, :w].reshape(key_heads, key_dim)
        k = act[b, w:2 * w].reshape(key_heads, key_dim)
        v = act[b, 2 * w:].reshape(value_heads, value_dim)
        q = l2_normalize(q, eps)
        k = l2_normalize(k, eps)
        st = state[b]
        o = gdn.gdn_step(st, q, k, v, beta[b], g[b])
        gt = np.asarray(gate[b], dtype=np.float64).reshape(value_heads, value_dim)
        out[b] = gated_rms_norm(o, norm_weight, gt, eps).reshape(-1)
    return out, new_hist


def attention_layer_prefill(query_gate, key, value, q_norm, k_norm, eps, position, sections,
                            base, key_cache, value_cache, *, round_rows=None):
    """The reference's token-sequential prefill of one Qwen3.5 full-attention
    layer after its projections (Qwen35Model.prefill_state ->
    forward_token -> _attention per token, qwen35_runtime.py:597-665,
    777-810) for one sequence: token t of ``query_gate [T, Hq * 2 D]``,
    ``key [T, Hkv * D]``, ``value [T, Hkv * Dv]`` runs the decode prologue at
    position ``position + t``, appends its rotated key / value at that cache
    row (``key_cache [cap, Hkv, D]``, ``value_cache [cap, Hkv, Dv]``, updated
    in place), attends over rows ``0 .. position + t`` and applies the
    sigmoid gate.  ``round_rows`` (e.g. a bf16 rounding function) is applied
    to each appended key / value row, as a cache of that dtype stores it.
    Returns ``[T, Hq, Dv]``."""
    from . import attention as A
    query_gate = np.asarray(query_gate, dtype=np.float64)
    tokens = query_gate.shape[0]
    d = np.asarray(q_norm).shape[0]
    hkv = np.asarray(key).shape[1] // d
    out = []
    for t in range(tokens):
        pos = position + t
        q, g, kr, v = attention_prologue(query_gate[t:t + 1], np.asarray(key)[t:t + 1],
                                         np.asarray(value)[t:t + 1], q_norm, k_norm, eps,
                                         [pos], sections, base)
        krow, vrow = kr[0], v[0]
        if round_rows is not None:
            krow, vrow = round_rows(krow), round_rows(vrow)
        key_cache[pos] = krow
        value_cache[pos] = vrow
        hq = q.shape[1]
        att = A.attention_decode_twopass(q[0].reshape(-1), key_cache[:pos + 1],
                                         value_cache[:pos + 1], hq // hkv, 1.0 / np.sqrt(d))
        out.append(A.sigmoid_gate(att, g[0]))
    return np.stack(out)


def recurrent_layer_prefill(mixed, conv_w, history, gate, beta_logits, alpha_logits, dt_bias,
                            ssm_a, norm_weight, state, *, key_heads, key_dim, value_heads,
                            value_dim, eps, round_qkv=None):
    """The reference's token-sequential prefill of one Qwen3.5 recurrent
    layer after its projections (the per-token chain of
    qwen35_numpy.py:63-131 run once per token by prefill_state,
    qwen35_runtime.py:777-810) for one sequence: ``recurrent_layer_step``
    on token t of ``mixed [T, C]``, ``gate [T, Hv * Dv]`` and the logits
    ``[T, Hv]``, carrying ``history [K-1, C]`` and ``state [Hv, Dv, Dk]``
    (updated in place).  ``round_qkv`` (e.g. bf16 rounding) is applied to
    the normalised q / k and to v before the GDN step, as a path that feeds
    the recurrence in that dtype does.  Returns ``(out [T, Hv * Dv],
    new_history)``."""
    mixed = np.asarray(mixed, dtype=np.float64)
    hist = np.asarray(history, dtype=np.float64)[None].copy()
    st = state[None]
    outs = []
    for t in range(mixed.shape[0]):
        if round_qkv is None:
            o, hist = recurrent_layer_step(
                mixed[t:t + 1], conv_w, hist, np.asarray(gate)[t:t + 1],
                np.asarray(beta_logits)[t:t + 1], np.asarray(alpha_logits)[t:t + 1], dt_bias,
                ssm_a, norm_weight, st, key_heads=key_heads, key_dim=key_dim,
                value_heads=value_heads, value_dim=value_dim, eps=eps)
        else:
            act, hist = conv_step(mixed[t:t + 1], conv_w, hist, apply_silu=True)
            w = key_heads * key_dim
            q = round_qkv(l2_normalize(act[0, :w].reshape(key_heads, key_dim), eps))
            k = round_qkv(l2_normalize(act[0, w:2 * w].reshape(key_heads, key_dim), eps))
            v = round_qkv(act[0, 2 * w:].reshape(value_heads, value_dim))
            beta, g = recurrent_parameters(np.asarray(beta_logits)[t:t + 1],
                                           np.asarray(alpha_logits)[t:t + 1], dt_bias, ssm_a)
            og = gdn.gdn_step(st[0], q, k, v, beta[0], g[0])
            gt = np.asarray(gate, dtype=np.float64)[t].reshape(value_heads, value_dim)
            o = gated_rms_norm(og, norm_weight, gt, eps).reshape(1, -1)
        outs.append(o[0])
    return np.stack(outs), hist[0]
