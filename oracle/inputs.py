"""Seeded synthetic inputs for the five benchmark configurations (oracle).

Rules: ``rng = numpy.random.default_rng(seed)`` with seed = config number;
arrays are drawn in the order listed in each generator, as float32 N(0, 1),
then rounded ONCE to the config dtype with round-to-nearest-even.  The
generators return float32 arrays holding exactly representable values plus
the storage-dtype name, so the oracle and the kernel read identical numbers.
"""

from __future__ import annotations

import math

import numpy as np

from . import gdn as _gdn
from . import rope as _rope


# ------------------------------------------------------------ rounding

def f32_to_bf16_bits(x):
    """float32 -> bfloat16 bit patterns (uint16), round-to-nearest-even.
    NaN stays NaN (quietened)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    rounded = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = rounded.copy()
        rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_bits_to_f32(bits):
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_to(x, dtype):
    """Round float32 values to ``dtype`` in {'f32', 'f16', 'bf16'} and return
    them as float32 (exactly representable in ``dtype``)."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    raise ValueError(f"unknown dtype {dtype!r}")


def _normal(rng, shape):
    return rng.standard_normal(size=shape, dtype=np.float32)


# ------------------------------------------------------------ configs

def c1_decode_fp32(seed=1, ctx=512, n_head=32, n_kv=8, hd=64):
    """C1: GQA decode, Llama-3.2-1B shape, fp32.  Draw order q, K, V."""
    rng = np.random.default_rng(seed)
    q = _normal(rng, (n_head, hd))
    K = _normal(rng, (ctx, n_kv, hd))
    V = _normal(rng, (ctx, n_kv, hd))
    return {"q": q, "K": K, "V": V, "group": n_head // n_kv,
            "scale": 1.0 / math.sqrt(hd), "dtype": "f32"}


def c2_decode_fp16(seed=2, batch=16, capacity=8192, n_head=32, n_kv=8, hd=128,
                   uniform=False, lo=1024, hi=8192):
    """C2: GQA decode, Llama-3-8B shape, fp16, ROCm cache layout
    ``[capacity, batch, n_kv, hd]``.  Draw order: lengths
    (``rng.integers(lo, hi + 1, batch)``), q ``[B, Hq, D]``, K, V."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, batch).astype(np.int32)
    if uniform:
        lens[:] = capacity
    lens = np.minimum(lens, capacity)
    q = round_to(_normal(rng, (batch, n_head, hd)), "f16")
    K = round_to(_normal(rng, (capacity, batch, n_kv, hd)), "f16")
    V = round_to(_normal(rng, (capacity, batch, n_kv, hd)), "f16")
    return {"q": q, "K": K, "V": V, "seq_lens": lens, "group": n_head // n_kv,
            "scale": 1.0 / math.sqrt(hd), "dtype": "f16"}


def c3_prefill_bf16(seed=3, prefix=2048, chunk=2048, n_head=32, n_kv=8, hd=128,
                    theta=500000.0):
    """C3: causal prefill of a ``chunk``-token bf16 chunk on a ``prefix``-row
    bf16 cache.  Draw order: cache K, cache V, chunk q, chunk k, chunk v.
    RoPE (norm style, base ``theta``) is applied in float32 to the cache K
    (positions 0..prefix-1) and to the chunk q/k (positions prefix..), then
    everything is rounded to bf16."""
    rng = np.random.default_rng(seed)
    total = prefix + chunk
    cos, sin = _rope.rope_tables(total, hd, theta)
    k_cache = _normal(rng, (prefix, n_kv, hd))
    v_cache = _normal(rng, (prefix, n_kv, hd))
    q = _normal(rng, (chunk, n_head, hd))
    k_new = _normal(rng, (chunk, n_kv, hd))
    v_new = _normal(rng, (chunk, n_kv, hd))
    pos_cache = np.arange(prefix)
    pos_new = np.arange(prefix, total)
    if prefix:
        k_cache = _rope.rope_norm_batch(k_cache, pos_cache, cos, sin)
    q = _rope.rope_norm_batch(q, pos_new, cos, sin)
    k_new = _rope.rope_norm_batch(k_new, pos_new, cos, sin)
    r = lambda a: round_to(a, "bf16")  # noqa: E731
    return {"k_cache": r(k_cache), "v_cache": r(v_cache), "q": r(q),
            "k_new": r(k_new), "v_new": r(v_new), "prefix": prefix,
            "group": n_head // n_kv, "scale": 1.0 / math.sqrt(hd),
            "dtype": "bf16"}


def c4_decode_gated_bf16(seed=4, batch=4, ctx=32768, n_head=16, n_kv=2, hd=256):
    """C4: Qwen3.5 full-attention decode with sigmoid output gate, bf16,
    ROCm cache layout ``[ctx, batch, n_kv, hd]``.  Draw order q, K, V, gate."""
    rng = np.random.default_rng(seed)
    q = round_to(_normal(rng, (batch, n_head, hd)), "bf16")
    K = round_to(_normal(rng, (ctx, batch, n_kv, hd)), "bf16")
    V = round_to(_normal(rng, (ctx, batch, n_kv, hd)), "bf16")
    gate = round_to(_normal(rng, (batch, n_head, hd)), "bf16")
    return {"q": q, "K": K, "V": V, "gate": gate, "group": n_head // n_kv,
            "scale": 1.0 / math.sqrt(hd), "dtype": "bf16"}


def c5_gdn_bf16(seed=5, tokens=1280, hk=16, hv=32, dk=128, dv=128, eps=1e-6, dtype="bf16"):
    """C5: gated delta rule inputs.  Draw order: q ``[T, Hk, Dk]``, k, v
    ``[T, Hv, Dv]``, beta logits ``[T, Hv]``, a ``[Hv]`` ~ U(-1, 1),
    x ``[T, Hv]``.  q/k are L2-normalised per head (qwen35_normalize_qk,
    qwen35_kernels.py:277-287) then rounded to ``dtype`` (bf16 for C5;
    "f32" keeps the fp32 values); v is rounded likewise;
    ``beta = sigmoid(logits)`` and ``g = -exp(a) * softplus(x)``
    (qwen35_beta_decay with dt_bias = 0, qwen35_kernels.py:290-307) stay
    float32."""
    rng = np.random.default_rng(seed)
    q = _normal(rng, (tokens, hk, dk))
    k = _normal(rng, (tokens, hk, dk))
    v = _normal(rng, (tokens, hv, dv))
    b = _normal(rng, (tokens, hv))
    a = rng.uniform(-1.0, 1.0, size=hv).astype(np.float32)
    x = _normal(rng, (tokens, hv))
    qn, kn = _gdn.normalize_qk(q, k, eps)
    ssm_a = -np.exp(a.astype(np.float64)).astype(np.float32)
    beta, g = _gdn.beta_decay(b, x, np.zeros(hv, np.float32), ssm_a[None, :])
    return {"q": round_to(qn, dtype), "k": round_to(kn, dtype),
            "v": round_to(v, dtype), "beta": beta.astype(np.float32),
            "g": g.astype(np.float32), "dtype": dtype}
