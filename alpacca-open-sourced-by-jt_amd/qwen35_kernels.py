"""Drop-in for alpaccaroo's ``qwen35_kernels`` attention/recurrence wrappers.

Same names, argument order and layouts as the reference (qwen35_kernels.py):

* ``qwen35_full_attention_decode(queries [Hq, D], keys [T, Hkv, D],
  values [T, Hkv, Dv]) -> [Hq, Dv]`` (qwen35_kernels.py:363-392)
* ``qwen35_full_attention_prefill(queries [Tq, Hq, D], keys, values,
  prefix_length=0) -> [Tq, Hq, Dv]``: token t attends to cache rows
  ``0 .. prefix_length + t`` (qwen35_kernels.py:395-411)

NumPy in -> NumPy out (upload, compute on the device, download); torch
device tensors in -> device tensor out.  All arithmetic runs in libalpx.so.
"""

from __future__ import annotations

import math

from . import _host, _ops


def available() -> bool:
    from .kernels import available as _available
    return _available()


def backend_name() -> str:
    return "hip-gfx950-libalpx"


def qwen35_full_attention_decode(queries, keys, values):
    host = _host.is_host(keys)
    K = _host.to_device(keys)
    V = _host.to_device(values, K.dtype)
    q = _host.to_device(queries, K.dtype)
    t, n_kv, d = (int(x) for x in K.shape)
    hq = int(q.shape[0])
    if hq % n_kv:
        raise ValueError("query heads must be a multiple of KV heads")
    dv = int(V.shape[2])
    out = _ops.decode(q.reshape(1, hq, d), K, V, length=t, k_strides=(n_kv * d, 0, d),
                      v_strides=(n_kv * dv, 0, dv), batch=1, kv_heads=n_kv,
                      scale=1.0 / math.sqrt(d))
    out = out.reshape(hq, dv)
    return _host.to_host(out) if host else out


def qwen35_full_attention_prefill(queries, keys, values, prefix_length: int = 0):
    host = _host.is_host(keys)
    K = _host.to_device(keys)
    V = _host.to_device(values, K.dtype)
    q = _host.to_device(queries, K.dtype)
    prefix_length = int(prefix_length)
    if prefix_length < 0:
        raise ValueError("prefix_length must be non-negative")
    if prefix_length + int(q.shape[0]) > int(K.shape[0]):
        raise ValueError("keys/values must hold prefix_length + query tokens rows")
    if int(q.shape[1]) % int(K.shape[1]):
        raise ValueError("query heads must be a multiple of KV heads")
    out = _ops.prefill(q, K, V, pos0=prefix_length, scale=1.0 / math.sqrt(int(q.shape[2])))
    return _host.to_host(out) if host else out


__all__ = ["available", "backend_name", "qwen35_full_attention_decode",
           "qwen35_full_attention_prefill"]
