"""Drop-in for alpaccaroo's ``qwen35_kernels`` attention/recurrence wrappers.

Same names, argument order and layouts as the reference (qwen35_kernels.py):

* ``qwen35_full_attention_decode(queries [Hq, D], keys [T, Hkv, D],
  values [T, Hkv, Dv]) -> [Hq, Dv]`` (qwen35_kernels.py:363-392)

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


__all__ = ["available", "backend_name", "qwen35_full_attention_decode"]
