"""Drop-in for alpaccaroo's ``qwen35_kernels`` attention/recurrence wrappers.

Same names, argument order and layouts as the reference (qwen35_kernels.py):

* ``qwen35_full_attention_decode(queries [Hq, D], keys [T, Hkv, D],
  values [T, Hkv, Dv]) -> [Hq, Dv]`` (qwen35_kernels.py:363-392)
* ``qwen35_gdn_step(state [Hv, Dv, Dk], queries [Hk, Dk], keys [Hk, Dk],
  values [Hv, Dv], beta [Hv], log_decay [Hv]) -> [Hv, Dv]``, updating the
  state in place (qwen35_kernels.py:310-332)
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


def qwen35_gdn_step(state_matrix, queries, keys, values, beta, log_decay):
    torch = _host.torch_mod()
    host = _host.is_host(state_matrix)
    if host:
        import numpy as np
        if not (isinstance(state_matrix, np.ndarray) and state_matrix.dtype == np.float32
                and state_matrix.flags.c_contiguous):
            raise ValueError("state must be a contiguous float32 NumPy array (updated in place)")
    S = _host.to_device(state_matrix, torch.float32)
    q = _host.to_device(queries, torch.float32)
    k = _host.to_device(keys, torch.float32)
    v = _host.to_device(values, torch.float32)
    b = _host.to_device(beta, torch.float32)
    g = _host.to_device(log_decay, torch.float32)
    out = _ops.gdn_step(S.unsqueeze(0), q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                        b.unsqueeze(0), g.unsqueeze(0))[0]
    if host:
        state_matrix[...] = S.cpu().numpy()
        return _host.to_host(out)
    if S.data_ptr() != state_matrix.data_ptr():
        state_matrix.copy_(S)
    return out


__all__ = ["available", "backend_name", "qwen35_full_attention_decode",
           "qwen35_full_attention_prefill", "qwen35_gdn_step"]
