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
* the recurrent-layer helpers around the GDN step: ``qwen35_conv_step``
  (:261-274), ``qwen35_normalize_qk`` (:277-287), ``qwen35_beta_decay``
  (:290-307), ``qwen35_gated_rms`` (:335-352) and
  ``qwen35_recurrent_layer`` (:349-360)
* ``qwen35_state_copy_restore(source, target)`` (:414-425) and
  ``diagnostics()`` (:428-445)

NumPy in -> NumPy out (upload, compute on the device, download); torch
device tensors in -> device tensor out.  All arithmetic runs in libalpx.so.
"""

from __future__ import annotations

import math

from . import _host, _lib, _ops


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


def _writeback(host_array, device_tensor):
    """Copy a device result into a caller-owned NumPy array (in-place
    contract of the reference's mutating helpers)."""
    host_array[...] = device_tensor.cpu().numpy()


def _check_inplace_host(array, what):
    import numpy as np
    if not (isinstance(array, np.ndarray) and array.dtype == np.float32
            and array.flags.c_contiguous):
        raise ValueError(f"{what} must be a contiguous float32 NumPy array (updated in place)")


def qwen35_conv_step(current, weights, history):
    """Depthwise causal convolution step + SiLU: ``current [C]``,
    ``weights [C, K]``, ``history [K-1, C]`` (shifted in place).  Returns
    ``(output [C], history)`` (qwen35_kernels.py:261-274)."""
    torch = _host.torch_mod()
    host = _host.is_host(current)
    if host and len(history):
        _check_inplace_host(history, "convolution history")
    cur = _host.to_device(current, torch.float32)
    w = _host.to_device(weights, torch.float32)
    kernel = int(w.shape[1])
    if int(w.shape[0]) != int(cur.shape[0]):
        raise ValueError("convolution weights must match current channels")
    hist = _host.to_device(history, torch.float32) if kernel > 1 else None
    if hist is not None and tuple(hist.shape) != (kernel - 1, int(cur.shape[0])):
        raise ValueError("convolution history must hold kernel - 1 rows of every channel")
    out = _ops.conv_step(cur.unsqueeze(0), w, None if hist is None else hist.unsqueeze(0),
                         weight_layout="ck", apply_silu=True)[0]
    if host:
        if hist is not None:
            _writeback(history, hist)
        return _host.to_host(out), history
    if hist is not None and hist.data_ptr() != history.data_ptr():
        history.copy_(hist)
    return out, history


def qwen35_normalize_qk(queries, keys, epsilon: float):
    """Each head row divided by ``max(||row||, epsilon)``
    (qwen35_kernels.py:277-287)."""
    torch = _host.torch_mod()
    host = _host.is_host(queries)
    q = _host.to_device(queries, torch.float32)
    k = _host.to_device(keys, torch.float32)
    qn = _ops.row_norm(q, mode=_lib.NORM_L2, eps=float(epsilon))
    kn = _ops.row_norm(k, mode=_lib.NORM_L2, eps=float(epsilon))
    return (_host.to_host(qn), _host.to_host(kn)) if host else (qn, kn)


def qwen35_beta_decay(beta_logits, alpha_logits, dt_bias, ssm_a):
    """``(sigmoid(beta_logits), softplus(alpha_logits + dt_bias) * ssm_a)``
    per value head (qwen35_kernels.py:290-307)."""
    torch = _host.torch_mod()
    host = _host.is_host(beta_logits)
    b, a, d, s = (_host.to_device(x, torch.float32).reshape(-1)
                  for x in (beta_logits, alpha_logits, dt_bias, ssm_a))
    beta, g = _ops.recurrent_parameters(b.unsqueeze(0), a.unsqueeze(0), d, s)
    return (_host.to_host(beta[0]), _host.to_host(g[0])) if host else (beta[0], g[0])


def qwen35_gated_rms(values, weight, gates, epsilon: float):
    """RMSNorm of each head row times ``silu(gates)``
    (qwen35_kernels.py:335-352)."""
    torch = _host.torch_mod()
    host = _host.is_host(values)
    v = _host.to_device(values, torch.float32)
    w = _host.to_device(weight, torch.float32)
    g = _host.to_device(gates, torch.float32)
    out = _ops.row_norm(v, mode=_lib.NORM_RMS_GATE, eps=float(epsilon), weight=w, gate=g)
    return _host.to_host(out) if host else out


def qwen35_recurrent_layer(state_matrix, queries, keys, values, beta_logits, alpha_logits,
                           dt_bias, ssm_a, norm_weight, gates, epsilon: float):
    """Normalise q / k, form beta / log decay, run the GDN step on the
    state (in place) and apply the gated RMSNorm; returns
    ``(gated, queries, keys)`` with the normalised queries / keys
    (qwen35_kernels.py:349-360)."""
    queries, keys = qwen35_normalize_qk(queries, keys, epsilon)
    beta, log_decay = qwen35_beta_decay(beta_logits, alpha_logits, dt_bias, ssm_a)
    output = qwen35_gdn_step(state_matrix, queries, keys, values, beta, log_decay)
    return qwen35_gated_rms(output, norm_weight, gates, epsilon), queries, keys


def qwen35_state_copy_restore(source, target):
    """Copy a recurrent state into ``target`` and return it
    (qwen35_kernels.py:414-425, same checks and messages): ``target`` is a
    float32 NumPy array of ``source``'s shape, overwritten in place.  The
    state lives in host memory, so the copy stays there (the reference's
    accelerated path is the same copy, spread over threads).  Extension: a
    float32 torch device tensor as ``target`` is filled on its device."""
    import numpy as np
    torch = _host.torch_mod() if not isinstance(target, np.ndarray) else None
    if torch is not None and torch.is_tensor(target) and target.dtype == torch.float32:
        src = source if torch.is_tensor(source) else torch.from_numpy(
            np.ascontiguousarray(source, dtype=np.float32))
        if tuple(src.shape) != tuple(target.shape):
            raise ValueError(f"state restore shapes differ: {tuple(src.shape)} != "
                             f"{tuple(target.shape)}")
        target.copy_(src.to(device=target.device, dtype=torch.float32))
        return target
    src = np.ascontiguousarray(source, dtype=np.float32)
    if getattr(target, "dtype", None) is None or target.dtype.name != "float32":
        raise ValueError("state restore target must be a float32 NumPy array")
    if src.shape != target.shape:
        raise ValueError(f"state restore shapes differ: {src.shape} != {target.shape}")
    np.copyto(target, src)
    return target


def diagnostics() -> dict:
    """What this backend runs on (qwen35_kernels.py:428-445 reports its
    numba build the same way): availability, backend name, the library and
    its ABI version, and the device architecture when a device is there."""
    info = {"available": available(), "backend": backend_name(), "library": _lib.LIB_PATH,
            "abi_version": _lib.ABI_VERSION}
    if info["available"]:
        torch = _host.torch_mod()
        info["device"] = _lib.device_arch(torch.cuda.current_device())
    return info


__all__ = ["available", "backend_name", "diagnostics", "qwen35_beta_decay", "qwen35_conv_step",
           "qwen35_full_attention_decode", "qwen35_full_attention_prefill", "qwen35_gated_rms",
           "qwen35_gdn_step", "qwen35_normalize_qk", "qwen35_recurrent_layer",
           "qwen35_state_copy_restore"]
