"""Drop-in for the attention entry point of alpaccaroo's ``kernels`` module.

``attention_decode(q, K, V, group, inv_sqrt)`` mirrors kernels.py:1183-1200
(the Numba single-token GQA kernel behind ``Model._attention_np``,
model.py:1243-1245): q flat ``(n_head*hd,)``, K/V ``(t, n_kv, hd)``, returns
``(n_head, hd)`` -- computed by the split-K decode kernel of libalpx.so.
``available()`` mirrors kernels.py:842 as the probe a caller gates on.
"""

from __future__ import annotations

from . import _host, _lib, _ops


def available() -> bool:
    """True when libalpx.so loads and a gfx950 device is visible."""
    try:
        from .qwen35_rocm_ops import rocm_capability
        return rocm_capability().available
    except Exception:
        return False


def attention_decode(q, K, V, group, inv_sqrt):
    """Single-token grouped-query attention over the KV cache
    (kernels.py:1183-1200).  NumPy in -> NumPy out; device tensors in ->
    device tensor out."""
    host = _host.is_host(K)
    Kd = _host.to_device(K)
    Vd = _host.to_device(V, Kd.dtype)
    if Kd.dim() != 3 or Vd.dim() != 3 or Kd.shape[:2] != Vd.shape[:2]:
        raise ValueError("K and V must be (t, n_kv, hd) with matching t and n_kv")
    t, n_kv, hd = (int(x) for x in Kd.shape)
    group = int(group)
    if group < 1:
        raise ValueError("group must be a positive integer")
    qd = _host.to_device(q, Kd.dtype).reshape(1, n_kv * group, hd)
    out = _ops.decode(qd, Kd, Vd, length=t, k_strides=(n_kv * hd, 0, hd),
                      v_strides=(n_kv * int(Vd.shape[2]), 0, int(Vd.shape[2])), batch=1,
                      kv_heads=n_kv, scale=float(inv_sqrt))
    out = out.reshape(n_kv * group, int(Vd.shape[2]))
    return _host.to_host(out) if host else out


__all__ = ["attention_decode", "available"]
