"""Drop-in for the attention entry point of alpaccaroo's ``kernels`` module.

``attention_decode(q, K, V, group, inv_sqrt)`` mirrors kernels.py:1183-1200
(the Numba single-token GQA kernel behind ``Model._attention_np``,
model.py:1243-1245): q flat ``(n_head*hd,)``, K/V ``(t, n_kv, hd)``, returns
``(n_head, hd)`` -- computed by the split-K decode kernel of libalpx.so.
``available()`` mirrors kernels.py:842 as the probe a caller gates on.

With host arrays, a call uploads all ``t`` rows of K and V.  A decode loop
passes ``mirror=DeviceKVMirror(...)`` (one per layer) instead: the rows
reach the device once, as the reference's device tier keeps its mirror
(cuda.py:1881-1900, synced after a prefill or truncation, appended per
token), and each call moves only the query, the rows the mirror does not
hold yet (one per token) and the output across PCIe.
"""

from __future__ import annotations

import numpy as np

from . import _host, _lib, _ops


def available() -> bool:
    """True when libalpx.so loads and a gfx950 device is visible."""
    try:
        from .qwen35_rocm_ops import rocm_capability
        return rocm_capability().available
    except Exception:
        return False


class DeviceKVMirror:
    """Device copy of one layer's host K/V cache rows ``(capacity, n_kv,
    head_dim)`` (float32, or float16 for a float16 host cache), for
    ``attention_decode(..., mirror=...)``.

    The mirror holds host rows ``[0, valid_upto)``.  A call with ``t`` host
    rows uploads rows ``[valid_upto, t)`` (a prefill's rows in one bulk copy,
    then one row per token together with the query) and attends rows
    ``[0, t)`` on the device.  A host write to a row below ``valid_upto``
    (truncation and regeneration, an edited row) must be reported with
    ``invalidate(pos)``, as the reference's model reports every cache
    mutation to its device tier (Model._chain_invalidate); without that the
    mirror keeps the old rows.

    Per token the work is one pinned host-to-device copy (query, the new K
    and V row and the row's position), the row append (device position) and
    the split-K decode over ``t`` rows as prepared calls (nothing is
    re-validated or re-packed per token; the decode plans its split from
    ``t`` as the device-tensor call does), whose output lands in pinned host
    memory (written there by the kernel where the runtime maps that memory
    for the device, else copied back)."""

    def __init__(self, capacity: int, n_kv: int, head_dim: int, dtype=np.float32) -> None:
        torch = _host.torch_mod()
        if capacity <= 0 or n_kv <= 0 or head_dim <= 0:
            raise ValueError("capacity, n_kv and head_dim must be positive")
        self.np_dtype = np.dtype(np.float16 if np.dtype(dtype) == np.float16 else np.float32)
        tdt = torch.float16 if self.np_dtype == np.float16 else torch.float32
        self.device = _host.device()
        self.capacity, self.n_kv, self.head_dim = int(capacity), int(n_kv), int(head_dim)
        shape = (self.capacity, 1, self.n_kv, self.head_dim)  # [C, B = 1, Hkv, D]
        self.key = torch.zeros(shape, dtype=tdt, device=self.device)
        self.value = torch.zeros(shape, dtype=tdt, device=self.device)
        self.valid_upto = 0
        self._steps: dict = {}  # (group, inv_sqrt) -> per-token staging and prepared calls

    def invalidate(self, pos: int) -> None:
        """Host rows from ``pos`` on changed: upload them again when used."""
        if pos < self.valid_upto:
            self.valid_upto = max(0, int(pos))

    def _bulk(self, K, V, a: int, b: int) -> None:
        torch = _host.torch_mod()
        for src, dst in ((K, self.key), (V, self.value)):
            rows = np.ascontiguousarray(src[a:b], dtype=self.np_dtype)
            dst[a:b, 0].copy_(torch.from_numpy(rows).pin_memory(), non_blocking=True)

    def _step(self, group: int, inv_sqrt: float):
        key = (group, inv_sqrt)
        st = self._steps.get(key)
        if st is not None:
            return st
        torch = _host.torch_mod()
        n_head, hd, es = self.n_kv * group, self.head_dim, self.np_dtype.itemsize
        row = self.n_kv * hd
        # staging bytes: the position (int32, padded to 16 bytes), then the
        # key row, the value row and the query (16-byte aligned pieces)
        q_off = 16 + 2 * ((row * es + 15) // 16 * 16)
        nbytes = q_off + (n_head * hd * es + 15) // 16 * 16
        host = torch.empty(nbytes, dtype=torch.uint8).pin_memory()
        dev = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        v_off = 16 + (row * es + 15) // 16 * 16
        tdt = self.key.dtype
        k_row = dev[16:16 + row * es].view(tdt).view(1, 1, self.n_kv, hd)
        v_row = dev[v_off:v_off + row * es].view(tdt).view(1, 1, self.n_kv, hd)
        q_dev = dev[q_off:q_off + n_head * hd * es].view(tdt).view(1, n_head, hd)
        ints = dev[:4].view(torch.int32)
        out_dev = torch.empty((1, n_head, hd), dtype=torch.float32, device=self.device)
        out_host = torch.empty((n_head, hd), dtype=torch.float32).pin_memory()
        # the decode writes its output straight into the pinned host buffer
        # when the runtime maps it for the device (no copy back)
        out_mapped = _lib.host_device_pointer(out_host.data_ptr())
        append = _ops.prepare_kv_append(self.key, self.value, k_row, v_row, positions=ints[0:1])
        row_stride = self.n_kv * hd
        decode = _ops.prepare_decode(q_dev, self.key, self.value, length=self.capacity,
                                     k_strides=(row_stride, row_stride, hd),
                                     v_strides=(row_stride, row_stride, hd), batch=1,
                                     kv_heads=self.n_kv, scale=float(inv_sqrt),
                                     out_dtype=torch.float32, out=out_dev,
                                     out_address=out_mapped)
        hb = host.numpy()
        st = {"host": host, "dev": dev, "ints": hb[:4].view(np.int32),
              "k": hb[16:16 + row * es].view(self.np_dtype),
              "v": hb[v_off:v_off + row * es].view(self.np_dtype),
              "q": hb[q_off:q_off + n_head * hd * es].view(self.np_dtype),
              "append": append, "decode": decode, "out_dev": out_dev, "out_host": out_host,
              "out_mapped": out_mapped is not None, "n_head": n_head}
        self._steps[key] = st
        return st

    def decode(self, q, K, V, group: int, inv_sqrt: float):
        """``attention_decode`` over host rows ``K, V [:t]`` through the mirror."""
        torch = _host.torch_mod()
        t = int(K.shape[0])
        if K.shape[1:] != (self.n_kv, self.head_dim) or V.shape != K.shape:
            raise ValueError("K and V must be (t, n_kv, hd) matching the mirror")
        if t < 1 or t > self.capacity:
            raise ValueError("the attended rows must be in [1, capacity]")
        if self.valid_upto > t:  # the host cache was cut back: rows >= t may change
            self.valid_upto = t
        if self.valid_upto < t - 1:
            self._bulk(K, V, self.valid_upto, t - 1)
        st = self._step(int(group), float(inv_sqrt))
        st["ints"][0] = t - 1
        st["k"][:] = np.asarray(K[t - 1], dtype=self.np_dtype).reshape(-1)
        st["v"][:] = np.asarray(V[t - 1], dtype=self.np_dtype).reshape(-1)
        st["q"][:] = np.asarray(q, dtype=self.np_dtype).reshape(-1)
        st["dev"].copy_(st["host"], non_blocking=True)
        st["append"]()
        st["decode"](t)
        self.valid_upto = t
        if not st["out_mapped"]:
            st["out_host"].copy_(st["out_dev"][0], non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        return st["out_host"].numpy().copy()


def attention_decode(q, K, V, group, inv_sqrt, mirror: DeviceKVMirror | None = None):
    """Single-token grouped-query attention over the KV cache
    (kernels.py:1183-1200).  NumPy in -> NumPy out; device tensors in ->
    device tensor out.  ``mirror`` (extension, host arrays only): keep the
    rows on the device between calls (``DeviceKVMirror``)."""
    host = _host.is_host(K)
    if mirror is not None:
        if not host:
            raise TypeError("a mirror serves host K/V arrays")
        if int(group) < 1:
            raise ValueError("group must be a positive integer")
        return mirror.decode(q, K, V, int(group), inv_sqrt)
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


__all__ = ["attention_decode", "available", "DeviceKVMirror"]
