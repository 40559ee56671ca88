"""Drop-in for the batched-attention (prefill) seam of alpaccaroo's ``cuda``
module, under the name the reference's ``model.py`` imports
(``from . import cuda as _gpu``).

``attention_batch(q, K, V, positions, group, inv_sqrt, window=0,
kv_start=0)`` mirrors cuda.py:1186-1244: q ``(t_q, n_head, hd)``, K/V
``(t_kv, n_kv, hd)``, absolute int positions, optional sliding window and
``kv_start``; returns ``(t_q, n_head*hd)`` float32, or ``None`` to decline
(geometry it does not cover, or a previous HIP runtime failure parked the
path) so the caller keeps its NumPy path (model.py:1256-1263).  A missing
library or device raises instead of declining.  The work runs in the
causal prefill kernel of libalpx.so; positions must be contiguous and
ascending (``positions[t] = positions[0] + t``), which every prefill chunk
of the reference satisfies (model.py:2063-2072).
"""

from __future__ import annotations

import sys

import numpy as np

from . import _host, _lib, _ops

_state = {"dead": False}


def attention_batch(q, K, V, positions, group: int, inv_sqrt: float, window: int = 0,
                    kv_start: int = 0):
    if _state["dead"]:
        return None
    try:
        pos = np.asarray(positions if _host.is_host(positions) else positions.cpu(),
                         dtype=np.int64).reshape(-1)
        qa = q if not _host.is_host(q) else np.asarray(q)
        if len(qa.shape) != 3 or len(K.shape) != 3 or tuple(K.shape) != tuple(V.shape):
            return None
        t_q, n_head, hd = (int(x) for x in qa.shape)
        t_kv, n_kv, hd_k = (int(x) for x in K.shape)
        if (hd != hd_k or hd > 256 or t_q == 0 or t_kv == 0 or group < 1
                or n_kv * group != n_head or pos.shape != (t_q,)):
            return None
        if t_q > 1 and not np.array_equal(np.diff(pos), np.ones(t_q - 1, np.int64)):
            return None
        if pos[0] < 0 or window < 0 or kv_start < 0:
            return None
    except Exception:
        return None
    try:
        host = _host.is_host(K)
        Kd = _host.to_device(K)
        Vd = _host.to_device(V, Kd.dtype)
        qd = _host.to_device(q, Kd.dtype)
        out = _ops.prefill(qd, Kd, Vd, pos0=int(pos[0]), scale=float(inv_sqrt),
                           window=int(window), kv_start=int(kv_start))
        out = out.reshape(t_q, n_head * hd)
        return _host.to_host(out) if host else out
    except _lib.AlpxError as exc:  # park, as the reference's tier does (cuda.py:1238-1244)
        _state["dead"] = True
        print(f"alpx: batch attention declined from now on ({type(exc).__name__}: {exc})",
              file=sys.stderr)
        return None


__all__ = ["attention_batch"]
