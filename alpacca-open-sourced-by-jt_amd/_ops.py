"""Device-level operations: validated torch buffers -> one C-ABI call.

Every facade module (``qwen35_rocm_ops``, ``qwen35_kernels``, ``kernels``,
``cuda``, ``qwen35_ops``) funnels into these functions.  Tensors are used
only as device buffers (pointer, shape, dtype, stream); all arithmetic runs
in libalpx.so.  Nothing here computes on the CPU.
"""

from __future__ import annotations

import math

from . import _lib


def _torch():
    import torch
    return torch


def kv_append(key_cache, value_cache, key, value, *, position=None, positions=None):
    """Append ``tokens`` rows ``key/value [T, B, Hkv, D]`` to caches
    ``[C, B, Hkv, D]`` at ``position + t`` (or ``positions[b] + t``)."""
    torch = _torch()
    capacity, batch, kv_heads, key_dim = (int(x) for x in key_cache.shape)
    value_dim = int(value_cache.shape[3])
    tokens = int(key.shape[0])
    pos_ptr = None
    if positions is not None:
        positions = positions.to(device=key_cache.device, dtype=torch.int32).contiguous()
        pos_ptr = positions.data_ptr()
    rc = _lib.lib().alpx_kv_append(
        key_cache.data_ptr(), value_cache.data_ptr(), key.data_ptr(), value.data_ptr(),
        _lib.dtype_code(torch, key_cache.dtype), capacity, batch, kv_heads, key_dim,
        value_dim, tokens, 0 if position is None else int(position), pos_ptr,
        _lib.stream_handle(torch, key_cache.device))
    _lib.check(rc)


def decode(q, key_cache, value_cache, *, length, k_strides, v_strides, batch, kv_heads,
           seq_lens=None, gate=None, scale=None, out_dtype=None, out=None):
    """Split-K GQA decode.  ``q [B, Hq, D]`` contiguous; K/V addressed by
    (pos, batch, head) element strides; returns ``[B, Hq, Dv]``."""
    torch = _torch()
    bsz, q_heads, key_dim = (int(x) for x in q.shape)
    value_dim = int(value_cache.shape[-1])
    if scale is None:
        scale = 1.0 / math.sqrt(key_dim)
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((bsz, q_heads, value_dim), dtype=out_dtype, device=q.device)
    lens_ptr = None
    if seq_lens is not None:
        seq_lens = seq_lens.to(device=q.device, dtype=torch.int32).contiguous()
        lens_ptr = seq_lens.data_ptr()
    L = _lib.lib()
    nbytes = L.alpx_decode_workspace_bytes(batch, q_heads, kv_heads, value_dim, int(length))
    if nbytes == 0:
        raise ValueError("invalid decode sizes")
    ws = _lib.workspace(torch, q.device, nbytes)
    rc = L.alpx_decode_gqa(
        q.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), lens_ptr, int(length),
        None if gate is None else gate.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
        batch, q_heads, kv_heads, key_dim, value_dim, *k_strides, *v_strides, float(scale),
        _lib.dtype_code(torch, q.dtype), _lib.dtype_code(torch, out.dtype),
        _lib.stream_handle(torch, q.device))
    _lib.check(rc)
    return out


def sigmoid_gate(values, gate, out_dtype=None):
    """``values * sigmoid(gate)`` elementwise on the device."""
    torch = _torch()
    out = torch.empty(values.shape, dtype=values.dtype if out_dtype is None else out_dtype,
                      device=values.device)
    rc = _lib.lib().alpx_sigmoid_gate(
        values.data_ptr(), gate.data_ptr(), out.data_ptr(), values.numel(),
        _lib.dtype_code(torch, values.dtype), _lib.dtype_code(torch, out.dtype),
        _lib.stream_handle(torch, values.device))
    _lib.check(rc)
    return out


def prefill(q, key, value, *, pos0, scale=None, window=0, kv_start=0, kv_tokens=None,
            k_pos_stride=None, v_pos_stride=None, out_dtype=None, out=None):
    """Causal GQA prefill.  ``q [T, Hq, D]`` contiguous; ``key``/``value``
    cache rows ``j < kv_tokens`` of ``kv_heads`` heads, row stride given in
    elements (default: contiguous ``[T_kv, Hkv, D]``).  Returns
    ``[T, Hq, Dv]``."""
    torch = _torch()
    q_tokens, q_heads, key_dim = (int(x) for x in q.shape)
    kv_heads = int(key.shape[-2])
    value_dim = int(value.shape[-1])
    if kv_tokens is None:
        kv_tokens = int(key.shape[0])
    if k_pos_stride is None:
        k_pos_stride = kv_heads * key_dim
    if v_pos_stride is None:
        v_pos_stride = kv_heads * value_dim
    if scale is None:
        scale = 1.0 / math.sqrt(key_dim)
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((q_tokens, q_heads, value_dim), dtype=out_dtype, device=q.device)
    L = _lib.lib()
    nbytes = L.alpx_prefill_workspace_bytes(q_tokens, q_heads, kv_heads, value_dim, kv_tokens)
    if nbytes == 0:
        raise ValueError("invalid prefill sizes")
    # only the split-K fallback (fp32, odd shapes) touches the workspace
    fast = (q.dtype != torch.float32 and key_dim == value_dim and key_dim in (64, 128, 256))
    ws = None if fast else _lib.workspace(torch, q.device, nbytes)
    rc = L.alpx_prefill_causal(
        q.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr(),
        None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
        q_tokens, int(kv_tokens), q_heads, kv_heads, key_dim, value_dim, int(k_pos_stride),
        int(v_pos_stride), int(pos0), int(window), int(kv_start), float(scale),
        _lib.dtype_code(torch, q.dtype), _lib.dtype_code(torch, out.dtype),
        _lib.stream_handle(torch, q.device))
    if rc == _lib.EINVAL and ws is None:  # unaligned rows fell back: retry with workspace
        ws = _lib.workspace(torch, q.device, nbytes)
        rc = L.alpx_prefill_causal(
            q.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr(), ws.data_ptr(),
            ws.numel(), q_tokens, int(kv_tokens), q_heads, kv_heads, key_dim, value_dim,
            int(k_pos_stride), int(v_pos_stride), int(pos0), int(window), int(kv_start),
            float(scale), _lib.dtype_code(torch, q.dtype), _lib.dtype_code(torch, out.dtype),
            _lib.stream_handle(torch, q.device))
    _lib.check(rc)
    return out


def gdn_step(state, q, k, v, beta, log_decay, out_dtype=None):
    """One GDN decode step in place on ``state [B, Hv, Dv, Dk]`` (fp32);
    q/k ``[B, Hk, Dk]``, v ``[B, Hv, Dv]``, beta/log_decay ``[B, Hv]`` fp32.
    Returns ``[B, Hv, Dv]``."""
    torch = _torch()
    bsz, hv, dv, dk = (int(x) for x in state.shape)
    hk = int(q.shape[1])
    out = torch.empty((bsz, hv, dv), dtype=q.dtype if out_dtype is None else out_dtype,
                      device=state.device)
    rc = _lib.lib().alpx_gdn_step(
        state.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
        log_decay.data_ptr(), out.data_ptr(), bsz, hk, hv, dk, dv,
        _lib.dtype_code(torch, q.dtype), _lib.dtype_code(torch, out.dtype),
        _lib.stream_handle(torch, state.device))
    _lib.check(rc)
    return out


def gdn_chunk(state, q, k, v, beta, log_decay, out_dtype=None):
    """GDN over ``T`` tokens in place on ``state``; q/k ``[B, T, Hk, Dk]``,
    v ``[B, T, Hv, Dv]``, beta/log_decay ``[B, T, Hv]`` fp32.  Returns
    ``[B, T, Hv, Dv]``."""
    torch = _torch()
    bsz, hv, dv, dk = (int(x) for x in state.shape)
    tokens, hk = int(q.shape[1]), int(q.shape[2])
    out = torch.empty((bsz, tokens, hv, dv), dtype=q.dtype if out_dtype is None else out_dtype,
                      device=state.device)
    L = _lib.lib()
    nbytes = L.alpx_gdn_chunk_workspace_bytes(bsz, tokens, hv, dk)
    ws = _lib.workspace(torch, state.device, nbytes)
    rc = L.alpx_gdn_chunk_prefill(
        state.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
        log_decay.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), bsz, tokens, hk, hv,
        dk, dv, _lib.dtype_code(torch, q.dtype), _lib.dtype_code(torch, out.dtype),
        _lib.stream_handle(torch, state.device))
    _lib.check(rc)
    return out
