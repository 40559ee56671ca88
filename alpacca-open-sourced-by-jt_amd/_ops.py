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


def _run(fn, args, device, out):
    """Enqueues one C-ABI call (argument list with the stream last) on torch's
    current stream of ``device`` and returns ``out``."""
    args[-1] = _lib.stream_handle(_torch(), device)
    rc = fn(*args)
    if rc:
        _lib.check(rc)
    return out


class PreparedCall:
    """One library call whose buffers were validated and whose C-ABI argument
    list was packed once, for decode loops that call a step many times
    without capturing a graph.  Each call enqueues the same launch as the
    immediate entry point on torch's current stream of the device (read at
    call time) and returns ``out``.  The object holds a reference to every
    buffer it was prepared with (including the library workspace it was
    sized for), so their device pointers stay valid: their contents may
    change between calls (new query rows, device lengths, an advanced
    state), their shapes, dtypes and storage must not (no ``resize_`` or
    ``set_``).  Calls of one object must be ordered on one stream, as the
    immediate calls sharing a workspace are."""

    __slots__ = ("_fn", "_args", "_index", "_buffers", "out")

    def __init__(self, fn, args, device, buffers, out):
        self._fn = fn
        self._args = list(args)
        self._index = device.index
        self._buffers = buffers
        self.out = out

    def __call__(self):
        args = self._args
        args[-1] = _lib.current_stream(self._index)
        rc = self._fn(*args)
        if rc:
            _lib.check(rc)
        return self.out


def _kv_append_call(key_cache, value_cache, key, value, *, position=None, positions=None):
    torch = _torch()
    capacity, batch, kv_heads, key_dim = key_cache.shape
    value_dim = value_cache.shape[3]
    device = key_cache.device
    pos_ptr = None
    if positions is not None:
        if positions.dtype != torch.int32 or positions.device != device or \
                not positions.is_contiguous():
            positions = positions.to(device=device, dtype=torch.int32).contiguous()
        pos_ptr = positions.data_ptr()
    args = [key_cache.data_ptr(), value_cache.data_ptr(), key.data_ptr(), value.data_ptr(),
            _lib.dtype_code(torch, key_cache.dtype), capacity, batch, kv_heads, key_dim,
            value_dim, key.shape[0], 0 if position is None else int(position), pos_ptr, None]
    return (_lib.lib().alpx_kv_append, args, device, None,
            (key_cache, value_cache, key, value, positions))


def kv_append(key_cache, value_cache, key, value, *, position=None, positions=None):
    """Append ``tokens`` rows ``key/value [T, B, Hkv, D]`` to caches
    ``[C, B, Hkv, D]`` at ``position + t`` (or ``positions[b] + t``)."""
    fn, args, device, _, _ = _kv_append_call(key_cache, value_cache, key, value,
                                             position=position, positions=positions)
    _run(fn, args, device, None)


def prepare_kv_append(key_cache, value_cache, key, value, *, position=None, positions=None):
    """``kv_append`` as a PreparedCall (device ``positions`` may change
    between calls)."""
    fn, args, device, _, buffers = _kv_append_call(key_cache, value_cache, key, value,
                                                   position=position, positions=positions)
    return PreparedCall(fn, args, device, buffers, None)


def kv_append_paged(key_pages, value_pages, block_table, key, value, *, position=None,
                    positions=None):
    """Appends ``key/value [T, B, Hkv, D|Dv]`` through ``block_table
    [B, max_pages]`` (int32) into pages ``[P, page_size, Hkv, D|Dv]``."""
    torch = _torch()
    num_pages, page_size, kv_heads, dim = (int(x) for x in key_pages.shape)
    value_dim = int(value_pages.shape[3])
    tokens, batch = int(key.shape[0]), int(key.shape[1])
    max_pages = int(block_table.shape[1])
    pos_ptr = None
    if positions is not None:
        positions = positions.to(device=key_pages.device, dtype=torch.int32).contiguous()
        pos_ptr = positions.data_ptr()
    rc = _lib.lib().alpx_kv_append_paged(
        key_pages.data_ptr(), value_pages.data_ptr(), key.data_ptr(), value.data_ptr(),
        block_table.data_ptr(), max_pages, page_size, num_pages,
        _lib.dtype_code(torch, key_pages.dtype), batch, kv_heads, dim, value_dim, tokens,
        0 if position is None else int(position), pos_ptr,
        _lib.stream_handle(torch, key_pages.device))
    _lib.check(rc)


def decode_paged(q, key_pages, value_pages, block_table, *, length, seq_lens=None, gate=None,
                 scale, out_dtype=None):
    """Split-K decode of ``q [B, Hq, D]`` over paged caches; returns
    ``[B, Hq, Dv]``."""
    torch = _torch()
    num_pages, page_size, kv_heads, dim = (int(x) for x in key_pages.shape)
    value_dim = int(value_pages.shape[3])
    batch, q_heads = int(q.shape[0]), int(q.shape[1])
    out = torch.empty((batch, q_heads, value_dim),
                      dtype=q.dtype if out_dtype is None else out_dtype, device=q.device)
    L = _lib.lib()
    nbytes = L.alpx_decode_workspace_bytes(batch, q_heads, kv_heads, value_dim, int(length))
    ws = _lib.workspace(torch, q.device, nbytes)
    lens_ptr = None
    if seq_lens is not None:
        seq_lens = seq_lens.to(device=q.device, dtype=torch.int32).contiguous()
        lens_ptr = seq_lens.data_ptr()
    rc = L.alpx_decode_gqa_paged(
        q.data_ptr(), key_pages.data_ptr(), value_pages.data_ptr(), block_table.data_ptr(),
        int(block_table.shape[1]), page_size, num_pages, lens_ptr, int(length),
        None if gate is None else gate.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
        batch, q_heads, kv_heads, dim, value_dim, float(scale),
        _lib.dtype_code(torch, q.dtype), _lib.dtype_code(torch, out.dtype),
        _lib.stream_handle(torch, q.device))
    _lib.check(rc)
    return out


def prefill_append(q, key, value, key_cache, value_cache, *, position, scale=None, window=0,
                   out_dtype=None, gate=None):
    """Writes the chunk's rows ``key/value [T, Hkv, D]`` to rows ``position ..``
    of the batch-1 caches ``[C, 1, Hkv, D]`` and returns the causal prefill
    of ``q [T, Hq, D]`` over cache rows ``0 .. position + t`` (one launch on
    the MFMA path)."""
    torch = _torch()
    q_tokens, q_heads, key_dim = (int(x) for x in q.shape)
    capacity, _, kv_heads, _ = (int(x) for x in key_cache.shape)
    value_dim = int(value_cache.shape[3])
    if scale is None:
        scale = 1.0 / math.sqrt(key_dim)
    out_dtype = q.dtype if out_dtype is None else out_dtype
    out = torch.empty((q_tokens, q_heads, value_dim), dtype=out_dtype, device=q.device)
    L = _lib.lib()
    nbytes = L.alpx_prefill_workspace_bytes(q_tokens, q_heads, kv_heads, value_dim,
                                            int(position) + q_tokens)
    if nbytes == 0:
        raise ValueError("invalid prefill sizes")
    fast = (q.dtype != torch.float32 and key_dim == value_dim and key_dim in (64, 128, 256))
    ws = None if fast else _lib.workspace(torch, q.device, nbytes)

    def call(workspace):
        return L.alpx_prefill_append(
            q.data_ptr(), key.data_ptr(), value.data_ptr(), key_cache.data_ptr(),
            value_cache.data_ptr(), None if gate is None else gate.data_ptr(), out.data_ptr(),
            None if workspace is None else workspace.data_ptr(),
            0 if workspace is None else workspace.numel(), q_tokens, capacity, q_heads, kv_heads,
            key_dim, value_dim, int(position), int(window), float(scale),
            _lib.dtype_code(torch, q.dtype), _lib.dtype_code(torch, out.dtype),
            _lib.stream_handle(torch, q.device))

    rc = call(ws)
    # unaligned rows or a cache of 2 GiB or more leave the MFMA kernels; the
    # split-K path refuses a null workspace before its append
    if rc == _lib.EINVAL and ws is None:
        ws = _lib.workspace(torch, q.device, nbytes)
        rc = call(ws)
    _lib.check(rc)
    return out


def prefill_paged(q, key_pages, value_pages, block_table, *, batch_index, pos0, kv_tokens,
                  scale=None, window=0, kv_start=0, gate=None):
    """Causal prefill of ``q [T, Hq, D]`` at positions ``pos0 ..`` over the
    first ``kv_tokens`` logical rows of sequence ``batch_index`` of paged
    caches ``[num_pages, page_size, Hkv, D]``; output ``[T, Hq, D]`` in q's
    dtype, times sigmoid(gate) when ``gate`` is given."""
    torch = _torch()
    num_pages, page_size, kv_heads, dim = (int(x) for x in key_pages.shape)
    tokens, q_heads = int(q.shape[0]), int(q.shape[1])
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    out = torch.empty((tokens, q_heads, dim), dtype=q.dtype, device=q.device)
    rc = _lib.lib().alpx_prefill_causal_paged(
        q.data_ptr(), key_pages.data_ptr(), value_pages.data_ptr(), block_table.data_ptr(),
        int(block_table.shape[1]), page_size, num_pages, int(batch_index),
        None if gate is None else gate.data_ptr(), out.data_ptr(), tokens, int(kv_tokens),
        q_heads, kv_heads, dim, int(pos0), int(window), int(kv_start), float(scale),
        _lib.dtype_code(torch, q.dtype), _lib.stream_handle(torch, q.device))
    _lib.check(rc)
    return out


def kv_export(key_cache, value_cache, *, batch_index, row0, rows):
    """Rows ``[row0, row0 + rows)`` of cache sequence ``batch_index`` as
    contiguous fp32 ``(key [rows, Hkv, D], value [rows, Hkv, Dv])``."""
    torch = _torch()
    capacity, batch, kv_heads, dim = (int(x) for x in key_cache.shape)
    value_dim = int(value_cache.shape[3])
    dev = key_cache.device
    k = torch.empty((rows, kv_heads, dim), dtype=torch.float32, device=dev)
    v = torch.empty((rows, kv_heads, value_dim), dtype=torch.float32, device=dev)
    rc = _lib.lib().alpx_kv_export(
        key_cache.data_ptr(), value_cache.data_ptr(), k.data_ptr(), v.data_ptr(),
        _lib.dtype_code(torch, key_cache.dtype), capacity, batch, kv_heads, dim, value_dim,
        int(batch_index), int(row0), int(rows), _lib.stream_handle(torch, dev))
    _lib.check(rc)
    return k, v


def kv_import(key_rows, value_rows, key_cache, value_cache, *, batch_index, row0):
    """Writes fp32 rows ``[rows, Hkv, D|Dv]`` into cache sequence
    ``batch_index`` from row ``row0`` (rounded to the cache dtype)."""
    torch = _torch()
    capacity, batch, kv_heads, dim = (int(x) for x in key_cache.shape)
    value_dim = int(value_cache.shape[3])
    rc = _lib.lib().alpx_kv_import(
        key_rows.data_ptr(), value_rows.data_ptr(), key_cache.data_ptr(),
        value_cache.data_ptr(), _lib.dtype_code(torch, key_cache.dtype), capacity, batch,
        kv_heads, dim, value_dim, int(batch_index), int(row0), int(key_rows.shape[0]),
        _lib.stream_handle(torch, key_cache.device))
    _lib.check(rc)


def kv_export_paged(key_pages, value_pages, block_table, *, batch_index, row0, rows):
    """Logical rows ``[row0, row0 + rows)`` of sequence ``batch_index`` of a
    paged pool (``block_table [B, max_pages]`` int32) as contiguous fp32
    ``(key [rows, Hkv, D], value [rows, Hkv, Dv])``; rows whose table entry
    lies outside the pool read as zero."""
    torch = _torch()
    num_pages, page_size, kv_heads, dim = (int(x) for x in key_pages.shape)
    value_dim = int(value_pages.shape[3])
    batch, max_pages = (int(x) for x in block_table.shape)
    dev = key_pages.device
    k = torch.empty((rows, kv_heads, dim), dtype=torch.float32, device=dev)
    v = torch.empty((rows, kv_heads, value_dim), dtype=torch.float32, device=dev)
    rc = _lib.lib().alpx_kv_export_paged(
        key_pages.data_ptr(), value_pages.data_ptr(), block_table.data_ptr(), batch, max_pages,
        page_size, num_pages, k.data_ptr(), v.data_ptr(), _lib.dtype_code(torch, key_pages.dtype),
        kv_heads, dim, value_dim, int(batch_index), int(row0), int(rows),
        _lib.stream_handle(torch, dev))
    _lib.check(rc)
    return k, v


def kv_import_paged(key_rows, value_rows, key_pages, value_pages, block_table, *, batch_index,
                    row0):
    """Writes fp32 rows ``[rows, Hkv, D|Dv]`` into sequence ``batch_index`` of a
    paged pool from logical row ``row0`` (rounded to the page dtype; rows
    whose table entry lies outside the pool are skipped)."""
    torch = _torch()
    num_pages, page_size, kv_heads, dim = (int(x) for x in key_pages.shape)
    value_dim = int(value_pages.shape[3])
    batch, max_pages = (int(x) for x in block_table.shape)
    rc = _lib.lib().alpx_kv_import_paged(
        key_rows.data_ptr(), value_rows.data_ptr(), key_pages.data_ptr(), value_pages.data_ptr(),
        block_table.data_ptr(), batch, max_pages, page_size, num_pages,
        _lib.dtype_code(torch, key_pages.dtype), kv_heads, dim, value_dim, int(batch_index),
        int(row0), int(key_rows.shape[0]), _lib.stream_handle(torch, key_pages.device))
    _lib.check(rc)


def _decode_call(q, key_cache, value_cache, *, length, k_strides, v_strides, batch, kv_heads,
                 seq_lens=None, gate=None, scale=None, out_dtype=None, out=None,
                 out_address=None):
    """(C function, argument list with the stream last, device, out, buffers)
    of one alpx_decode_gqa call.  ``out_address``: the device address the
    output is written to when it is not ``out``'s own (page-locked host
    memory mapped for the device, alpx_host_device_pointer)."""
    torch = _torch()
    bsz, q_heads, key_dim = q.shape
    value_dim = value_cache.shape[-1]
    device = q.device
    if scale is None:
        scale = 1.0 / math.sqrt(key_dim)
    if out is None:
        out = torch.empty((bsz, q_heads, value_dim), dtype=q.dtype if out_dtype is None
                          else out_dtype, device=device)
    lens_ptr = None
    if seq_lens is not None:
        if seq_lens.dtype != torch.int32 or seq_lens.device != device or \
                not seq_lens.is_contiguous():
            seq_lens = seq_lens.to(device=device, dtype=torch.int32).contiguous()
        lens_ptr = seq_lens.data_ptr()
    L = _lib.lib()
    length = int(length)
    sizes = (batch, q_heads, kv_heads, value_dim, length)
    nbytes = _decode_ws_bytes.get(sizes)
    if nbytes is None:
        nbytes = L.alpx_decode_workspace_bytes(*sizes)
        if nbytes == 0:
            raise ValueError("invalid decode sizes")
        if len(_decode_ws_bytes) >= _DECODE_WS_CACHE_MAX:  # a decode loop asks per length
            _decode_ws_bytes.clear()
        _decode_ws_bytes[sizes] = nbytes
    ws = _lib.workspace(torch, device, nbytes)
    args = [q.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), lens_ptr, length,
            None if gate is None else gate.data_ptr(),
            out.data_ptr() if out_address is None else out_address, ws.data_ptr(), ws.numel(),
            batch, q_heads, kv_heads, key_dim, value_dim, *k_strides, *v_strides, float(scale),
            _lib.dtype_code(torch, q.dtype), _lib.dtype_code(torch, out.dtype), None]
    return L.alpx_decode_gqa, args, device, out, (q, key_cache, value_cache, seq_lens, gate, ws)


def decode(q, key_cache, value_cache, **kwargs):
    """Split-K GQA decode.  ``q [B, Hq, D]`` contiguous; K/V addressed by
    (pos, batch, head) element strides (keywords: length, k_strides,
    v_strides, batch, kv_heads, seq_lens, gate, scale, out_dtype, out);
    returns ``[B, Hq, Dv]``."""
    fn, args, device, out, _ = _decode_call(q, key_cache, value_cache, **kwargs)
    return _run(fn, args, device, out)


class PreparedDecode(PreparedCall):
    """A prepared ``decode`` whose call may name the rows to attend:
    ``call(length)`` attends rows ``0 .. length - 1`` (at most the length it
    was prepared with, which sized its workspace) from this call on."""

    __slots__ = ("_max_length",)

    def __call__(self, length=None):
        if length is not None:
            length = int(length)
            if not 0 < length <= self._max_length:
                raise ValueError(f"attention length {length} outside [1, {self._max_length}]")
            self._args[4] = length
        return PreparedCall.__call__(self)


def prepare_decode(q, key_cache, value_cache, **kwargs):
    """``decode`` as a PreparedDecode (same keywords)."""
    fn, args, device, out, buffers = _decode_call(q, key_cache, value_cache, **kwargs)
    call = PreparedDecode(fn, args, device, buffers + (out,), out)
    call._max_length = args[4]
    return call


# alpx_decode_workspace_bytes per (batch, q_heads, kv_heads, value_dim, length):
# a pure function of the sizes, asked once per shape; cleared when it holds
# _DECODE_WS_CACHE_MAX entries (the length changes every token of a decode
# loop, so the cache would otherwise grow for the life of the process).
_decode_ws_bytes: dict = {}
_DECODE_WS_CACHE_MAX = 1024


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
            k_pos_stride=None, v_pos_stride=None, out_dtype=None, out=None, gate=None):
    """Causal GQA prefill.  ``q [T, Hq, D]`` contiguous; ``key``/``value``
    cache rows ``j < kv_tokens`` of ``kv_heads`` heads, row stride given in
    elements (default: contiguous ``[T_kv, Hkv, D]``).  With ``gate``
    (contiguous ``[T, Hq, Dv]``, q's dtype) the output is multiplied by
    sigmoid(gate) before it is rounded.  Returns ``[T, Hq, Dv]``."""
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

    def call(workspace):
        args = (None if workspace is None else workspace.data_ptr(),
                0 if workspace is None else workspace.numel(), q_tokens, int(kv_tokens), q_heads,
                kv_heads, key_dim, value_dim, int(k_pos_stride), int(v_pos_stride), int(pos0),
                int(window), int(kv_start), float(scale), _lib.dtype_code(torch, q.dtype),
                _lib.dtype_code(torch, out.dtype), _lib.stream_handle(torch, q.device))
        if gate is None:
            return L.alpx_prefill_causal(q.data_ptr(), key.data_ptr(), value.data_ptr(),
                                         out.data_ptr(), *args)
        return L.alpx_prefill_causal_gated(q.data_ptr(), key.data_ptr(), value.data_ptr(),
                                           gate.data_ptr(), out.data_ptr(), *args)

    rc = call(ws)
    if rc == _lib.EINVAL and ws is None:  # unaligned rows fell back: retry with workspace
        ws = _lib.workspace(torch, q.device, nbytes)
        rc = call(ws)
    _lib.check(rc)
    return out


def _gdn_step_call(state, q, k, v, beta, log_decay, out_dtype=None, out=None):
    torch = _torch()
    bsz, hv, dv, dk = state.shape
    device = state.device
    if out is None:
        out = torch.empty((bsz, hv, dv), dtype=q.dtype if out_dtype is None else out_dtype,
                          device=device)
    args = [state.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
            log_decay.data_ptr(), out.data_ptr(), bsz, q.shape[1], hv, dk, dv,
            _lib.dtype_code(torch, q.dtype), _lib.dtype_code(torch, out.dtype), None]
    return _lib.lib().alpx_gdn_step, args, device, out, (state, q, k, v, beta, log_decay)


def gdn_step(state, q, k, v, beta, log_decay, out_dtype=None, out=None):
    """One GDN decode step in place on ``state [B, Hv, Dv, Dk]`` (fp32);
    q/k ``[B, Hk, Dk]``, v ``[B, Hv, Dv]``, beta/log_decay ``[B, Hv]`` fp32.
    Returns ``[B, Hv, Dv]`` (``out`` when given: a contiguous buffer of
    that shape, already checked by the caller)."""
    fn, args, device, out, _ = _gdn_step_call(state, q, k, v, beta, log_decay, out_dtype, out)
    return _run(fn, args, device, out)


def prepare_gdn_step(state, q, k, v, beta, log_decay, out_dtype=None, out=None):
    """``gdn_step`` as a PreparedCall."""
    fn, args, device, out, buffers = _gdn_step_call(state, q, k, v, beta, log_decay, out_dtype,
                                                    out)
    return PreparedCall(fn, args, device, buffers + (out,), out)


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
    dtype = _lib.dtype_code(torch, q.dtype)
    ws = None
    if L.alpx_gdn_chunk_uses_mfma(dtype, tokens, hk, hv, dk, dv):
        ws = _lib.workspace(torch, state.device,
                            L.alpx_gdn_chunk_workspace_bytes(bsz, tokens, hv, dk))
    rc = L.alpx_gdn_chunk_prefill(
        state.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
        log_decay.data_ptr(), out.data_ptr(), None if ws is None else ws.data_ptr(),
        0 if ws is None else ws.numel(), bsz, tokens, hk, hv, dk, dv, dtype,
        _lib.dtype_code(torch, out.dtype), _lib.stream_handle(torch, state.device))
    _lib.check(rc)
    return out


def silu(values, out_dtype=None):
    """Elementwise ``x * sigmoid(x)``; returns a new tensor."""
    torch = _torch()
    out = torch.empty(values.shape, dtype=values.dtype if out_dtype is None else out_dtype,
                      device=values.device)
    rc = _lib.lib().alpx_silu(values.data_ptr(), out.data_ptr(), values.numel(),
                              _lib.dtype_code(torch, values.dtype),
                              _lib.dtype_code(torch, out.dtype),
                              _lib.stream_handle(torch, values.device))
    _lib.check(rc)
    return out


def row_norm(x, *, mode, eps, weight=None, gate=None, n=None, rows=None, group_rows=0,
             group_stride=0, out_dtype=None, out=None):
    """Row-wise L2 / RMS / gated-RMS normalisation over the last axis of
    ``x`` (contiguous unless ``rows``/``group_*`` describe a strided view of
    its storage, with ``n`` the row width).  ``weight`` fp32 ``[n]``;
    ``gate`` contiguous like the output.  Returns ``[rows, n]`` (shaped like
    ``x`` for contiguous rows)."""
    torch = _torch()
    n = int(x.shape[-1]) if n is None else int(n)
    if rows is None:
        rows = x.numel() // n
    if out is None:
        shape = x.shape if group_rows == 0 else (rows, n)
        out = torch.empty(shape, dtype=x.dtype if out_dtype is None else out_dtype,
                          device=x.device)
    rc = _lib.lib().alpx_row_norm(
        x.data_ptr(), None if weight is None else weight.data_ptr(),
        None if gate is None else gate.data_ptr(), out.data_ptr(), int(rows), n,
        int(group_rows), int(group_stride), float(eps), int(mode),
        _lib.dtype_code(torch, x.dtype), _lib.dtype_code(torch, out.dtype),
        _lib.stream_handle(torch, x.device))
    _lib.check(rc)
    return out


def conv_step(current, weight, history, *, weight_layout="kc", apply_silu=False,
              out_dtype=None):
    """Causal depthwise convolution step on ``current [B, C]`` with
    ``history [B, K-1, C]`` (fp32, shifted in place) and ``weight`` ``[K, C]``
    (``"kc"``) or ``[C, K]`` (``"ck"``).  Returns ``[B, C]``."""
    torch = _torch()
    bsz, channels = (int(x) for x in current.shape)
    if weight_layout == "kc":
        kernel = int(weight.shape[0])
        tap_stride, ch_stride = channels, 1
    else:
        kernel = int(weight.shape[1])
        tap_stride, ch_stride = 1, kernel
    out = torch.empty((bsz, channels), dtype=torch.float32 if out_dtype is None else out_dtype,
                      device=current.device)
    rc = _lib.lib().alpx_conv_step(
        current.data_ptr(), weight.data_ptr(), None if history is None else history.data_ptr(),
        out.data_ptr(), bsz, channels, kernel, tap_stride, ch_stride, 1 if apply_silu else 0,
        _lib.dtype_code(torch, out.dtype), _lib.stream_handle(torch, current.device))
    _lib.check(rc)
    return out


def recurrent_parameters(beta_logits, alpha_logits, dt_bias, ssm_a):
    """``(beta, log_decay)`` shaped like ``beta_logits`` (fp32)."""
    torch = _torch()
    beta = torch.empty_like(beta_logits)
    g = torch.empty_like(beta_logits)
    heads = int(dt_bias.shape[0])
    rc = _lib.lib().alpx_recurrent_parameters(
        beta_logits.data_ptr(), alpha_logits.data_ptr(), dt_bias.data_ptr(), ssm_a.data_ptr(),
        beta.data_ptr(), g.data_ptr(), beta_logits.numel(), heads,
        _lib.stream_handle(torch, beta_logits.device))
    _lib.check(rc)
    return beta, g


def _sections(sections):
    import ctypes
    sec = (ctypes.c_int * 4)(*[int(x) for x in sections])
    return sec


def imrope(values, position_lanes, sections, *, frequency_base, frequency_scale=1.0,
           out_dtype=None):
    """IMROPE over the last axis of ``values``.  ``position_lanes`` int64
    ``(4,)`` (one lane vector for every row) or ``[rows, 4]`` (one per row,
    rows = values.numel() // values.shape[-1])."""
    torch = _torch()
    dim = int(values.shape[-1])
    rows = values.numel() // dim
    lanes = position_lanes.to(device=values.device, dtype=torch.int64).contiguous()
    stride = 0 if lanes.numel() == 4 else 4
    out = torch.empty(values.shape, dtype=values.dtype if out_dtype is None else out_dtype,
                      device=values.device)
    rc = _lib.lib().alpx_imrope(
        values.data_ptr(), out.data_ptr(), lanes.data_ptr(), stride, rows, 1, dim,
        _sections(sections), float(frequency_base), float(frequency_scale),
        _lib.dtype_code(torch, values.dtype), _lib.dtype_code(torch, out.dtype),
        _lib.stream_handle(torch, values.device))
    _lib.check(rc)
    return out


def attention_prologue(query_gate, key, value, q_norm, k_norm, key_cache, value_cache, *,
                       position=0, positions=None, sections, frequency_base, eps):
    """Fused Qwen3.5 attention prologue for one token per sequence:
    ``query_gate [B, Hq, 2D]``, ``key [B, Hkv, D]``, ``value [B, Hkv, Dv]``;
    appends the normalised, rotated key and the value to the caches
    ``[C, B, Hkv, D|Dv]``.  Returns ``(query [B, Hq, D], gate [B, Hq, D])``."""
    torch = _torch()
    capacity, bsz, kv_heads, dim = (int(x) for x in key_cache.shape)
    value_dim = int(value_cache.shape[3])
    q_heads = int(query_gate.shape[1])
    query = torch.empty((bsz, q_heads, dim), dtype=key_cache.dtype, device=key_cache.device)
    gate = torch.empty_like(query)
    pos_ptr = None
    if positions is not None:
        positions = positions.to(device=key_cache.device, dtype=torch.int32).contiguous()
        pos_ptr = positions.data_ptr()
    rc = _lib.lib().alpx_attention_prologue(
        query_gate.data_ptr(), key.data_ptr(), value.data_ptr(), q_norm.data_ptr(),
        k_norm.data_ptr(), query.data_ptr(), gate.data_ptr(), key_cache.data_ptr(),
        value_cache.data_ptr(), _lib.dtype_code(torch, key_cache.dtype), capacity, bsz,
        q_heads, kv_heads, dim, value_dim, int(position), pos_ptr, _sections(sections),
        float(frequency_base), float(eps), _lib.stream_handle(torch, key_cache.device))
    _lib.check(rc)
    return query, gate


def attention_layer_step(query_gate, key, value, q_norm, k_norm, key_cache, value_cache, *,
                         position, sections, frequency_base, eps, positions=None, scale=None,
                         out_dtype=None):
    """One decode token of the Qwen3.5 attention layer in two launches: the
    prologue (Q/K RMSNorm + IMROPE, cache append at ``position``) inside the
    split-K decode launch, then the combine with the sigmoid gate taken from
    the second half of ``query_gate [B, Hq, 2D]``.  ``key`` / ``value``
    ``[B, Hkv, D]``; caches ``[C, B, Hkv, D]`` (fp16 / bf16, D in 64, 128,
    256).  With ``positions`` (device int32 ``[B]``, each at most
    ``position``) sequence b's token sits at row ``positions[b]`` and
    attends rows ``0 .. positions[b]``.  Returns the gated output
    ``[B, Hq, D]``."""
    torch = _torch()
    capacity, bsz, kv_heads, dim = (int(x) for x in key_cache.shape)
    q_heads = int(query_gate.shape[1])
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    out_dtype = key_cache.dtype if out_dtype is None else out_dtype
    out = torch.empty((bsz, q_heads, dim), dtype=out_dtype, device=key_cache.device)
    L = _lib.lib()
    nbytes = L.alpx_decode_workspace_bytes(bsz, q_heads, kv_heads, dim, int(position) + 1)
    if nbytes == 0:
        raise ValueError("invalid attention step sizes")
    ws = _lib.workspace(torch, key_cache.device, nbytes)
    pos_ptr = None
    if positions is not None:
        positions = positions.to(device=key_cache.device, dtype=torch.int32).contiguous()
        pos_ptr = positions.data_ptr()
    rc = L.alpx_attention_layer_step(
        query_gate.data_ptr(), key.data_ptr(), value.data_ptr(), q_norm.data_ptr(),
        k_norm.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), out.data_ptr(),
        ws.data_ptr(), ws.numel(), _lib.dtype_code(torch, key_cache.dtype),
        _lib.dtype_code(torch, out.dtype), capacity, bsz, q_heads, kv_heads, dim, int(position),
        pos_ptr, _sections(sections), float(frequency_base), float(eps), float(scale),
        _lib.stream_handle(torch, key_cache.device))
    _lib.check(rc)
    return out


def attention_layer_step_paged(query_gate, key, value, q_norm, k_norm, key_pages, value_pages,
                               block_table, *, position, sections, frequency_base, eps,
                               positions=None, scale=None, out_dtype=None):
    """``attention_layer_step`` over a paged pool: pages ``[P, page_size,
    Hkv, D]`` (fp16 / bf16, D in 64, 128, 256) and ``block_table [B,
    max_pages]`` (device int32).  Sequence b's rotated key and value land at
    its logical row ``position`` (or ``positions[b]``) through the table.
    Returns the gated output ``[B, Hq, D]``."""
    torch = _torch()
    num_pages, page_size, kv_heads, dim = (int(x) for x in key_pages.shape)
    bsz, max_pages = (int(x) for x in block_table.shape)
    q_heads = int(query_gate.shape[1])
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    out_dtype = key_pages.dtype if out_dtype is None else out_dtype
    out = torch.empty((bsz, q_heads, dim), dtype=out_dtype, device=key_pages.device)
    L = _lib.lib()
    nbytes = L.alpx_decode_workspace_bytes(bsz, q_heads, kv_heads, dim, int(position) + 1)
    if nbytes == 0:
        raise ValueError("invalid attention step sizes")
    ws = _lib.workspace(torch, key_pages.device, nbytes)
    pos_ptr = None
    if positions is not None:
        positions = positions.to(device=key_pages.device, dtype=torch.int32).contiguous()
        pos_ptr = positions.data_ptr()
    rc = L.alpx_attention_layer_step_paged(
        query_gate.data_ptr(), key.data_ptr(), value.data_ptr(), q_norm.data_ptr(),
        k_norm.data_ptr(), key_pages.data_ptr(), value_pages.data_ptr(), block_table.data_ptr(),
        max_pages, page_size, num_pages, out.data_ptr(), ws.data_ptr(), ws.numel(),
        _lib.dtype_code(torch, key_pages.dtype), _lib.dtype_code(torch, out.dtype), bsz, q_heads,
        kv_heads, dim, int(position), pos_ptr, _sections(sections), float(frequency_base),
        float(eps), float(scale), _lib.stream_handle(torch, key_pages.device))
    _lib.check(rc)
    return out


def attention_layer_prefill_paged(query_gate, key, value, q_norm, k_norm, key_pages, value_pages,
                                  block_table, *, batch_index, position, sections,
                                  frequency_base, eps, scale=None):
    """``attention_layer_prefill`` (the form without a query buffer) over a
    paged pool: pages ``[P, page_size, Hkv, D]`` (fp16 / bf16, D in 64, 128,
    256, page_size a power of two >= 64) and ``block_table [B, max_pages]``
    (device int32); the chunk's rotated keys and values land at logical
    rows ``position ..`` of sequence ``batch_index`` through the table.
    Returns the gated output ``[T, Hq, D]`` in the pages' dtype."""
    torch = _torch()
    num_pages, page_size, kv_heads, dim = (int(x) for x in key_pages.shape)
    max_pages = int(block_table.shape[1])
    tokens, q_heads = int(query_gate.shape[0]), int(query_gate.shape[1])
    dev = key_pages.device
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    out = torch.empty((tokens, q_heads, dim), dtype=key_pages.dtype, device=dev)
    pairs = sum(int(x) for x in sections)
    ws = _lib.workspace(torch, dev, max(tokens * pairs * 8, 1))
    rc = _lib.lib().alpx_attention_layer_prefill_paged(
        query_gate.data_ptr(), key.data_ptr(), value.data_ptr(), q_norm.data_ptr(),
        k_norm.data_ptr(), key_pages.data_ptr(), value_pages.data_ptr(), block_table.data_ptr(),
        max_pages, page_size, num_pages, int(batch_index), out.data_ptr(), ws.data_ptr(),
        ws.numel(), _lib.dtype_code(torch, key_pages.dtype), tokens, q_heads, kv_heads, dim,
        int(position), _sections(sections), float(frequency_base), float(eps), float(scale),
        _lib.stream_handle(torch, dev))
    _lib.check(rc)
    return out


def attention_prologue_chunk(query_gate, key, value, q_norm, k_norm, key_cache, value_cache, *,
                             batch_index, position, sections, frequency_base, eps):
    """Attention prologue for ``T`` consecutive tokens of cache sequence
    ``batch_index`` at positions ``position ..``: ``query_gate [T, Hq, 2D]``,
    ``key [T, Hkv, D]``, ``value [T, Hkv, Dv]``.  Returns
    ``(query [T, Hq, D], gate [T, Hq, D])``."""
    torch = _torch()
    capacity, cache_batch, kv_heads, dim = (int(x) for x in key_cache.shape)
    value_dim = int(value_cache.shape[3])
    tokens, q_heads = int(query_gate.shape[0]), int(query_gate.shape[1])
    query = torch.empty((tokens, q_heads, dim), dtype=key_cache.dtype, device=key_cache.device)
    gate = torch.empty_like(query)
    rc = _lib.lib().alpx_attention_prologue_chunk(
        query_gate.data_ptr(), key.data_ptr(), value.data_ptr(), q_norm.data_ptr(),
        k_norm.data_ptr(), query.data_ptr(), gate.data_ptr(), key_cache.data_ptr(),
        value_cache.data_ptr(), _lib.dtype_code(torch, key_cache.dtype), capacity, cache_batch,
        int(batch_index), tokens, q_heads, kv_heads, dim, value_dim, int(position),
        _sections(sections), float(frequency_base), float(eps),
        _lib.stream_handle(torch, key_cache.device))
    _lib.check(rc)
    return query, gate


def attention_layer_prefill(query_gate, key, value, q_norm, k_norm, key_cache, value_cache, *,
                            batch_index, position, sections, frequency_base, eps, scale=None,
                            out_dtype=None, fused_query=None):
    """Qwen3.5 attention-layer prefill chunk (``alpx_attention_layer_prefill``):
    the chunk prologue for ``query_gate [T, Hq, 2D]``, ``key [T, Hkv, D]``,
    ``value [T, Hkv, D]`` of cache sequence ``batch_index`` at positions
    ``position ..``, then the causal prefill over the cache with the sigmoid
    gate read from ``query_gate``.  Returns the gated output ``[T, Hq, D]``.

    ``fused_query`` picks the form: True has the prefill form the query
    rows from ``query_gate`` itself (no query buffer; fp16 / bf16, D in
    {64, 128, 256}, rotary sections summing to a multiple of 32), False
    writes them to a query buffer first, None takes the first where it
    applies.  Both give the same bits."""
    torch = _torch()
    capacity, cache_batch, kv_heads, dim = (int(x) for x in key_cache.shape)
    tokens, q_heads = int(query_gate.shape[0]), int(query_gate.shape[1])
    dev = key_cache.device
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    out_dtype = key_cache.dtype if out_dtype is None else out_dtype
    out = torch.empty((tokens, q_heads, dim), dtype=out_dtype, device=dev)
    L = _lib.lib()
    fast = key_cache.dtype != torch.float32 and dim in (64, 128, 256)
    pairs = sum(int(x) for x in sections)
    auto = fused_query is None
    if auto:
        fused_query = (fast and pairs % 32 == 0 and 2 * pairs <= dim
                       and _lib.get_override(_lib.OVERRIDE_PREFILL_GENERIC) == 0)

    def call(query, ws):
        return L.alpx_attention_layer_prefill(
            query_gate.data_ptr(), key.data_ptr(), value.data_ptr(), q_norm.data_ptr(),
            k_norm.data_ptr(), None if query is None else query.data_ptr(),
            key_cache.data_ptr(), value_cache.data_ptr(), out.data_ptr(),
            None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
            _lib.dtype_code(torch, key_cache.dtype), _lib.dtype_code(torch, out.dtype), capacity,
            cache_batch, int(batch_index), tokens, q_heads, kv_heads, dim, int(position),
            _sections(sections), float(frequency_base), float(eps), float(scale),
            _lib.stream_handle(torch, dev))

    # Every refusal below comes before the library's first launch, so a
    # refused form has written nothing and the next form may run.
    if fused_query:
        rc = call(None, _lib.workspace(torch, dev, max(tokens * pairs * 8, 1)))
        if not (auto and rc == _lib.EUNSUPPORTED):  # e.g. a cache of 2 GiB or more
            _lib.check(rc)
            return out
    query = torch.empty((tokens, q_heads, dim), dtype=key_cache.dtype, device=dev)
    rc = call(query, None)
    if rc == _lib.EINVAL:  # the split-K prefill (fp32, unaligned, >= 2 GiB) needs a workspace
        nbytes = L.alpx_prefill_workspace_bytes(tokens, q_heads, kv_heads, dim,
                                                int(position) + tokens)
        if nbytes == 0:
            raise ValueError("invalid prefill sizes")
        rc = call(query, _lib.workspace(torch, dev, nbytes))
    _lib.check(rc)
    return out


def recurrent_prefill_prep(current, conv_weight, conv_history, beta_logits, alpha_logits,
                           dt_bias, ssm_a, *, key_heads, key_dim, value_heads, value_dim, eps,
                           qkv_dtype, weight_layout="kc"):
    """Recurrent-layer inputs for ``T`` consecutive tokens of one sequence
    (all fp32 inputs): ``current [T, C]``, ``conv_history [K-1, C]`` (moved
    on in place).  Returns ``(q [T, Hk, Dk], k, v [T, Hv, Dv]`` in
    ``qkv_dtype``, ``beta [T, Hv], log_decay [T, Hv])``."""
    torch = _torch()
    tokens, channels = (int(x) for x in current.shape)
    if weight_layout == "kc":
        kernel = int(conv_weight.shape[0])
        tap_stride, ch_stride = channels, 1
    else:
        kernel = int(conv_weight.shape[1])
        tap_stride, ch_stride = 1, kernel
    dev = current.device
    q = torch.empty((tokens, int(key_heads), int(key_dim)), dtype=qkv_dtype, device=dev)
    k = torch.empty_like(q)
    v = torch.empty((tokens, int(value_heads), int(value_dim)), dtype=qkv_dtype, device=dev)
    beta = torch.empty((tokens, int(value_heads)), dtype=torch.float32, device=dev)
    g = torch.empty_like(beta)
    rc = _lib.lib().alpx_recurrent_prefill_prep(
        current.data_ptr(), conv_weight.data_ptr(), tap_stride, ch_stride,
        None if conv_history is None else conv_history.data_ptr(), kernel,
        beta_logits.data_ptr(), alpha_logits.data_ptr(), dt_bias.data_ptr(), ssm_a.data_ptr(),
        q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), g.data_ptr(), tokens,
        int(key_heads), int(value_heads), int(key_dim), int(value_dim), float(eps),
        _lib.dtype_code(torch, qkv_dtype), _lib.stream_handle(torch, dev))
    _lib.check(rc)
    return q, k, v, beta, g


def _recurrent_step_call(current, conv_weight, conv_history, gate, beta_logits, alpha_logits,
                         dt_bias, ssm_a, norm_weight, state, *, key_heads, key_dim, eps,
                         weight_layout="kc", out_dtype=None, out=None):
    torch = _torch()
    bsz, hv, dv, dk = state.shape
    channels = current.shape[1]
    if weight_layout == "kc":
        kernel = conv_weight.shape[0]
        tap_stride, ch_stride = channels, 1
    else:
        kernel = conv_weight.shape[1]
        tap_stride, ch_stride = 1, kernel
    device = state.device
    if out is None:
        out = torch.empty((bsz, hv * dv),
                          dtype=torch.float32 if out_dtype is None else out_dtype, device=device)
    L = _lib.lib()
    key_heads, key_dim = int(key_heads), int(key_dim)
    nbytes = L.alpx_recurrent_step_workspace_bytes(bsz, key_heads, hv, key_dim, dv)
    if nbytes == 0:
        raise ValueError("invalid recurrent step sizes")
    ws = _lib.workspace(torch, device, nbytes)
    args = [current.data_ptr(), conv_weight.data_ptr(), tap_stride, ch_stride,
            None if conv_history is None else conv_history.data_ptr(), kernel, gate.data_ptr(),
            beta_logits.data_ptr(), alpha_logits.data_ptr(), dt_bias.data_ptr(),
            ssm_a.data_ptr(), norm_weight.data_ptr(), state.data_ptr(), out.data_ptr(),
            ws.data_ptr(), ws.numel(), bsz, key_heads, hv, key_dim, dv, float(eps),
            _lib.dtype_code(torch, out.dtype), None]
    buffers = (current, conv_weight, conv_history, gate, beta_logits, alpha_logits, dt_bias,
               ssm_a, norm_weight, state, ws)
    return L.alpx_recurrent_step, args, device, out, buffers


def recurrent_step(*args, **kwargs):
    """Fused Qwen3.5 recurrent-layer token (all fp32 inputs): arguments
    current, conv_weight, conv_history, gate, beta_logits, alpha_logits,
    dt_bias, ssm_a, norm_weight, state and the keywords key_heads, key_dim,
    eps, weight_layout ("kc": [K, C] weights, else [C, K]), out_dtype, out.
    Updates ``conv_history [B, K-1, C]`` and ``state [B, Hv, Dv, Dk]`` in
    place and returns ``[B, Hv * Dv]``."""
    fn, call_args, device, out, _ = _recurrent_step_call(*args, **kwargs)
    return _run(fn, call_args, device, out)


def prepare_recurrent_step(*args, **kwargs):
    """``recurrent_step`` as a PreparedCall (same arguments)."""
    fn, call_args, device, out, buffers = _recurrent_step_call(*args, **kwargs)
    return PreparedCall(fn, call_args, device, buffers + (out,), out)
