"""Drop-in for alpaccaroo's ``Qwen35RocmOps`` attention/recurrence surface.

Mirrors ``alpaccaroo/qwen35_rocm_ops.py`` (class ``Qwen35RocmOps``,
qwen35_rocm_ops.py:89-589): same method names, argument order, tensor
layouts, return conventions and exception types for the hot path:

* ``initialize_attention_workspace`` -> caches ``[capacity, batch, kv_heads,
  dim]`` (qwen35_rocm_ops.py:214-238)
* ``initialize_recurrent_workspace`` -> conv history + delta state
  ``[batch, value_heads, value, key]`` (qwen35_rocm_ops.py:186-212)
* ``attention_append_`` (qwen35_rocm_ops.py:475-500)
* ``online_attention`` (qwen35_rocm_ops.py:502-564)
* ``append_online_attention_`` (qwen35_rocm_ops.py:566-589)
* ``sigmoid_gate`` (qwen35_rocm_ops.py:286-290)
* ``gated_delta_net_step_`` (qwen35_rocm_ops.py:362-407)
* ``state_copy`` / ``state_restore_`` (qwen35_rocm_ops.py:240-249)

Differences, all extensions that keep the base signatures:

* float16 and bfloat16 buffers are accepted next to float32 (the reference
  is float32-only, qwen35_rocm_ops.py:153-158); arithmetic is fp32;
* ``online_attention`` takes optional ``seq_lens`` (ragged batch),
  ``gate`` (fused sigmoid output gate) and ``out_dtype``;
* the capability check qualifies a gfx950 (MI355X) device and the built
  library instead of the reference's gfx1151 APU gate.

Every method runs in the HIP library (libalpx.so) through its C-ABI; there
is no PyTorch compute fallback.
"""

from __future__ import annotations

import importlib
import math
from dataclasses import dataclass
from typing import Any, Sequence

from . import _lib, _ops


class Qwen35RocmUnavailable(RuntimeError):
    """Raised when the gfx950 path cannot be used (qwen35_rocm.py:43-53)."""

    def __init__(self, message: str, *, diagnostics=None) -> None:
        super().__init__(message)
        self.diagnostics = None if diagnostics is None else dict(diagnostics)


@dataclass(frozen=True)
class RocmCapability:
    available: bool
    reason: str
    device_index: int | None = None
    gcn_arch_name: str | None = None


TARGET_GFX = "gfx950"


def rocm_capability(device_index: int | None = None) -> RocmCapability:
    """Fail-closed check: PyTorch-ROCm, a visible gfx950 device, libalpx."""
    try:
        torch = importlib.import_module("torch")
    except Exception as exc:  # pragma: no cover
        return RocmCapability(False, f"PyTorch is not importable: {exc}")
    if getattr(torch.version, "hip", None) is None:
        return RocmCapability(False, "PyTorch is not a ROCm build")
    if not torch.cuda.is_available():
        return RocmCapability(False, "no HIP device is visible")
    index = torch.cuda.current_device() if device_index is None else int(device_index)
    try:
        arch = _lib.device_arch(index)
    except Exception as exc:
        return RocmCapability(False, f"libalpx unavailable: {exc}", index)
    if arch.split(":")[0] != TARGET_GFX:
        return RocmCapability(False, f"device {index} is {arch}, not {TARGET_GFX}", index, arch)
    return RocmCapability(True, "ok", index, arch)


def _positive_integer(name: str, value: int) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
        raise ValueError(f"{name} must be a positive integer")
    return value


def _nonnegative_integer(name: str, value: int) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ValueError(f"{name} must be a non-negative integer")
    return value


def _positive_finite(name: str, value: float) -> float:
    value = float(value)
    if not math.isfinite(value) or value <= 0.0:
        raise ValueError(f"{name} must be positive and finite")
    return value


def _shape(tensor: Any) -> tuple[int, ...]:
    shape = tensor.shape
    if isinstance(shape, tuple):  # torch.Size: already a tuple of ints
        return shape
    return tuple(int(value) for value in shape)


def _tensor_descriptor(tensor: Any) -> dict[str, Any]:
    device = tensor.device
    index = getattr(device, "index", None)
    return {
        "shape": list(_shape(tensor)),
        "dtype": str(tensor.dtype),
        "device": f"{device.type}:{0 if index is None else index}",
        "contiguous": bool(tensor.is_contiguous()),
    }


@dataclass(frozen=True)
class RocmRecurrentWorkspace:
    """Zero-initialized recurrent state on the device (qwen35_rocm_ops.py:57-70)."""

    convolution_history: Any
    delta_state: Any

    def descriptor(self) -> dict[str, Any]:
        return {
            "convolution_history": _tensor_descriptor(self.convolution_history),
            "delta_state": _tensor_descriptor(self.delta_state),
            "delta_state_orientation": "batch,value_head,value,key",
            "initialization": "deterministic-zero",
        }


@dataclass(frozen=True)
class RocmAttentionWorkspace:
    """Preallocated K/V capacity; the chain owns the logical length
    (qwen35_rocm_ops.py:73-86)."""

    key_cache: Any
    value_cache: Any

    def descriptor(self) -> dict[str, Any]:
        return {
            "key_cache": _tensor_descriptor(self.key_cache),
            "value_cache": _tensor_descriptor(self.value_cache),
            "layout": "capacity,batch,kv_head,head_dimension",
            "initialization": "deterministic-zero",
        }


@dataclass(frozen=True)
class RocmPagedAttentionWorkspace:
    """A paged K/V pool (extension): pages ``[num_pages, page_size,
    kv_heads, dim]``; a caller-owned int32 block table ``[batch, max_pages]``
    maps each sequence's logical pages to pool pages."""

    key_pages: Any
    value_pages: Any
    page_size: int

    def descriptor(self) -> dict[str, Any]:
        return {
            "key_pages": _tensor_descriptor(self.key_pages),
            "value_pages": _tensor_descriptor(self.value_pages),
            "layout": "page,row_in_page,kv_head,head_dimension",
            "page_size": self.page_size,
            "initialization": "deterministic-zero",
        }


class Qwen35RocmOps:
    """gfx950 implementation of the Qwen35 attention/recurrence boundaries."""

    def __init__(self, *, device_index: int | None = None, _torch: Any | None = None,
                 _capability: RocmCapability | None = None) -> None:
        capability = rocm_capability(device_index) if _capability is None else _capability
        if not capability.available:
            raise Qwen35RocmUnavailable(capability.reason)
        selected = capability.device_index if device_index is None else device_index
        if selected is None:
            raise Qwen35RocmUnavailable("ROCm capability has no target device index")
        _nonnegative_integer("device_index", selected)
        if capability.device_index is not None and selected != capability.device_index:
            raise ValueError(
                f"device_index {selected} differs from qualified target "
                f"{capability.device_index}")
        self.torch = importlib.import_module("torch") if _torch is None else _torch
        self.capability = capability
        self.device_index = selected
        self.device = f"cuda:{selected}"
        t = self.torch
        self._float_dtypes = frozenset((t.float32, t.float16, t.bfloat16))
        self._int_dtypes = self._float_dtypes | {t.int64, t.int32}

    def descriptor(self) -> dict[str, Any]:
        return {
            "backend": "hip-gfx950-libalpx",
            "device": self.device,
            "gcn_arch_name": self.capability.gcn_arch_name,
            "tensor_dtype": "float32|float16|bfloat16",
            "host_transfer_api": False,
            "state_orientation": "batch,value_head,value,key",
            "recurrent_key_mapping": "value_head % key_head_count",
            "attention_key_mapping": "contiguous-query-head-groups",
            "attention_algorithm": "split-k-online-softmax",
            "supported_attention_head_dimensions": "1..256",
        }

    # ------------------------------------------------------------ validation

    def _tensor(self, value: Any, name: str, *, dimensions: int | None = None,
                allow_integer: bool = False) -> Any:
        """Contract check of qwen35_rocm_ops.py:134-165, widened to fp16/bf16."""
        torch = self.torch
        if not isinstance(value, torch.Tensor):
            raise TypeError(f"{name} must be a PyTorch tensor")
        if not value.is_cuda:
            raise TypeError(f"{name} must remain on the ROCm device")
        index = value.get_device()
        if index != self.device_index:
            raise ValueError(f"{name} is on device {index}, expected {self.device_index}")
        if value.dtype not in (self._int_dtypes if allow_integer else self._float_dtypes):
            expected = "float32, float16 or bfloat16"
            raise TypeError(f"{name} must use {expected}" + (" or int" if allow_integer else ""))
        if dimensions is not None and value.dim() != dimensions:
            raise ValueError(f"{name} has {_shape(value)}, expected {dimensions} dimensions")
        if not value.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        return value

    def _out_buffer(self, out: Any, shape: tuple, dtype: Any, name: str) -> None:
        """An ``out=`` buffer: a contiguous tensor of ``shape`` and ``dtype`` on
        this device."""
        self._tensor(out, name)
        if out.dtype != dtype:
            raise TypeError(f"{name} must use {dtype}")
        if out.shape != shape:
            raise ValueError(f"{name} has {_shape(out)}, expected {tuple(shape)}")

    @staticmethod
    def _same_shape(left: Any, right: Any, what: str) -> None:
        if _shape(left) != _shape(right):
            raise ValueError(f"{what} shapes differ: {_shape(left)} != {_shape(right)}")

    @staticmethod
    def _same_dtype(what: str, *tensors: Any) -> None:
        dtypes = {t.dtype for t in tensors}
        if len(dtypes) != 1:
            raise TypeError(f"{what} tensors must share one dtype, got {sorted(map(str, dtypes))}")

    # ------------------------------------------------------------ workspaces

    def zeros(self, shape: Sequence[int], dtype: Any = None) -> Any:
        normalized = tuple(_positive_integer("workspace dimension", v) for v in shape)
        if not normalized:
            raise ValueError("workspace shape cannot be empty")
        dtype = self.torch.float32 if dtype is None else dtype
        return self.torch.zeros(normalized, dtype=dtype, device=self.device)

    def initialize_recurrent_workspace(self, *, batch_size: int, convolution_kernel: int,
                                       convolution_channels: int, value_heads: int,
                                       value_dimension: int,
                                       key_dimension: int) -> RocmRecurrentWorkspace:
        batch = _positive_integer("batch_size", batch_size)
        kernel = _positive_integer("convolution_kernel", convolution_kernel)
        channels = _positive_integer("convolution_channels", convolution_channels)
        heads = _positive_integer("value_heads", value_heads)
        value_width = _positive_integer("value_dimension", value_dimension)
        key_width = _positive_integer("key_dimension", key_dimension)
        history = self.torch.zeros((batch, kernel - 1, channels), dtype=self.torch.float32,
                                   device=self.device)
        state = self.torch.zeros((batch, heads, value_width, key_width),
                                 dtype=self.torch.float32, device=self.device)
        return RocmRecurrentWorkspace(history, state)

    def initialize_attention_workspace(self, *, capacity: int, batch_size: int, kv_heads: int,
                                       key_dimension: int, value_dimension: int,
                                       dtype: Any = None) -> RocmAttentionWorkspace:
        length = _positive_integer("capacity", capacity)
        batch = _positive_integer("batch_size", batch_size)
        heads = _positive_integer("kv_heads", kv_heads)
        key_width = _positive_integer("key_dimension", key_dimension)
        value_width = _positive_integer("value_dimension", value_dimension)
        dtype = self.torch.float32 if dtype is None else dtype
        keys = self.torch.zeros((length, batch, heads, key_width), dtype=dtype, device=self.device)
        values = self.torch.zeros((length, batch, heads, value_width), dtype=dtype,
                                  device=self.device)
        return RocmAttentionWorkspace(keys, values)

    def state_copy(self, source: Any) -> Any:
        source = self._tensor(source, "state source")
        return source.clone()

    def state_restore_(self, target: Any, snapshot: Any) -> Any:
        target = self._tensor(target, "state target")
        snapshot = self._tensor(snapshot, "state snapshot")
        self._same_shape(target, snapshot, "state restore")
        target.copy_(snapshot)
        return target

    # ------------------------------------------------------------ attention

    def attention_append_(self, key_cache: Any, value_cache: Any, position: int, key: Any,
                          value: Any) -> int:
        key_cache = self._tensor(key_cache, "attention key cache", dimensions=4)
        value_cache = self._tensor(value_cache, "attention value cache", dimensions=4)
        key = self._tensor(key, "attention key", dimensions=3)
        value = self._tensor(value, "attention value", dimensions=3)
        position = _nonnegative_integer("attention cache position", position)
        if int(key_cache.shape[0]) != int(value_cache.shape[0]):
            raise ValueError("attention K/V cache capacities differ")
        if position >= int(key_cache.shape[0]):
            raise ValueError("attention cache position exceeds capacity")
        if _shape(key_cache)[1:3] != _shape(value_cache)[1:3]:
            raise ValueError("attention K/V cache batch and head axes differ")
        if _shape(key) != _shape(key_cache)[1:]:
            raise ValueError("attention key does not match cache token shape")
        if _shape(value) != _shape(value_cache)[1:]:
            raise ValueError("attention value does not match cache token shape")
        self._same_dtype("attention append", key_cache, value_cache, key, value)
        _ops.kv_append(key_cache, value_cache, key.unsqueeze(0), value.unsqueeze(0),
                       position=position)
        return position + 1

    def attention_append_rows_(self, key_cache: Any, value_cache: Any, key: Any, value: Any, *,
                               position: int | None = None, positions: Any = None) -> None:
        """Multi-token / ragged append (extension): ``key [T, B, Hkv, D]``
        rows land at ``position + t`` or, per sequence, ``positions[b] + t``."""
        key_cache = self._tensor(key_cache, "attention key cache", dimensions=4)
        value_cache = self._tensor(value_cache, "attention value cache", dimensions=4)
        key = self._tensor(key, "attention key rows", dimensions=4)
        value = self._tensor(value, "attention value rows", dimensions=4)
        if _shape(key)[1:] != _shape(key_cache)[1:] or _shape(value)[1:] != _shape(value_cache)[1:]:
            raise ValueError("attention rows do not match cache token shape")
        if int(key.shape[0]) != int(value.shape[0]):
            raise ValueError("attention K/V row counts differ")
        self._same_dtype("attention append", key_cache, value_cache, key, value)
        tokens = int(key.shape[0])
        capacity = int(key_cache.shape[0])
        if positions is None:
            position = _nonnegative_integer("attention cache position", position)
            if position + tokens > capacity:
                raise ValueError("attention cache position exceeds capacity")
        elif not self.torch.is_tensor(positions) or positions.device.type != "cuda":
            host = [int(p) for p in positions]
            if len(host) != int(key_cache.shape[1]):
                raise ValueError("positions must have one entry per sequence")
            if any(p < 0 or p + tokens > capacity for p in host):
                raise ValueError("attention cache position exceeds capacity")
            positions = self.torch.tensor(host, dtype=self.torch.int32, device=self.device)
        _ops.kv_append(key_cache, value_cache, key, value, position=position, positions=positions)

    def online_attention(self, query: Any, key_cache: Any, value_cache: Any, *, length: int,
                         scale: float | None = None, seq_lens: Any = None, gate: Any = None,
                         out_dtype: Any = None, out: Any = None) -> Any:
        """Single-token GQA decode over the ROCm cache layout
        (qwen35_rocm_ops.py:502-564).  Extensions: fp16 / bf16 tensors,
        device ``seq_lens [B]`` (ragged batch), the sigmoid output ``gate``,
        ``out_dtype`` and an ``out`` buffer."""
        return _ops.decode(query, key_cache, value_cache,
                           **self._online_attention_args(query, key_cache, value_cache, length,
                                                         scale, seq_lens, gate, out_dtype, out))

    def prepare_online_attention(self, query: Any, key_cache: Any, value_cache: Any, *,
                                 length: int, scale: float | None = None, seq_lens: Any = None,
                                 gate: Any = None, out_dtype: Any = None,
                                 out: Any = None) -> Any:
        """``online_attention`` validated and packed once (extension): returns a
        call object whose every call runs the decode on the buffers given here
        (their contents, e.g. the query row and device ``seq_lens``, may change
        between calls; their shapes and storage may not) and returns the
        output buffer.  For decode loops that do not capture graphs."""
        return _ops.prepare_decode(
            query, key_cache, value_cache,
            **self._online_attention_args(query, key_cache, value_cache, length, scale, seq_lens,
                                          gate, out_dtype, out))

    def _online_attention_args(self, query, key_cache, value_cache, length, scale, seq_lens,
                               gate, out_dtype, out):
        query = self._tensor(query, "attention query", dimensions=3)
        key_cache = self._tensor(key_cache, "attention key cache", dimensions=4)
        value_cache = self._tensor(value_cache, "attention value cache", dimensions=4)
        length = _positive_integer("attention cache length", length)
        capacity, batch, kv_heads, key_width = _shape(key_cache)
        value_shape = _shape(value_cache)
        if length > capacity:
            raise ValueError("attention cache length exceeds capacity")
        if value_shape[:3] != (capacity, batch, kv_heads):
            raise ValueError("attention K/V cache capacity, batch, or heads differ")
        query_batch, query_heads, query_width = _shape(query)
        if query_batch != batch or query_width != key_width:
            raise ValueError("attention query does not match K cache batch/head width")
        if kv_heads <= 0 or query_heads % kv_heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        scale_value = (1.0 / math.sqrt(key_width) if scale is None
                       else _positive_finite("attention scale", scale))
        self._same_dtype("attention", query, key_cache, value_cache)
        if gate is not None:
            gate = self._tensor(gate, "sigmoid-gate logits", dimensions=3)
            if _shape(gate) != (batch, query_heads, value_shape[3]):
                raise ValueError("sigmoid-gate logits must match the attention output")
            self._same_dtype("attention gate", query, gate)
        if seq_lens is not None:
            if not self.torch.is_tensor(seq_lens) or seq_lens.device.type != "cuda":
                host = [int(n) for n in seq_lens]
                if len(host) != batch or any(n < 1 or n > length for n in host):
                    raise ValueError("seq_lens must hold one length in [1, length] per sequence")
                seq_lens = self.torch.tensor(host, dtype=self.torch.int32, device=self.device)
            elif _shape(seq_lens) != (batch,):
                raise ValueError("seq_lens must hold one length per sequence")
        if out is not None:
            self._out_buffer(out, (batch, query_heads, value_shape[3]),
                             query.dtype if out_dtype is None else out_dtype,
                             "attention output")
        c, b, h = batch * kv_heads * key_width, kv_heads * key_width, key_width
        cv, bv, hv = batch * kv_heads * value_shape[3], kv_heads * value_shape[3], value_shape[3]
        return dict(length=length, k_strides=(c, b, h), v_strides=(cv, bv, hv), batch=batch,
                    kv_heads=kv_heads, seq_lens=seq_lens, gate=gate, scale=scale_value,
                    out_dtype=out_dtype, out=out)

    def append_online_attention_(self, query: Any, key: Any, value: Any, key_cache: Any,
                                 value_cache: Any, *, position: int,
                                 scale: float | None = None) -> tuple[Any, int]:
        length = self.attention_append_(key_cache, value_cache, position, key, value)
        return (self.online_attention(query, key_cache, value_cache, length=length,
                                      scale=scale), length)

    def attention_prefill(self, query: Any, key_cache: Any, value_cache: Any, *,
                          position: int, batch_index: int = 0, scale: float | None = None,
                          window: int = 0, out_dtype: Any = None, gate: Any = None) -> Any:
        """Causal prefill over the ROCm cache layout (extension): query
        ``[T, Hq, D]`` of sequence ``batch_index`` at positions
        ``position .. position + T - 1`` attends to its cache rows
        ``0 .. position + t`` (``qwen35_full_attention_prefill`` semantics,
        qwen35_kernels.py:395-411, with prefix_length = position).  With
        ``gate [T, Hq, Dv]`` the output is ``attention * sigmoid(gate)``
        (the gate placement of qwen35_runtime.py:653-660), formed before
        the output is rounded."""
        query = self._tensor(query, "prefill query", dimensions=3)
        key_cache = self._tensor(key_cache, "attention key cache", dimensions=4)
        value_cache = self._tensor(value_cache, "attention value cache", dimensions=4)
        position = _nonnegative_integer("attention cache position", position)
        batch_index = _nonnegative_integer("batch_index", batch_index)
        window = _nonnegative_integer("window", window)
        capacity, batch, kv_heads, key_width = _shape(key_cache)
        value_shape = _shape(value_cache)
        tokens, query_heads, query_width = _shape(query)
        if value_shape[:3] != (capacity, batch, kv_heads):
            raise ValueError("attention K/V cache capacity, batch, or heads differ")
        if batch_index >= batch:
            raise ValueError("batch_index exceeds the cache batch")
        if position + tokens > capacity:
            raise ValueError("attention cache position exceeds capacity")
        if query_width != key_width:
            raise ValueError("prefill query does not match K cache head width")
        if query_heads % kv_heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        self._same_dtype("prefill", query, key_cache, value_cache)
        if gate is not None:
            gate = self._tensor(gate, "attention output gate", dimensions=3)
            if _shape(gate) != (tokens, query_heads, value_shape[3]):
                raise ValueError("sigmoid gate must match values")
            self._same_dtype("prefill gate", query, gate)
        scale_value = (1.0 / math.sqrt(key_width) if scale is None
                       else _positive_finite("attention scale", scale))
        return _ops.prefill(query, key_cache[0, batch_index], value_cache[0, batch_index],
                            pos0=position, scale=scale_value, window=window,
                            kv_tokens=position + tokens,
                            k_pos_stride=batch * kv_heads * key_width,
                            v_pos_stride=batch * kv_heads * value_shape[3],
                            out_dtype=out_dtype, gate=gate)

    def append_prefill_attention_(self, query: Any, key: Any, value: Any, key_cache: Any,
                                  value_cache: Any, *, position: int,
                                  scale: float | None = None) -> tuple[Any, int]:
        """Prefill-chunk form of ``append_online_attention_`` for a batch-1
        cache (extension): append ``key/value [T, Hkv, D]`` at ``position``
        (bit-exact), then causal prefill attention of ``query [T, Hq, D]``
        over cache rows ``0 .. position + t``.  One kernel does both on the
        MFMA path (it reads the chunk's rows from ``key/value`` and writes
        them to the caches).  Returns ``(output [T, Hq, Dv], position + T)``."""
        query = self._tensor(query, "prefill query", dimensions=3)
        key_cache = self._tensor(key_cache, "attention key cache", dimensions=4)
        value_cache = self._tensor(value_cache, "attention value cache", dimensions=4)
        key = self._tensor(key, "attention key rows", dimensions=3)
        value = self._tensor(value, "attention value rows", dimensions=3)
        capacity, batch, kv_heads, key_width = _shape(key_cache)
        if batch != 1:
            raise ValueError("append_prefill_attention_ needs a batch-1 cache")
        value_shape = _shape(value_cache)
        if value_shape[:3] != (capacity, batch, kv_heads):
            raise ValueError("attention K/V cache capacity, batch, or heads differ")
        if _shape(key)[1:] != (kv_heads, key_width) or _shape(value)[1:] != value_shape[2:]:
            raise ValueError("attention rows do not match cache token shape")
        tokens, query_heads, query_width = _shape(query)
        if int(key.shape[0]) != int(value.shape[0]):
            raise ValueError("attention K/V row counts differ")
        if int(key.shape[0]) != tokens:
            raise ValueError("prefill query and K/V row counts differ")
        position = _nonnegative_integer("attention cache position", position)
        if position + tokens > capacity:
            raise ValueError("attention cache position exceeds capacity")
        if query_width != key_width:
            raise ValueError("prefill query does not match K cache head width")
        if query_heads % kv_heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        self._same_dtype("prefill", query, key_cache, value_cache, key, value)
        scale_value = (1.0 / math.sqrt(key_width) if scale is None
                       else _positive_finite("attention scale", scale))
        out = _ops.prefill_append(query, key, value, key_cache, value_cache, position=position,
                                  scale=scale_value)
        return out, position + tokens

    # ------------------------------------------------------------ recurrence

    def _gdn_checks(self, state, query, key, value, beta, log_decay, *, chunk):
        dims = 4 if chunk else 3
        state = self._tensor(state, "GDN state", dimensions=4)
        query = self._tensor(query, "GDN query", dimensions=dims)
        key = self._tensor(key, "GDN key", dimensions=dims)
        value = self._tensor(value, "GDN value", dimensions=dims)
        beta = self._tensor(beta, "GDN beta", dimensions=dims - 1)
        log_decay = self._tensor(log_decay, "GDN log decay", dimensions=dims - 1)
        torch = self.torch
        if state.dtype != torch.float32:
            raise TypeError("GDN state must use float32")
        if beta.dtype != torch.float32 or log_decay.dtype != torch.float32:
            raise TypeError("GDN beta and log decay must use float32")
        self._same_dtype("GDN", query, key, value)
        batch, value_heads, value_width, key_width = _shape(state)
        lead = _shape(query)[:-2]
        if _shape(query) != _shape(key):
            raise ValueError("GDN query and key shapes must agree")
        if lead[0] != batch or _shape(query)[-1] != key_width:
            raise ValueError("GDN query/key must match state batch and key dimension")
        key_heads = int(query.shape[-2])
        if key_heads <= 0 or value_heads % key_heads:
            raise ValueError("GDN value heads must be a multiple of key heads")
        if _shape(value) != lead + (value_heads, value_width):
            raise ValueError("GDN value must match state batch/value-head/value axes")
        if _shape(beta) != lead + (value_heads,):
            raise ValueError("GDN beta must match batch and value heads")
        if _shape(log_decay) != lead + (value_heads,):
            raise ValueError("GDN log decay must match batch and value heads")
        return state, query, key, value, beta, log_decay

    def gated_delta_net_step_(self, state: Any, query: Any, key: Any, value: Any, beta: Any,
                              log_decay: Any, *, out: Any = None) -> Any:
        """One GDN step in place on ``state [B, Hv, Dv, Dk]``
        (qwen35_rocm_ops.py:362-407); value head h reads key head h % Hk.
        ``out`` (extension): a contiguous ``[B, Hv, Dv]`` buffer of the
        query dtype on the same device that receives the result (no
        allocation per step); it is returned."""
        args = self._gdn_checks(state, query, key, value, beta, log_decay, chunk=False)
        if out is not None:
            self._out_buffer(out, (state.shape[0], state.shape[1], state.shape[2]), query.dtype,
                             "GDN output")
        return _ops.gdn_step(*args, out=out)

    def prepare_gated_delta_net_step_(self, state: Any, query: Any, key: Any, value: Any,
                                      beta: Any, log_decay: Any, *, out: Any = None) -> Any:
        """``gated_delta_net_step_`` validated and packed once (extension):
        returns a call object whose every call advances ``state`` in place by
        one step from the current contents of the buffers given here and
        returns the output buffer (allocated once when ``out`` is None).  For
        decode loops that do not capture graphs."""
        args = self._gdn_checks(state, query, key, value, beta, log_decay, chunk=False)
        if out is not None:
            self._out_buffer(out, (state.shape[0], state.shape[1], state.shape[2]), query.dtype,
                             "GDN output")
        return _ops.prepare_gdn_step(*args, out=out)

    def gated_delta_net_chunk_(self, state: Any, query: Any, key: Any, value: Any, beta: Any,
                               log_decay: Any, *, out_dtype: Any = None) -> Any:
        """GDN over a prefill chunk (extension): query/key ``[B, T, Hk, Dk]``,
        value ``[B, T, Hv, Dv]``, beta/log_decay ``[B, T, Hv]``; the state is
        advanced in place exactly as T calls of ``gated_delta_net_step_``
        would, computed in 64-token chunks.  Returns ``[B, T, Hv, Dv]``."""
        args = self._gdn_checks(state, query, key, value, beta, log_decay, chunk=True)
        return _ops.gdn_chunk(*args, out_dtype=out_dtype)

    def sigmoid_gate(self, values: Any, gate: Any) -> Any:
        values = self._tensor(values, "sigmoid-gate values")
        gate = self._tensor(gate, "sigmoid-gate logits")
        self._same_shape(values, gate, "sigmoid gate")
        self._same_dtype("sigmoid gate", values, gate)
        return _ops.sigmoid_gate(values, gate)

    # ------------------------------------------------ layer primitives

    def _fp32(self, value: Any, name: str, *, dimensions: int | None = None) -> Any:
        value = self._tensor(value, name, dimensions=dimensions)
        if value.dtype != self.torch.float32:
            raise TypeError(f"{name} must use float32")
        return value

    def silu(self, values: Any) -> Any:
        """``values * sigmoid(values)`` (qwen35_rocm_ops.py:276-278)."""
        values = self._tensor(values, "SiLU input")
        return _ops.silu(values)

    def rms_norm(self, values: Any, weight: Any, epsilon: float) -> Any:
        """Learned RMSNorm over the final axis (qwen35_rocm_ops.py:251-258)."""
        values = self._tensor(values, "RMSNorm input")
        weight = self._fp32(weight, "RMSNorm weight", dimensions=1)
        epsilon = _positive_finite("epsilon", epsilon)
        if not values.shape or int(values.shape[-1]) != int(weight.shape[0]):
            raise ValueError("RMSNorm weight must match the input's final dimension")
        return _ops.row_norm(values, mode=_lib.NORM_RMS, eps=epsilon, weight=weight)

    def l2_normalize(self, values: Any, epsilon: float) -> Any:
        """``values / max(||values||, epsilon)`` over the final axis
        (qwen35_rocm_ops.py:260-268)."""
        values = self._tensor(values, "L2 input")
        epsilon = _positive_finite("epsilon", epsilon)
        if not values.shape or int(values.shape[-1]) <= 0:
            raise ValueError("L2 input final dimension must be nonempty")
        return _ops.row_norm(values, mode=_lib.NORM_L2, eps=epsilon)

    def recurrent_gate(self, values: Any, weight: Any, gate: Any, epsilon: float) -> Any:
        """``rms_norm(values) * silu(gate)`` (qwen35_rocm_ops.py:292-296)."""
        values = self._tensor(values, "RMSNorm input")
        weight = self._fp32(weight, "RMSNorm weight", dimensions=1)
        epsilon = _positive_finite("epsilon", epsilon)
        if not values.shape or int(values.shape[-1]) != int(weight.shape[0]):
            raise ValueError("RMSNorm weight must match the input's final dimension")
        gate = self._tensor(gate, "recurrent SiLU gate")
        self._same_shape(values, gate, "recurrent gate")
        self._same_dtype("recurrent gate", values, gate)
        return _ops.row_norm(values, mode=_lib.NORM_RMS_GATE, eps=epsilon, weight=weight,
                             gate=gate)

    def split_query_gate(self, projected: Any, *, query_heads: int,
                         head_dimension: int) -> tuple[Any, Any]:
        """Split the joint Q/gate projection: per head ``head_dimension``
        query values then as many gate values (qwen35_rocm_ops.py:298-318)."""
        projected = self._tensor(projected, "joint Q/gate projection")
        heads = _positive_integer("query_heads", query_heads)
        width = _positive_integer("head_dimension", head_dimension)
        expected = heads * 2 * width
        actual = int(projected.shape[-1]) if projected.shape else 0
        if actual != expected:
            raise ValueError(
                f"joint Q/gate width is {actual}, expected "
                f"{expected} ({heads} heads * Q/gate stride {2 * width})")
        reshaped = projected.reshape(_shape(projected)[:-1] + (heads, 2 * width))
        return reshaped[..., :width].contiguous(), reshaped[..., width:].contiguous()

    def causal_convolution_step_(self, current: Any, weights: Any, history: Any) -> Any:
        """Raw depthwise causal convolution of ``current [B, C]`` with
        ``weights [K, C]``; ``history [B, K-1, C]`` shifts in place
        (qwen35_rocm_ops.py:320-341).  SiLU is the separate ``silu``."""
        current = self._fp32(current, "convolution current", dimensions=2)
        weights = self._fp32(weights, "convolution weights", dimensions=2)
        history = self._fp32(history, "convolution history", dimensions=3)
        batch, channels = _shape(current)
        kernel, weight_channels = _shape(weights)
        if weight_channels != channels:
            raise ValueError("convolution weights must match current channels")
        if _shape(history) != (batch, kernel - 1, channels):
            raise ValueError(
                "convolution history must have shape "
                f"{(batch, kernel - 1, channels)}, got {_shape(history)}")
        return _ops.conv_step(current, weights, history if kernel > 1 else None)

    def recurrent_parameters(self, beta_logits: Any, alpha_logits: Any, dt_bias: Any,
                             ssm_a: Any) -> tuple[Any, Any]:
        """``(sigmoid(beta_logits), softplus(alpha_logits + dt_bias) * ssm_a)``
        (qwen35_rocm_ops.py:343-360)."""
        beta_logits = self._fp32(beta_logits, "beta logits", dimensions=2)
        alpha_logits = self._fp32(alpha_logits, "alpha logits", dimensions=2)
        dt_bias = self._fp32(dt_bias, "time-step bias", dimensions=1)
        ssm_a = self._fp32(ssm_a, "converted ssm_a", dimensions=1)
        self._same_shape(beta_logits, alpha_logits, "recurrent parameter logits")
        heads = int(beta_logits.shape[1])
        if _shape(dt_bias) != (heads,) or _shape(ssm_a) != (heads,):
            raise ValueError("time-step bias and ssm_a must match value heads")
        return _ops.recurrent_parameters(beta_logits, alpha_logits, dt_bias, ssm_a)

    def imrope(self, values: Any, position_lanes: Any, sections: Sequence[int], *,
               frequency_base: float, frequency_scale: float = 1.0) -> Any:
        """IMROPE with one position-lane vector ``(4,)`` (int64) for every
        row (qwen35_rocm_ops.py:409-473); a ``[rows, 4]`` lane array gives
        each row (all axes but the last) its own lanes (extension)."""
        values = self._tensor(values, "IMRoPE input")
        position_lanes = self._tensor(position_lanes, "IMRoPE position lanes",
                                      allow_integer=True)
        rows = values.numel() // max(1, int(values.shape[-1])) if values.shape else 0
        if position_lanes.dtype != self.torch.int64 or (
                _shape(position_lanes) != (4,) and _shape(position_lanes) != (rows, 4)):
            raise ValueError("IMRoPE position lanes must be int64 shape (4,)")
        if len(sections) != 4:
            raise ValueError("IMRoPE requires four sections")
        section = tuple(_nonnegative_integer("IMRoPE section", item) for item in sections)
        rotary_pairs = sum(section)
        if rotary_pairs <= 0:
            raise ValueError("IMRoPE requires at least one rotary pair")
        if not values.shape or int(values.shape[-1]) < 2 * rotary_pairs:
            raise ValueError("IMRoPE input is shorter than twice the section sum")
        base = _positive_finite("frequency_base", frequency_base)
        scale = _positive_finite("frequency_scale", frequency_scale)
        return _ops.imrope(values, position_lanes, section, frequency_base=base,
                           frequency_scale=scale)

    def attention_prologue_(self, query_gate: Any, key: Any, value: Any, query_norm: Any,
                            key_norm: Any, key_cache: Any, value_cache: Any, *, position: int,
                            sections: Sequence[int], frequency_base: float,
                            epsilon: float) -> tuple[Any, Any, int]:
        """Fused Qwen3.5 full-attention prologue for one decode token per
        sequence (extension; the steps of qwen35_runtime.py:597-650): split
        the joint projection ``query_gate [B, Hq * 2 D]``, RMSNorm the query
        heads with ``query_norm`` and the key heads ``key [B, Hkv * D]`` with
        ``key_norm``, IMROPE at the text position, and append the rotated
        key and ``value [B, Hkv * Dv]`` at ``position``.  Returns
        ``(query [B, Hq, D], gate [B, Hq, D], position + 1)``; pass the gate
        to ``online_attention(..., gate=gate)``."""
        key_cache = self._tensor(key_cache, "attention key cache", dimensions=4)
        value_cache = self._tensor(value_cache, "attention value cache", dimensions=4)
        capacity, batch, kv_heads, width = _shape(key_cache)
        value_width = int(value_cache.shape[3])
        query_gate = self._tensor(query_gate, "joint Q/gate projection", dimensions=2)
        key = self._tensor(key, "attention key", dimensions=2)
        value = self._tensor(value, "attention value", dimensions=2)
        query_norm = self._fp32(query_norm, "query RMSNorm weight", dimensions=1)
        key_norm = self._fp32(key_norm, "key RMSNorm weight", dimensions=1)
        position = _nonnegative_integer("attention cache position", position)
        if position >= capacity:
            raise ValueError("attention cache position exceeds capacity")
        if _shape(value_cache)[:3] != (capacity, batch, kv_heads):
            raise ValueError("attention K/V cache capacity, batch, or heads differ")
        if int(query_gate.shape[0]) != batch or int(query_gate.shape[1]) % (2 * width):
            raise ValueError("joint Q/gate projection does not match the cache head width")
        query_heads = int(query_gate.shape[1]) // (2 * width)
        if query_heads % kv_heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        if _shape(key) != (batch, kv_heads * width) or _shape(value) != (batch,
                                                                          kv_heads * value_width):
            raise ValueError("attention key/value do not match cache token shape")
        if _shape(query_norm) != (width,) or _shape(key_norm) != (width,):
            raise ValueError("RMSNorm weight must match the head dimension")
        self._same_dtype("attention prologue", query_gate, key, value, key_cache, value_cache)
        if len(sections) != 4:
            raise ValueError("IMRoPE requires four sections")
        section = tuple(_nonnegative_integer("IMRoPE section", item) for item in sections)
        query, gate = _ops.attention_prologue(
            query_gate.reshape(batch, query_heads, 2 * width), key, value, query_norm, key_norm,
            key_cache, value_cache, position=position, sections=section,
            frequency_base=_positive_finite("frequency_base", frequency_base),
            eps=_positive_finite("epsilon", epsilon))
        return query, gate, position + 1

    def attention_layer_step_(self, query_gate: Any, key: Any, value: Any, query_norm: Any,
                              key_norm: Any, key_cache: Any, value_cache: Any, *, position: int,
                              sections: Sequence[int], frequency_base: float, epsilon: float,
                              positions: Any = None, scale: float | None = None,
                              out_dtype: Any = None) -> tuple[Any, int]:
        """One decode token of the Qwen3.5 full-attention layer after its
        projections (extension; qwen35_runtime.py:597-665 for one token per
        sequence): the prologue of ``attention_prologue_`` and the gated
        ``online_attention`` over ``position + 1`` cache rows.  fp16 / bf16
        caches with equal key and value widths of 64, 128 or 256 run it as
        two launches (prologue fused into the split-K launch, gate in the
        combine); other shapes run the prologue and the gated decode as
        separate launches.  ``positions`` (extension; host ints or a device
        int32 tensor ``[B]``) puts sequence b's token at row ``positions[b]``
        (ragged batch); ``position`` then bounds them, and host values above
        it or below 0 are rejected.  Returns ``(gated output [B, Hq, Dv],
        position + 1)``."""
        key_cache = self._tensor(key_cache, "attention key cache", dimensions=4)
        value_cache = self._tensor(value_cache, "attention value cache", dimensions=4)
        capacity, batch, kv_heads, width = _shape(key_cache)
        value_width = int(value_cache.shape[3])
        query_gate = self._tensor(query_gate, "joint Q/gate projection", dimensions=2)
        key = self._tensor(key, "attention key", dimensions=2)
        value = self._tensor(value, "attention value", dimensions=2)
        query_norm = self._fp32(query_norm, "query RMSNorm weight", dimensions=1)
        key_norm = self._fp32(key_norm, "key RMSNorm weight", dimensions=1)
        position = _nonnegative_integer("attention cache position", position)
        if position >= capacity:
            raise ValueError("attention cache position exceeds capacity")
        if _shape(value_cache)[:3] != (capacity, batch, kv_heads):
            raise ValueError("attention K/V cache capacity, batch, or heads differ")
        if int(query_gate.shape[0]) != batch or int(query_gate.shape[1]) % (2 * width):
            raise ValueError("joint Q/gate projection does not match the cache head width")
        query_heads = int(query_gate.shape[1]) // (2 * width)
        if query_heads % kv_heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        if _shape(key) != (batch, kv_heads * width) or _shape(value) != (batch,
                                                                          kv_heads * value_width):
            raise ValueError("attention key/value do not match cache token shape")
        if _shape(query_norm) != (width,) or _shape(key_norm) != (width,):
            raise ValueError("RMSNorm weight must match the head dimension")
        self._same_dtype("attention step", query_gate, key, value, key_cache, value_cache)
        if len(sections) != 4:
            raise ValueError("IMRoPE requires four sections")
        section = tuple(_nonnegative_integer("IMRoPE section", item) for item in sections)
        base = _positive_finite("frequency_base", frequency_base)
        eps = _positive_finite("epsilon", epsilon)
        if positions is not None:
            if not self.torch.is_tensor(positions) or positions.device.type != "cuda":
                host = [int(p) for p in positions]
                if len(host) != batch or any(p < 0 or p > position for p in host):
                    raise ValueError("positions must hold one row in [0, position] per sequence")
                positions = self.torch.tensor(host, dtype=self.torch.int32, device=self.device)
            elif _shape(positions) != (batch,):
                raise ValueError("positions must hold one row per sequence")
            positions = positions.to(self.torch.int32).contiguous()
        query_gate = query_gate.reshape(batch, query_heads, 2 * width)
        fused = (key_cache.dtype in (self.torch.float16, self.torch.bfloat16)
                 and width == value_width and width in (64, 128, 256))
        if not fused:
            # Views of the first position + 1 rows: the prologue writes no
            # row past them, so a device position beyond `position` leaves
            # the cache untouched, as in the fused step.
            kc, vc = key_cache[:position + 1], value_cache[:position + 1]
            query, gate = _ops.attention_prologue(
                query_gate, key, value, query_norm, key_norm, kc, vc, position=position,
                positions=positions, sections=section, frequency_base=base, eps=eps)
            out = self.online_attention(query, kc, vc, length=position + 1, scale=scale,
                                        seq_lens=None if positions is None else positions + 1,
                                        gate=gate, out_dtype=out_dtype)
            return out, position + 1
        scale_value = (1.0 / math.sqrt(width) if scale is None
                       else _positive_finite("attention scale", scale))
        out = _ops.attention_layer_step(
            query_gate, key, value, query_norm, key_norm, key_cache, value_cache,
            position=position, sections=section, frequency_base=base, eps=eps,
            positions=positions, scale=scale_value, out_dtype=out_dtype)
        return out, position + 1

    def recurrent_layer_step_(self, workspace: RocmRecurrentWorkspace, mixed: Any,
                              convolution_weights: Any, gate: Any, beta_logits: Any,
                              alpha_logits: Any, dt_bias: Any, ssm_a: Any, norm_weight: Any, *,
                              key_heads: int, key_dimension: int, epsilon: float,
                              out_dtype: Any = None, out: Any = None) -> Any:
        """One token of the Qwen3.5 recurrent (GDN) layer after its
        projections, fused (extension; the chain of qwen35_numpy.py:63-131):
        convolution + SiLU of ``mixed [B, 2 Hk Dk + Hv Dv]`` against the
        workspace's history, split, Q/K L2 norm, recurrent parameters, the
        GDN step on the workspace's delta state and the gated RMSNorm with
        ``gate [B, Hv * Dv]``.  Both workspace tensors advance in place.
        Returns ``[B, Hv * Dv]``."""
        args, kwargs = self._recurrent_step_args(
            workspace, mixed, convolution_weights, gate, beta_logits, alpha_logits, dt_bias,
            ssm_a, norm_weight, key_heads, key_dimension, epsilon, out_dtype, out)
        return _ops.recurrent_step(*args, **kwargs)

    def prepare_recurrent_layer_step_(self, workspace: RocmRecurrentWorkspace, mixed: Any,
                                      convolution_weights: Any, gate: Any, beta_logits: Any,
                                      alpha_logits: Any, dt_bias: Any, ssm_a: Any,
                                      norm_weight: Any, *, key_heads: int, key_dimension: int,
                                      epsilon: float, out_dtype: Any = None,
                                      out: Any = None) -> Any:
        """``recurrent_layer_step_`` validated and packed once (extension):
        returns a call object whose every call runs one token from the current
        contents of the buffers given here (advancing the workspace in place)
        and returns the output buffer.  For decode loops that do not capture
        graphs."""
        args, kwargs = self._recurrent_step_args(
            workspace, mixed, convolution_weights, gate, beta_logits, alpha_logits, dt_bias,
            ssm_a, norm_weight, key_heads, key_dimension, epsilon, out_dtype, out)
        return _ops.prepare_recurrent_step(*args, **kwargs)

    def _recurrent_step_args(self, workspace, mixed, convolution_weights, gate, beta_logits,
                             alpha_logits, dt_bias, ssm_a, norm_weight, key_heads,
                             key_dimension, epsilon, out_dtype, out):
        history = self._fp32(workspace.convolution_history, "convolution history",
                             dimensions=3)
        state = self._fp32(workspace.delta_state, "GDN state", dimensions=4)
        mixed = self._fp32(mixed, "convolution current", dimensions=2)
        weights = self._fp32(convolution_weights, "convolution weights", dimensions=2)
        gate = self._fp32(gate, "recurrent SiLU gate", dimensions=2)
        beta_logits = self._fp32(beta_logits, "beta logits", dimensions=2)
        alpha_logits = self._fp32(alpha_logits, "alpha logits", dimensions=2)
        dt_bias = self._fp32(dt_bias, "time-step bias", dimensions=1)
        ssm_a = self._fp32(ssm_a, "converted ssm_a", dimensions=1)
        norm_weight = self._fp32(norm_weight, "RMSNorm weight", dimensions=1)
        batch, value_heads, value_width, key_width = _shape(state)
        key_heads = _positive_integer("key_heads", key_heads)
        key_dimension = _positive_integer("key_dimension", key_dimension)
        if key_dimension != key_width:
            raise ValueError("GDN query/key must match state batch and key dimension")
        if value_heads % key_heads:
            raise ValueError("GDN value heads must be a multiple of key heads")
        channels = 2 * key_heads * key_width + value_heads * value_width
        kernel = int(weights.shape[0])
        if _shape(mixed) != (batch, channels) or _shape(weights) != (kernel, channels):
            raise ValueError("convolution weights must match current channels")
        if _shape(history) != (batch, kernel - 1, channels):
            raise ValueError(
                "convolution history must have shape "
                f"{(batch, kernel - 1, channels)}, got {_shape(history)}")
        if _shape(gate) != (batch, value_heads * value_width):
            raise ValueError("recurrent gate must match batch, value heads and width")
        if _shape(beta_logits) != (batch, value_heads) or _shape(alpha_logits) != (batch,
                                                                                 value_heads):
            raise ValueError("GDN beta must match batch and value heads")
        if _shape(dt_bias) != (value_heads,) or _shape(ssm_a) != (value_heads,):
            raise ValueError("time-step bias and ssm_a must match value heads")
        if _shape(norm_weight) != (value_width,):
            raise ValueError("RMSNorm weight must match the input's final dimension")
        if out is not None:
            self._out_buffer(out, (batch, value_heads * value_width),
                             self.torch.float32 if out_dtype is None else out_dtype,
                             "recurrent output")
        return ((mixed, weights, history if kernel > 1 else None, gate, beta_logits,
                 alpha_logits, dt_bias, ssm_a, norm_weight, state),
                dict(key_heads=key_heads, key_dim=key_dimension,
                     eps=_positive_finite("epsilon", epsilon), out_dtype=out_dtype, out=out))

    # ------------------------------------------------------------ paged K/V

    def initialize_paged_attention_workspace(self, *, num_pages: int, page_size: int,
                                             kv_heads: int, key_dimension: int,
                                             value_dimension: int,
                                             dtype: Any = None) -> RocmPagedAttentionWorkspace:
        """A zeroed page pool (extension; the contiguous counterpart is
        ``initialize_attention_workspace``, qwen35_rocm_ops.py:73-86)."""
        pages = _positive_integer("num_pages", num_pages)
        size = _positive_integer("page_size", page_size)
        if size < 32 or size & (size - 1):
            raise ValueError("page_size must be a power of two of at least 32")
        heads = _positive_integer("kv_heads", kv_heads)
        key_width = _positive_integer("key_dimension", key_dimension)
        value_width = _positive_integer("value_dimension", value_dimension)
        dtype = self.torch.float32 if dtype is None else dtype
        keys = self.torch.zeros((pages, size, heads, key_width), dtype=dtype, device=self.device)
        values = self.torch.zeros((pages, size, heads, value_width), dtype=dtype,
                                  device=self.device)
        return RocmPagedAttentionWorkspace(keys, values, size)

    def _paged(self, key_pages, value_pages, block_table):
        key_pages = self._tensor(key_pages, "attention key pages", dimensions=4)
        value_pages = self._tensor(value_pages, "attention value pages", dimensions=4)
        if _shape(key_pages)[:3] != _shape(value_pages)[:3]:
            raise ValueError("attention K/V pages differ in count, size or heads")
        if block_table.dim() != 2 or block_table.dtype != self.torch.int32:
            raise TypeError("block table must be a [batch, max_pages] int32 tensor")
        if block_table.device != key_pages.device or not block_table.is_contiguous():
            raise ValueError("block table must be a contiguous tensor on the cache device")
        self._same_dtype("paged attention", key_pages, value_pages)
        return key_pages, value_pages

    def paged_attention_append_(self, key_pages: Any, value_pages: Any, block_table: Any,
                                position: Any, key: Any, value: Any) -> Any:
        """``attention_append_`` (qwen35_rocm_ops.py:475-500) through a block
        table: ``key [B, Hkv, D]`` / ``value [B, Hkv, Dv]`` of each sequence
        land at logical row ``position`` (an int, or a device int32 ``[B]``
        tensor of per-sequence positions).  Returns ``position + 1``."""
        key_pages, value_pages = self._paged(key_pages, value_pages, block_table)
        key = self._tensor(key, "attention key", dimensions=3)
        value = self._tensor(value, "attention value", dimensions=3)
        batch = int(block_table.shape[0])
        _, size, heads, width = _shape(key_pages)
        if _shape(key) != (batch, heads, width) or _shape(value) != (batch, heads,
                                                                     int(value_pages.shape[3])):
            raise ValueError("attention key/value do not match the page token shape")
        self._same_dtype("paged append", key, value, key_pages)
        if isinstance(position, int):
            position = _nonnegative_integer("attention cache position", position)
            if position >= int(block_table.shape[1]) * size:
                raise ValueError("attention cache position exceeds capacity")
            _ops.kv_append_paged(key_pages, value_pages, block_table, key.unsqueeze(0),
                                 value.unsqueeze(0), position=position)
            return position + 1
        _ops.kv_append_paged(key_pages, value_pages, block_table, key.unsqueeze(0),
                             value.unsqueeze(0), positions=position)
        return position + 1

    def paged_online_attention(self, query: Any, key_pages: Any, value_pages: Any,
                               block_table: Any, *, length: int, seq_lens: Any = None,
                               scale: float | None = None, gate: Any = None,
                               out_dtype: Any = None) -> Any:
        """``online_attention`` (qwen35_rocm_ops.py:502-564) over paged
        caches: query ``[B, Hq, D]`` attends to logical rows
        ``0 .. length - 1`` (or ``seq_lens[b]``) of its sequence's pages.
        Same plan and arithmetic as the contiguous call, so the same rows
        give the same bits.  Returns ``[B, Hq, Dv]``."""
        key_pages, value_pages = self._paged(key_pages, value_pages, block_table)
        query = self._tensor(query, "attention query", dimensions=3)
        length = _positive_integer("attention cache length", length)
        batch, query_heads, width = _shape(query)
        _, size, heads, key_width = _shape(key_pages)
        if int(block_table.shape[0]) != batch:
            raise ValueError("block table batch does not match the query batch")
        if length > int(block_table.shape[1]) * size:
            raise ValueError("attention cache length exceeds capacity")
        if width != key_width:
            raise ValueError("attention query does not match K cache head width")
        if query_heads % heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        self._same_dtype("paged attention", query, key_pages)
        if gate is not None:
            gate = self._tensor(gate, "attention gate", dimensions=3)
            if _shape(gate) != (batch, query_heads, int(value_pages.shape[3])):
                raise ValueError("attention gate must match the output shape")
        scale_value = (1.0 / math.sqrt(key_width) if scale is None
                       else _positive_finite("attention scale", scale))
        return _ops.decode_paged(query, key_pages, value_pages, block_table, length=length,
                                 seq_lens=seq_lens, gate=gate, scale=scale_value,
                                 out_dtype=out_dtype)

    def paged_attention_layer_prefill_(self, query_gate: Any, key: Any, value: Any,
                                       query_norm: Any, key_norm: Any, key_pages: Any,
                                       value_pages: Any, block_table: Any, *, position: int,
                                       sections: Sequence[int], frequency_base: float,
                                       epsilon: float, batch_index: int = 0,
                                       scale: float | None = None) -> tuple[Any, int]:
        """``attention_layer_prefill_`` over a paged pool (extension): the
        ``T`` tokens of sequence ``batch_index`` at logical rows
        ``position .. position + T - 1`` (through ``block_table``), with the
        contiguous chunk's prologue arithmetic and single-tile prefill
        kernel: the same rows give its bits on that kernel (within rounding
        of the paired kernel it may pick).  A table entry outside the pool
        writes no row.  fp16 / bf16 pages with equal key and value widths of
        64, 128 or 256, pages of a power-of-two size >= 64 rows, rotary
        sections summing to a multiple of 32.  Returns ``(gated output
        [T, Hq, D], position + T)``."""
        key_pages, value_pages = self._paged(key_pages, value_pages, block_table)
        num_pages, size, kv_heads, width = _shape(key_pages)
        batch, max_pages = (int(x) for x in block_table.shape)
        if (key_pages.dtype not in (self.torch.float16, self.torch.bfloat16)
                or int(value_pages.shape[3]) != width or width not in (64, 128, 256)):
            raise ValueError("paged attention layer prefill needs fp16/bf16 pages with equal key "
                             "and value widths of 64, 128 or 256")
        if size < 64 or size & (size - 1):
            raise ValueError("paged attention layer prefill needs pages of a power-of-two size "
                             ">= 64 rows")
        query_gate = self._tensor(query_gate, "joint Q/gate projection", dimensions=2)
        key = self._tensor(key, "attention key", dimensions=2)
        value = self._tensor(value, "attention value", dimensions=2)
        query_norm = self._fp32(query_norm, "query RMSNorm weight", dimensions=1)
        key_norm = self._fp32(key_norm, "key RMSNorm weight", dimensions=1)
        position = _nonnegative_integer("attention cache position", position)
        batch_index = _nonnegative_integer("batch_index", batch_index)
        tokens = int(query_gate.shape[0])
        if tokens <= 0:
            raise ValueError("prefill chunk must hold at least one token")
        if batch_index >= batch:
            raise ValueError("batch_index exceeds the block table")
        if position + tokens > max_pages * size:
            raise ValueError("attention cache position exceeds capacity")
        if int(query_gate.shape[1]) % (2 * width):
            raise ValueError("joint Q/gate projection does not match the page head width")
        query_heads = int(query_gate.shape[1]) // (2 * width)
        if query_heads % kv_heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        if _shape(key) != (tokens, kv_heads * width) or _shape(value) != (tokens,
                                                                           kv_heads * width):
            raise ValueError("attention key/value do not match the page token shape")
        if _shape(query_norm) != (width,) or _shape(key_norm) != (width,):
            raise ValueError("RMSNorm weight must match the head dimension")
        self._same_dtype("paged attention prefill", query_gate, key, value, key_pages)
        if len(sections) != 4:
            raise ValueError("IMRoPE requires four sections")
        section = tuple(_nonnegative_integer("IMRoPE section", item) for item in sections)
        if sum(section) % 32 or 2 * sum(section) > width:
            raise ValueError("paged attention layer prefill needs rotary sections summing to a "
                             "multiple of 32, at most half the head width")
        scale_value = (1.0 / math.sqrt(width) if scale is None
                       else _positive_finite("attention scale", scale))
        gated = _ops.attention_layer_prefill_paged(
            query_gate.reshape(tokens, query_heads, 2 * width), key, value, query_norm, key_norm,
            key_pages, value_pages, block_table, batch_index=batch_index, position=position,
            sections=section, frequency_base=_positive_finite("frequency_base", frequency_base),
            eps=_positive_finite("epsilon", epsilon), scale=scale_value)
        return gated, position + tokens

    def paged_attention_layer_step_(self, query_gate: Any, key: Any, value: Any,
                                    query_norm: Any, key_norm: Any, key_pages: Any,
                                    value_pages: Any, block_table: Any, *, position: int,
                                    sections: Sequence[int], frequency_base: float,
                                    epsilon: float, positions: Any = None,
                                    scale: float | None = None,
                                    out_dtype: Any = None) -> tuple[Any, int]:
        """``attention_layer_step_`` over a paged pool (extension): the same
        prologue, two launches and arithmetic, with sequence b's rotated key
        and value written to its logical row ``position`` (or
        ``positions[b]``) through ``block_table`` and attention over its
        rows ``0 .. position``; the same rows give the contiguous step's
        bits.  A table entry outside the pool writes no row.  fp16 / bf16
        pages with equal key and value widths of 64, 128 or 256.  Returns
        ``(gated output [B, Hq, D], position + 1)``."""
        key_pages, value_pages = self._paged(key_pages, value_pages, block_table)
        num_pages, size, kv_heads, width = _shape(key_pages)
        batch, max_pages = (int(x) for x in block_table.shape)
        if (key_pages.dtype not in (self.torch.float16, self.torch.bfloat16)
                or int(value_pages.shape[3]) != width or width not in (64, 128, 256)):
            raise ValueError("paged attention layer step needs fp16/bf16 pages with equal key "
                             "and value widths of 64, 128 or 256")
        query_gate = self._tensor(query_gate, "joint Q/gate projection", dimensions=2)
        key = self._tensor(key, "attention key", dimensions=2)
        value = self._tensor(value, "attention value", dimensions=2)
        query_norm = self._fp32(query_norm, "query RMSNorm weight", dimensions=1)
        key_norm = self._fp32(key_norm, "key RMSNorm weight", dimensions=1)
        position = _nonnegative_integer("attention cache position", position)
        if position >= max_pages * size:
            raise ValueError("attention cache position exceeds capacity")
        if int(query_gate.shape[0]) != batch or int(query_gate.shape[1]) % (2 * width):
            raise ValueError("joint Q/gate projection does not match the page head width")
        query_heads = int(query_gate.shape[1]) // (2 * width)
        if query_heads % kv_heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        if _shape(key) != (batch, kv_heads * width) or _shape(value) != (batch, kv_heads * width):
            raise ValueError("attention key/value do not match the page token shape")
        if _shape(query_norm) != (width,) or _shape(key_norm) != (width,):
            raise ValueError("RMSNorm weight must match the head dimension")
        self._same_dtype("paged attention step", query_gate, key, value, key_pages)
        if len(sections) != 4:
            raise ValueError("IMRoPE requires four sections")
        section = tuple(_nonnegative_integer("IMRoPE section", item) for item in sections)
        base = _positive_finite("frequency_base", frequency_base)
        eps = _positive_finite("epsilon", epsilon)
        if positions is not None:
            if not self.torch.is_tensor(positions) or positions.device.type != "cuda":
                host = [int(p) for p in positions]
                if len(host) != batch or any(p < 0 or p > position for p in host):
                    raise ValueError("positions must hold one row in [0, position] per sequence")
                positions = self.torch.tensor(host, dtype=self.torch.int32, device=self.device)
            elif _shape(positions) != (batch,):
                raise ValueError("positions must hold one row per sequence")
            positions = positions.to(self.torch.int32).contiguous()
        scale_value = (1.0 / math.sqrt(width) if scale is None
                       else _positive_finite("attention scale", scale))
        out = _ops.attention_layer_step_paged(
            query_gate.reshape(batch, query_heads, 2 * width), key, value, query_norm, key_norm,
            key_pages, value_pages, block_table, position=position, sections=section,
            frequency_base=base, eps=eps, positions=positions, scale=scale_value,
            out_dtype=out_dtype)
        return out, position + 1

    def paged_attention_prefill(self, query: Any, key_pages: Any, value_pages: Any,
                                block_table: Any, *, position: int, batch_index: int = 0,
                                scale: float | None = None, gate: Any = None) -> Any:
        """``attention_prefill`` over paged caches (extension): the ``T``
        query tokens ``[T, Hq, D]`` of sequence ``batch_index`` sit at
        logical rows ``position .. position + T - 1`` (already appended) and
        attend causally to rows ``0 ..`` of that sequence's pages.  Same
        kernel and arithmetic as the contiguous call, so the same rows give
        the same bits; output ``[T, Hq, D]`` in the query dtype (times
        sigmoid(gate) with ``gate [T, Hq, D]``).  fp16 / bf16, head width
        64, 128 or 256, page size a power of two >= 64."""
        key_pages, value_pages = self._paged(key_pages, value_pages, block_table)
        query = self._tensor(query, "attention query", dimensions=3)
        position = _nonnegative_integer("attention cache position", position)
        batch_index = _nonnegative_integer("batch_index", batch_index)
        tokens, query_heads, width = _shape(query)
        _, size, heads, key_width = _shape(key_pages)
        if batch_index >= int(block_table.shape[0]):
            raise ValueError("batch_index exceeds the block table batch")
        if tokens <= 0:
            raise ValueError("prefill chunk must hold at least one token")
        if position + tokens > int(block_table.shape[1]) * size:
            raise ValueError("attention cache position exceeds capacity")
        if width != key_width or int(value_pages.shape[3]) != width:
            raise ValueError("attention query does not match the K/V page head width")
        if query_heads % heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        self._same_dtype("paged attention prefill", query, key_pages)
        if gate is not None:
            gate = self._tensor(gate, "sigmoid-gate logits", dimensions=3)
            if _shape(gate) != (tokens, query_heads, width):
                raise ValueError("sigmoid-gate logits must match the attention output")
            self._same_dtype("attention gate", query, gate)
        scale_value = (1.0 / math.sqrt(key_width) if scale is None
                       else _positive_finite("attention scale", scale))
        return _ops.prefill_paged(query, key_pages, value_pages, block_table,
                                  batch_index=batch_index, pos0=position,
                                  kv_tokens=position + tokens, scale=scale_value, gate=gate)

    # ------------------------------------------------------ chunked prefill

    def attention_layer_prefill_(self, query_gate: Any, key: Any, value: Any, query_norm: Any,
                                 key_norm: Any, key_cache: Any, value_cache: Any, *,
                                 position: int, sections: Sequence[int], frequency_base: float,
                                 epsilon: float, batch_index: int = 0,
                                 scale: float | None = None) -> tuple[Any, int]:
        """A prefill chunk of the Qwen3.5 full-attention layer after its
        projections (extension): the reference runs Qwen35Model._attention
        once per token (qwen35_runtime.py:597-665, driven token by token by
        prefill_state, qwen35_runtime.py:777-810); this runs the ``T`` tokens
        of ``query_gate [T, Hq * 2 D]``, ``key [T, Hkv * D]`` and
        ``value [T, Hkv * Dv]`` of cache sequence ``batch_index`` at
        positions ``position .. position + T - 1`` as one fused prologue
        (split, Q/K RMSNorm, IMROPE, cache append) and one causal prefill
        attention over the cache with the sigmoid gate in its epilogue, read in
        place from ``query_gate`` (alpx_attention_layer_prefill).  Where the
        rotary sections sum to a multiple of 32 (Qwen3.5: 32), the prefill
        forms the query heads itself from ``query_gate`` (same bits) and the
        prologue launch writes only the key / value rows.  Returns
        ``(gated output [T, Hq, Dv], position + T)``."""
        key_cache = self._tensor(key_cache, "attention key cache", dimensions=4)
        value_cache = self._tensor(value_cache, "attention value cache", dimensions=4)
        capacity, batch, kv_heads, width = _shape(key_cache)
        value_width = int(value_cache.shape[3])
        query_gate = self._tensor(query_gate, "joint Q/gate projection", dimensions=2)
        key = self._tensor(key, "attention key", dimensions=2)
        value = self._tensor(value, "attention value", dimensions=2)
        query_norm = self._fp32(query_norm, "query RMSNorm weight", dimensions=1)
        key_norm = self._fp32(key_norm, "key RMSNorm weight", dimensions=1)
        position = _nonnegative_integer("attention cache position", position)
        batch_index = _nonnegative_integer("batch_index", batch_index)
        tokens = int(query_gate.shape[0])
        if tokens <= 0:
            raise ValueError("prefill chunk must hold at least one token")
        if batch_index >= batch:
            raise ValueError("batch_index exceeds the cache batch")
        if position + tokens > capacity:
            raise ValueError("attention cache position exceeds capacity")
        if _shape(value_cache)[:3] != (capacity, batch, kv_heads):
            raise ValueError("attention K/V cache capacity, batch, or heads differ")
        if int(query_gate.shape[1]) % (2 * width):
            raise ValueError("joint Q/gate projection does not match the cache head width")
        query_heads = int(query_gate.shape[1]) // (2 * width)
        if query_heads % kv_heads:
            raise ValueError("attention query heads must be a multiple of KV heads")
        if _shape(key) != (tokens, kv_heads * width) or _shape(value) != (tokens,
                                                                           kv_heads * value_width):
            raise ValueError("attention key/value do not match cache token shape")
        if _shape(query_norm) != (width,) or _shape(key_norm) != (width,):
            raise ValueError("RMSNorm weight must match the head dimension")
        self._same_dtype("attention prefill", query_gate, key, value, key_cache, value_cache)
        if len(sections) != 4:
            raise ValueError("IMRoPE requires four sections")
        section = tuple(_nonnegative_integer("IMRoPE section", item) for item in sections)
        if value_width != width:
            raise ValueError("sigmoid gate must match values")
        scale_value = (1.0 / math.sqrt(width) if scale is None
                       else _positive_finite("attention scale", scale))
        gated = _ops.attention_layer_prefill(
            query_gate.reshape(tokens, query_heads, 2 * width), key, value, query_norm,
            key_norm, key_cache, value_cache, batch_index=batch_index, position=position,
            sections=section, frequency_base=_positive_finite("frequency_base", frequency_base),
            eps=_positive_finite("epsilon", epsilon), scale=scale_value)
        return gated, position + tokens

    def recurrent_layer_prefill_(self, workspace: RocmRecurrentWorkspace, mixed: Any,
                                 convolution_weights: Any, gate: Any, beta_logits: Any,
                                 alpha_logits: Any, dt_bias: Any, ssm_a: Any, norm_weight: Any,
                                 *, key_heads: int, key_dimension: int, epsilon: float,
                                 batch_index: int = 0, out_dtype: Any = None,
                                 operand_dtype: Any = None) -> Any:
        """A prefill chunk of the Qwen3.5 recurrent (GDN) layer after its
        projections (extension): the reference runs the per-token chain of
        qwen35_numpy.py:63-131 / Qwen35Model._recurrent once per token
        (qwen35_runtime.py:777-810); this runs the ``T`` tokens of
        ``mixed [T, 2 Hk Dk + Hv Dv]``, ``gate [T, Hv * Dv]`` and the logits
        ``[T, Hv]`` of workspace sequence ``batch_index`` as one convolution
        prep (conv + SiLU over the chunk, split, Q/K L2 norm, beta / decay,
        history moved on), the chunked GDN on the sequence's delta state and
        one gated RMSNorm.  The chain is fp32 like the reference's: q / k / v
        stay fp32 and the chunked GDN (key_dimension 64 / 128 / 256, value
        width a multiple of 16; token by token otherwise) splits them into
        hi + lo bf16 MFMA operands, which keeps output and state within 1e-4
        of the fp64 token chain.  ``operand_dtype=torch.bfloat16`` (opt-in)
        rounds q / k / v to bf16 instead (fewer MFMAs), with the state within
        about 2e-3 and the output within 2e-2 of the fp32 chain.
        Returns ``[T, Hv * Dv]``."""
        torch = self.torch
        history = self._fp32(workspace.convolution_history, "convolution history",
                             dimensions=3)
        state = self._fp32(workspace.delta_state, "GDN state", dimensions=4)
        mixed = self._fp32(mixed, "convolution current", dimensions=2)
        weights = self._fp32(convolution_weights, "convolution weights", dimensions=2)
        gate = self._fp32(gate, "recurrent SiLU gate", dimensions=2)
        beta_logits = self._fp32(beta_logits, "beta logits", dimensions=2)
        alpha_logits = self._fp32(alpha_logits, "alpha logits", dimensions=2)
        dt_bias = self._fp32(dt_bias, "time-step bias", dimensions=1)
        ssm_a = self._fp32(ssm_a, "converted ssm_a", dimensions=1)
        norm_weight = self._fp32(norm_weight, "RMSNorm weight", dimensions=1)
        batch, value_heads, value_width, key_width = _shape(state)
        key_heads = _positive_integer("key_heads", key_heads)
        key_dimension = _positive_integer("key_dimension", key_dimension)
        batch_index = _nonnegative_integer("batch_index", batch_index)
        if batch_index >= batch:
            raise ValueError("batch_index exceeds the workspace batch")
        if key_dimension != key_width:
            raise ValueError("GDN query/key must match state batch and key dimension")
        if value_heads % key_heads:
            raise ValueError("GDN value heads must be a multiple of key heads")
        channels = 2 * key_heads * key_width + value_heads * value_width
        kernel = int(weights.shape[0])
        tokens = int(mixed.shape[0])
        if tokens <= 0:
            raise ValueError("prefill chunk must hold at least one token")
        if _shape(mixed) != (tokens, channels) or _shape(weights) != (kernel, channels):
            raise ValueError("convolution weights must match current channels")
        if _shape(history) != (batch, kernel - 1, channels):
            raise ValueError(
                "convolution history must have shape "
                f"{(batch, kernel - 1, channels)}, got {_shape(history)}")
        if _shape(gate) != (tokens, value_heads * value_width):
            raise ValueError("recurrent gate must match tokens, value heads and width")
        if _shape(beta_logits) != (tokens, value_heads) or _shape(alpha_logits) != (tokens,
                                                                                  value_heads):
            raise ValueError("GDN beta must match tokens and value heads")
        if _shape(dt_bias) != (value_heads,) or _shape(ssm_a) != (value_heads,):
            raise ValueError("time-step bias and ssm_a must match value heads")
        if _shape(norm_weight) != (value_width,):
            raise ValueError("RMSNorm weight must match the input's final dimension")
        eps = _positive_finite("epsilon", epsilon)
        if operand_dtype not in (None, torch.float32, torch.bfloat16):
            raise TypeError("operand_dtype must be torch.float32 or torch.bfloat16")
        mfma = key_width in (64, 128, 256) and value_width % 16 == 0
        qkv_dtype = (torch.bfloat16 if mfma and operand_dtype == torch.bfloat16
                     else torch.float32)
        q, k, v, beta, g = _ops.recurrent_prefill_prep(
            mixed, weights, history[batch_index] if kernel > 1 else None, beta_logits,
            alpha_logits, dt_bias, ssm_a, key_heads=key_heads, key_dim=key_width,
            value_heads=value_heads, value_dim=value_width, eps=eps, qkv_dtype=qkv_dtype)
        seq_state = state[batch_index:batch_index + 1]
        attended = _ops.gdn_chunk(seq_state, q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                                  beta.unsqueeze(0), g.unsqueeze(0), out_dtype=torch.float32)
        return _ops.row_norm(attended.reshape(tokens * value_heads, value_width),
                             mode=_lib.NORM_RMS_GATE, eps=eps, weight=norm_weight,
                             gate=gate, out_dtype=torch.float32 if out_dtype is None
                             else out_dtype).reshape(tokens, value_heads * value_width)


__all__ = [
    "Qwen35RocmOps",
    "RocmPagedAttentionWorkspace",
    "Qwen35RocmUnavailable",
    "RocmAttentionWorkspace",
    "RocmCapability",
    "RocmRecurrentWorkspace",
    "rocm_capability",
]
