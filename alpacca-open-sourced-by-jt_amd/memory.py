"""Device-resident layer state with the reference's state-transfer contract.

Counterparts of ``alpaccaroo.memory`` (memory.py:223-290, 385-585) for state
that lives in device buffers:

* ``DeviceFullAttentionState`` keeps one attention layer's K/V rows in a
  preallocated ``[capacity, batch, kv_heads, dim]`` cache (fp32, or fp16 /
  bf16 as the reference's half-precision device mirror, cuda.py:1729-1738)
  for one sequence, with the logical length on the host, as
  ``FullAttentionState`` keeps them in host arrays.
* ``DevicePagedAttentionState`` is the same for one sequence of a paged
  pool (pages + block table; an extension), with the same records.
* ``DeviceRecurrentState`` views one sequence of a ``RocmRecurrentWorkspace``
  (convolution history and delta matrix, fp32) as ``RecurrentState``.

``snapshot()`` returns the reference's own record types with the same
fields and the same ``"f32-le"`` bytes (row-major float32, little endian),
so a snapshot taken here restores into the reference's host state and back;
``restore()`` validates a record as the reference does
(``_validate_layer_snapshot``, memory.py:640-720) before writing it.  The
attention rows move through ``alpx_kv_export`` / ``alpx_kv_import`` (widen /
round-to-nearest-even on the device); the recurrent buffers are fp32 in
both places and move as plain copies.  ``truncate`` follows the reference:
attention drops rows (the device rows past the length are never read
again), recurrent state cannot be truncated without a replay.
"""

from __future__ import annotations

import sys
from dataclasses import dataclass
from typing import Any

from . import _ops


class StateError(RuntimeError):
    """Invalid state operation (memory.StateError)."""


class ReplayRequiredError(StateError):
    """A recurrent state operation needs checkpoint restore plus replay."""


class SnapshotMismatchError(StateError):
    """A snapshot record does not match the state it is restored into."""


def _strict_nonnegative(name: str, value: int) -> None:
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise StateError(f"{name} must be a non-negative integer, got {value!r}")


@dataclass(frozen=True, slots=True)
class FullAttentionSnapshot:
    """memory.FullAttentionSnapshot (memory.py:223-241)."""

    layer_index: int
    logical_length: int
    kv_heads: int
    key_dim: int
    value_dim: int
    key: bytes
    value: bytes
    dtype: str = "f32-le"
    kind: str = "attention"

    def __post_init__(self) -> None:
        object.__setattr__(self, "key", bytes(self.key))
        object.__setattr__(self, "value", bytes(self.value))

    def memory_bytes(self) -> int:
        return len(self.key) + len(self.value)


@dataclass(frozen=True, slots=True)
class RecurrentSnapshot:
    """memory.RecurrentSnapshot (memory.py:244-264)."""

    layer_index: int
    logical_position: int
    conv_channels: int
    conv_kernel: int
    recurrent_key_heads: int
    recurrent_value_heads: int
    recurrent_key_dim: int
    recurrent_value_dim: int
    conv_history: bytes
    delta_matrix: bytes
    dtype: str = "f32-le"
    kind: str = "recurrent"

    def __post_init__(self) -> None:
        object.__setattr__(self, "conv_history", bytes(self.conv_history))
        object.__setattr__(self, "delta_matrix", bytes(self.delta_matrix))

    def memory_bytes(self) -> int:
        return len(self.conv_history) + len(self.delta_matrix)


def _le_bytes(t) -> bytes:
    """Host bytes of an fp32 device tensor, little endian (the record's
    "f32-le" encoding; _f32_to_bytes, memory.py:71-78)."""
    host = t.detach().contiguous().cpu().numpy()
    if sys.byteorder != "little":
        host = host.byteswap()
    return host.tobytes()


def _from_le_bytes(torch, data: bytes, count: int, what: str, device):
    """fp32 device tensor from "f32-le" bytes, with the reference's checks
    (_validate_f32_bytes / _f32_from_bytes)."""
    import numpy as np
    if not isinstance(data, (bytes, bytearray, memoryview)):
        raise SnapshotMismatchError(f"{what} must be bytes")
    if len(data) != 4 * count:
        raise SnapshotMismatchError(f"{what} has {len(data)} bytes, expected {4 * count}")
    host = np.frombuffer(bytes(data), dtype="<f4").astype(np.float32)
    return torch.from_numpy(host.copy()).to(device)


class DeviceFullAttentionState:
    """One attention layer's K/V rows for sequence ``batch_index`` of a device
    cache ``[capacity, batch, kv_heads, key_dim|value_dim]`` (memory.
    FullAttentionState, memory.py:385-475).  The logical length is host-side;
    rows past it are dead (never read by the attention kernels)."""

    __slots__ = ("key_cache", "value_cache", "layer_index", "batch_index", "logical_length")

    def __init__(self, key_cache: Any, value_cache: Any, *, layer_index: int = 0,
                 batch_index: int = 0, logical_length: int = 0) -> None:
        _strict_nonnegative("logical_length", logical_length)
        _strict_nonnegative("batch_index", batch_index)
        if key_cache.dim() != 4 or value_cache.dim() != 4:
            raise StateError("attention caches must be [capacity, batch, kv_heads, dim]")
        if tuple(key_cache.shape[:3]) != tuple(value_cache.shape[:3]):
            raise StateError("attention K/V cache capacity, batch, or heads differ")
        if key_cache.dtype != value_cache.dtype:
            raise StateError("attention K/V caches must share a dtype")
        if not (key_cache.is_contiguous() and value_cache.is_contiguous()):
            raise StateError("attention caches must be contiguous")
        if batch_index >= int(key_cache.shape[1]):
            raise StateError("batch_index exceeds the cache batch")
        if logical_length > int(key_cache.shape[0]):
            raise StateError("logical_length exceeds the cache capacity")
        self.key_cache = key_cache
        self.value_cache = value_cache
        self.layer_index = layer_index
        self.batch_index = batch_index
        self.logical_length = logical_length

    @property
    def capacity(self) -> int:
        return int(self.key_cache.shape[0])

    @property
    def kv_heads(self) -> int:
        return int(self.key_cache.shape[2])

    @property
    def key_dim(self) -> int:
        return int(self.key_cache.shape[3])

    @property
    def value_dim(self) -> int:
        return int(self.value_cache.shape[3])

    def append(self, key: Any, value: Any) -> None:
        """Append one token's rows ``key [kv_heads * key_dim]`` and
        ``value [kv_heads * value_dim]`` (cache dtype) at the logical length
        (bit-exact copy; FullAttentionState.append, memory.py:419-428)."""
        import torch
        if self.logical_length >= self.capacity:
            raise StateError("attention cache capacity exhausted")
        if key.numel() != self.kv_heads * self.key_dim or (
                value.numel() != self.kv_heads * self.value_dim):
            raise StateError("attention rows must hold kv_heads * dim values")
        if key.dtype != self.key_cache.dtype or value.dtype != self.value_cache.dtype:
            raise StateError("attention rows must use the cache dtype")
        # one row per cache sequence; only this sequence's has a position in
        # the cache (the others are skipped by the append kernel)
        batch = int(self.key_cache.shape[1])
        pos = torch.full((batch,), -1, dtype=torch.int32, device=self.key_cache.device)
        pos[self.batch_index] = self.logical_length
        rows_k = self.key_cache.new_zeros((1, batch, self.kv_heads, self.key_dim))
        rows_v = self.value_cache.new_zeros((1, batch, self.kv_heads, self.value_dim))
        rows_k[0, self.batch_index] = key.reshape(self.kv_heads, self.key_dim)
        rows_v[0, self.batch_index] = value.reshape(self.kv_heads, self.value_dim)
        _ops.kv_append(self.key_cache, self.value_cache, rows_k, rows_v, positions=pos)
        self.logical_length += 1

    def reset(self) -> None:
        self.logical_length = 0

    def truncate(self, position: int) -> None:
        """Drop rows at and past ``position`` (FullAttentionState.truncate,
        memory.py:435-443)."""
        _strict_nonnegative("position", position)
        if position > self.logical_length:
            raise StateError(
                f"cannot extend attention state from {self.logical_length} to {position}")
        self.logical_length = position

    def snapshot(self) -> FullAttentionSnapshot:
        """The reference's record of this state (memory.py:451-460): fp32
        rows [logical_length, kv_heads, dim], little-endian bytes."""
        k, v = _ops.kv_export(self.key_cache, self.value_cache, batch_index=self.batch_index,
                              row0=0, rows=self.logical_length)
        return FullAttentionSnapshot(
            layer_index=self.layer_index, logical_length=self.logical_length,
            kv_heads=self.kv_heads, key_dim=self.key_dim, value_dim=self.value_dim,
            key=_le_bytes(k), value=_le_bytes(v))

    def restore(self, snapshot: FullAttentionSnapshot) -> None:
        """Validate a record as _validate_layer_snapshot does
        (memory.py:640-690) and write its rows into the cache (rounded to
        the cache dtype)."""
        length, k, v = _attention_record_rows(self, snapshot)
        _ops.kv_import(k, v, self.key_cache, self.value_cache, batch_index=self.batch_index,
                       row0=0)
        self.logical_length = length

    def memory_bytes(self) -> int:
        es = self.key_cache.element_size()
        return self.logical_length * self.kv_heads * (self.key_dim + self.value_dim) * es

    def describe(self) -> dict[str, Any]:
        return {
            "kind": "attention", "layer_index": self.layer_index,
            "logical_length": self.logical_length,
            "dtype": str(self.key_cache.dtype).replace("torch.", ""),
            "key_shape": [self.logical_length, self.kv_heads, self.key_dim],
            "value_shape": [self.logical_length, self.kv_heads, self.value_dim],
            "memory_bytes": self.memory_bytes(),
        }


def _attention_record_rows(state, snapshot):
    """Checks of an attention record against ``state`` (kind, layer, dtype,
    shape, capacity; _validate_layer_snapshot, memory.py:640-690) and its
    rows as fp32 device tensors ``(length, key [L, Hkv, D], value [L, Hkv, Dv])``."""
    import torch
    if getattr(snapshot, "kind", None) != "attention":
        raise SnapshotMismatchError("snapshot record is not an attention record")
    if getattr(snapshot, "layer_index", None) != state.layer_index:
        raise SnapshotMismatchError(f"snapshot layer index mismatch at layer {state.layer_index}")
    if snapshot.dtype != "f32-le":
        raise SnapshotMismatchError(f"snapshot has unsupported dtype {snapshot.dtype!r}")
    length = snapshot.logical_length
    _strict_nonnegative("logical_length", length)
    if (snapshot.kv_heads, snapshot.key_dim, snapshot.value_dim) != (
            state.kv_heads, state.key_dim, state.value_dim):
        raise SnapshotMismatchError("snapshot attention shape differs")
    if length > state.capacity:
        raise SnapshotMismatchError("snapshot length exceeds the cache capacity")
    dev = state.key_cache.device
    k = _from_le_bytes(torch, snapshot.key, length * state.kv_heads * state.key_dim,
                       "snapshot key", dev)
    v = _from_le_bytes(torch, snapshot.value, length * state.kv_heads * state.value_dim,
                       "snapshot value", dev)
    return (length, k.reshape(length, state.kv_heads, state.key_dim),
            v.reshape(length, state.kv_heads, state.value_dim))


class DevicePagedAttentionState(DeviceFullAttentionState):
    """``DeviceFullAttentionState`` for sequence ``batch_index`` of a paged
    pool (extension): pages ``[num_pages, page_size, kv_heads, dim]`` held in
    ``key_cache`` / ``value_cache`` and the pool's ``block_table [batch,
    max_pages]`` (device int32); logical row j lives at row j % page_size of
    page ``block_table[batch_index][j // page_size]``.  The capacity is
    ``max_pages * page_size``.  Appends, snapshots and restores move rows
    through the table (``alpx_kv_append_paged``, ``alpx_kv_export_paged`` /
    ``alpx_kv_import_paged``), with the same record bytes as the contiguous
    state."""

    __slots__ = ("block_table",)

    def __init__(self, key_pages: Any, value_pages: Any, block_table: Any, *,
                 layer_index: int = 0, batch_index: int = 0, logical_length: int = 0) -> None:
        import torch
        _strict_nonnegative("logical_length", logical_length)
        _strict_nonnegative("batch_index", batch_index)
        if key_pages.dim() != 4 or value_pages.dim() != 4:
            raise StateError("attention pages must be [num_pages, page_size, kv_heads, dim]")
        if tuple(key_pages.shape[:3]) != tuple(value_pages.shape[:3]):
            raise StateError("attention K/V pages differ in count, size or heads")
        if key_pages.dtype != value_pages.dtype:
            raise StateError("attention K/V pages must share a dtype")
        if not (key_pages.is_contiguous() and value_pages.is_contiguous()):
            raise StateError("attention pages must be contiguous")
        if (block_table.dim() != 2 or block_table.dtype != torch.int32
                or not block_table.is_contiguous() or block_table.device != key_pages.device):
            raise StateError("block table must be a contiguous [batch, max_pages] int32 tensor "
                             "on the pages' device")
        size = int(key_pages.shape[1])
        if size <= 0 or size & (size - 1):
            raise StateError("page size must be a power of two")
        if batch_index >= int(block_table.shape[0]):
            raise StateError("batch_index exceeds the block table batch")
        if logical_length > int(block_table.shape[1]) * size:
            raise StateError("logical_length exceeds the cache capacity")
        self.key_cache = key_pages
        self.value_cache = value_pages
        self.block_table = block_table
        self.layer_index = layer_index
        self.batch_index = batch_index
        self.logical_length = logical_length

    @property
    def capacity(self) -> int:
        return int(self.block_table.shape[1]) * int(self.key_cache.shape[1])

    def append(self, key: Any, value: Any) -> None:
        """Append one token's rows at the logical length through the block
        table (bit-exact copy; FullAttentionState.append, memory.py:419-428)."""
        import torch
        if self.logical_length >= self.capacity:
            raise StateError("attention cache capacity exhausted")
        if key.numel() != self.kv_heads * self.key_dim or (
                value.numel() != self.kv_heads * self.value_dim):
            raise StateError("attention rows must hold kv_heads * dim values")
        if key.dtype != self.key_cache.dtype or value.dtype != self.value_cache.dtype:
            raise StateError("attention rows must use the cache dtype")
        batch = int(self.block_table.shape[0])
        pos = torch.full((batch,), -1, dtype=torch.int32, device=self.key_cache.device)
        pos[self.batch_index] = self.logical_length
        rows_k = self.key_cache.new_zeros((1, batch, self.kv_heads, self.key_dim))
        rows_v = self.value_cache.new_zeros((1, batch, self.kv_heads, self.value_dim))
        rows_k[0, self.batch_index] = key.reshape(self.kv_heads, self.key_dim)
        rows_v[0, self.batch_index] = value.reshape(self.kv_heads, self.value_dim)
        _ops.kv_append_paged(self.key_cache, self.value_cache, self.block_table, rows_k, rows_v,
                             positions=pos)
        self.logical_length += 1

    def snapshot(self) -> FullAttentionSnapshot:
        """The reference's record of this state (memory.py:451-460)."""
        k, v = _ops.kv_export_paged(self.key_cache, self.value_cache, self.block_table,
                                    batch_index=self.batch_index, row0=0,
                                    rows=self.logical_length)
        return FullAttentionSnapshot(
            layer_index=self.layer_index, logical_length=self.logical_length,
            kv_heads=self.kv_heads, key_dim=self.key_dim, value_dim=self.value_dim,
            key=_le_bytes(k), value=_le_bytes(v))

    def restore(self, snapshot: FullAttentionSnapshot) -> None:
        """Validate a record (memory.py:640-690) and write its rows into the
        sequence's pages (rounded to the page dtype)."""
        length, k, v = _attention_record_rows(self, snapshot)
        _ops.kv_import_paged(k, v, self.key_cache, self.value_cache, self.block_table,
                             batch_index=self.batch_index, row0=0)
        self.logical_length = length


class DeviceRecurrentState:
    """One recurrent layer's convolution history ``[K-1, C]`` and delta
    matrix ``[Hv, Dv, Dk]`` (fp32) for sequence ``batch_index`` of a
    ``RocmRecurrentWorkspace`` (memory.RecurrentState, memory.py:478-585)."""

    __slots__ = ("workspace", "layer_index", "batch_index", "logical_position", "key_heads")

    def __init__(self, workspace: Any, *, key_heads: int, layer_index: int = 0,
                 batch_index: int = 0, logical_position: int = 0) -> None:
        _strict_nonnegative("logical_position", logical_position)
        _strict_nonnegative("batch_index", batch_index)
        if batch_index >= int(workspace.delta_state.shape[0]):
            raise StateError("batch_index exceeds the workspace batch")
        self.workspace = workspace
        self.key_heads = int(key_heads)
        self.layer_index = layer_index
        self.batch_index = batch_index
        self.logical_position = logical_position

    @property
    def conv_history(self) -> Any:
        return self.workspace.convolution_history[self.batch_index]

    @property
    def delta_matrix(self) -> Any:
        return self.workspace.delta_state[self.batch_index]

    def advance(self) -> None:
        """One token consumed by the device kernels (RecurrentState.advance,
        memory.py:520-533, whose buffers the kernels update in place)."""
        self.logical_position += 1

    def reset(self) -> None:
        self.conv_history.zero_()
        self.delta_matrix.zero_()
        self.logical_position = 0

    def truncate(self, position: int) -> None:
        """RecurrentState.truncate (memory.py:539-545): only the live
        position is allowed; anything else needs restore + replay."""
        _strict_nonnegative("position", position)
        if position != self.logical_position:
            raise ReplayRequiredError(
                "recurrent state cannot be truncated by changing its logical "
                "position; restore a complete checkpoint and replay")

    def snapshot(self) -> RecurrentSnapshot:
        hist, delta = self.conv_history, self.delta_matrix
        hv, dv, dk = (int(x) for x in delta.shape)
        return RecurrentSnapshot(
            layer_index=self.layer_index, logical_position=self.logical_position,
            conv_channels=int(hist.shape[1]), conv_kernel=int(hist.shape[0]) + 1,
            recurrent_key_heads=self.key_heads, recurrent_value_heads=hv,
            recurrent_key_dim=dk, recurrent_value_dim=dv,
            conv_history=_le_bytes(hist), delta_matrix=_le_bytes(delta))

    def restore(self, snapshot: RecurrentSnapshot) -> None:
        import torch
        if getattr(snapshot, "kind", None) != "recurrent":
            raise SnapshotMismatchError("snapshot record is not a recurrent record")
        if getattr(snapshot, "layer_index", None) != self.layer_index:
            raise SnapshotMismatchError(f"snapshot layer index mismatch at layer {self.layer_index}")
        if snapshot.dtype != "f32-le":
            raise SnapshotMismatchError(f"snapshot has unsupported dtype {snapshot.dtype!r}")
        hist, delta = self.conv_history, self.delta_matrix
        hv, dv, dk = (int(x) for x in delta.shape)
        expected = (int(hist.shape[1]), int(hist.shape[0]) + 1, self.key_heads, hv, dk, dv)
        actual = (snapshot.conv_channels, snapshot.conv_kernel, snapshot.recurrent_key_heads,
                  snapshot.recurrent_value_heads, snapshot.recurrent_key_dim,
                  snapshot.recurrent_value_dim)
        if actual != expected:
            raise SnapshotMismatchError("snapshot recurrent shape differs")
        _strict_nonnegative("logical_position", snapshot.logical_position)
        dev = delta.device
        h = _from_le_bytes(torch, snapshot.conv_history, hist.numel(), "snapshot conv history",
                           dev)
        d = _from_le_bytes(torch, snapshot.delta_matrix, delta.numel(), "snapshot delta matrix",
                           dev)
        hist.copy_(h.reshape(hist.shape))
        delta.copy_(d.reshape(delta.shape))
        self.logical_position = snapshot.logical_position

    def memory_bytes(self) -> int:
        return (self.conv_history.numel() + self.delta_matrix.numel()) * 4


__all__ = [
    "DeviceFullAttentionState",
    "DevicePagedAttentionState",
    "DeviceRecurrentState",
    "FullAttentionSnapshot",
    "RecurrentSnapshot",
    "ReplayRequiredError",
    "SnapshotMismatchError",
    "StateError",
]
