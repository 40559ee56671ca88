"""ctypes binding of libalpx.so (the gfx950 attention library).

The library is built in-tree by ``csrc/Makefile`` (``__graft_entry__.build``)
and loaded from this directory.  There is no fallback: if the library or a
gfx950 device is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# ALPX_LIBRARY overrides the in-tree build (e.g. to compare two builds).
LIB_PATH = os.environ.get("ALPX_LIBRARY") or os.path.join(_HERE, "libalpx.so")
ABI_VERSION = 1

F32, F16, BF16 = 0, 1, 2
OK, EINVAL, EUNSUPPORTED, EHIP, ERANGE = 0, -1, -2, -3, -4

_c_int, _c_i64, _c_ptr, _c_size = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
_c_float = ctypes.c_float

# name -> (restype, argtypes); mirrors include/alpx.h
SIGNATURES = {
    "alpx_abi_version": (_c_int, []),
    "alpx_last_error": (ctypes.c_char_p, []),
    "alpx_device_arch": (_c_int, [_c_int, ctypes.c_char_p, _c_int]),
    "alpx_host_device_pointer": (_c_int, [_c_ptr, ctypes.POINTER(_c_ptr)]),
    "alpx_kv_append": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_int, _c_int,
                                _c_int, _c_int, _c_int, _c_i64, _c_ptr, _c_ptr]),
    "alpx_kv_append_paged": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int,
                                      _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                      _c_i64, _c_ptr, _c_ptr]),
    "alpx_decode_gqa_paged": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int,
                                       _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_int,
                                       _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int,
                                       _c_ptr]),
    "alpx_kv_export": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_int, _c_int,
                                _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_ptr]),
    "alpx_kv_import": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_int, _c_int,
                                _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_ptr]),
    # pages, pages, block_table, batch, max_pages, page_size, num_pages, rows, rows, dtype,
    # kv_heads, key_dim, value_dim, batch_index, row0, rows, stream
    "alpx_kv_export_paged": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_int,
                                      _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_int, _c_int,
                                      _c_i64, _c_i64, _c_ptr]),
    # rows, rows, pages, pages, block_table, batch, max_pages, page_size, num_pages, dtype,
    # kv_heads, key_dim, value_dim, batch_index, row0, rows, stream
    "alpx_kv_import_paged": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int,
                                      _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                      _c_i64, _c_i64, _c_ptr]),
    "alpx_decode_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "alpx_decode_gqa": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr,
                                 _c_ptr, _c_size, _c_int, _c_int, _c_int, _c_int, _c_int,
                                 _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_float,
                                 _c_int, _c_int, _c_ptr]),
    "alpx_decode_gqa_noalloc": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr,
                                         _c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64,
                                         _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_int,
                                         _c_int, _c_ptr]),
    "alpx_sigmoid_gate": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_int, _c_int, _c_ptr]),
    "alpx_prefill_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "alpx_prefill_causal": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_int,
                                     _c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64,
                                     _c_i64, _c_int, _c_i64, _c_float, _c_int, _c_int, _c_ptr]),
    "alpx_prefill_causal_gated": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                           _c_size, _c_int, _c_int, _c_int, _c_int, _c_int,
                                           _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_i64,
                                           _c_float, _c_int, _c_int, _c_ptr]),
    "alpx_prefill_append": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                     _c_ptr, _c_size, _c_int, _c_i64, _c_int, _c_int, _c_int,
                                     _c_int, _c_i64, _c_int, _c_float, _c_int, _c_int, _c_ptr]),
    "alpx_attention_layer_prefill": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                              _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_int,
                                              _c_int, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                              _c_int, _c_int, _c_i64,
                                              ctypes.POINTER(ctypes.c_int), ctypes.c_double,
                                              _c_float, _c_float, _c_ptr]),
    "alpx_attention_layer_prefill_paged": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                                    _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int,
                                                    _c_int, _c_int, _c_ptr, _c_ptr, _c_size,
                                                    _c_int, _c_int, _c_int, _c_int, _c_int,
                                                    _c_i64, ctypes.POINTER(ctypes.c_int),
                                                    ctypes.c_double, _c_float, _c_float, _c_ptr]),
    "alpx_gdn_step": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int,
                               _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_ptr]),
    "alpx_gdn_chunk_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "alpx_gdn_chunk_uses_mfma": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "alpx_gdn_chunk_prefill": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                        _c_ptr, _c_size, _c_int, _c_int, _c_int, _c_int, _c_int,
                                        _c_int, _c_int, _c_int, _c_ptr]),
    "alpx_silu": (_c_int, [_c_ptr, _c_ptr, _c_i64, _c_int, _c_int, _c_ptr]),
    "alpx_row_norm": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_int, _c_i64, _c_i64,
                               _c_float, _c_int, _c_int, _c_int, _c_ptr]),
    "alpx_conv_step": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_i64,
                                _c_i64, _c_int, _c_int, _c_ptr]),
    "alpx_recurrent_parameters": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                           _c_i64, _c_int, _c_ptr]),
    "alpx_imrope": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_int, _c_int,
                             ctypes.POINTER(ctypes.c_int), ctypes.c_double, ctypes.c_double,
                             _c_int, _c_int, _c_ptr]),
    "alpx_attention_prologue": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                         _c_ptr, _c_ptr, _c_int, _c_i64, _c_int, _c_int, _c_int,
                                         _c_int, _c_int, _c_i64, _c_ptr,
                                         ctypes.POINTER(ctypes.c_int), ctypes.c_double,
                                         _c_float, _c_ptr]),
    "alpx_prefill_causal_paged": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int,
                                           _c_int, _c_int, _c_ptr, _c_ptr, _c_int, _c_int,
                                           _c_int, _c_int, _c_int, _c_i64, _c_int, _c_i64,
                                           _c_float, _c_int, _c_ptr]),
    "alpx_attention_layer_step": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                           _c_ptr, _c_ptr, _c_ptr, _c_size, _c_int, _c_int,
                                           _c_i64, _c_int, _c_int, _c_int, _c_int, _c_i64,
                                           _c_ptr, ctypes.POINTER(ctypes.c_int),
                                           ctypes.c_double, _c_float, _c_float, _c_ptr]),
    # query_gate, key, value, q_norm, k_norm, key_pages, value_pages, block_table,
    # max_pages, page_size, num_pages, out, workspace, workspace_bytes, dtype,
    # out_dtype, batch, q_heads, kv_heads, head_dim, position, positions,
    # sections, frequency_base, eps, scale, stream
    "alpx_attention_layer_step_paged": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                                 _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_ptr,
                                                 _c_ptr, _c_size, _c_int, _c_int, _c_int, _c_int,
                                                 _c_int, _c_int, _c_i64, _c_ptr,
                                                 ctypes.POINTER(ctypes.c_int), ctypes.c_double,
                                                 _c_float, _c_float, _c_ptr]),
    "alpx_attention_prologue_chunk": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                               _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_int,
                                               _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                               _c_i64, ctypes.POINTER(ctypes.c_int),
                                               ctypes.c_double, _c_float, _c_ptr]),
    "alpx_recurrent_prefill_prep": (_c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_int,
                                             _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                             _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int,
                                             _c_int, _c_int, _c_float, _c_int, _c_ptr]),
    "alpx_recurrent_step_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "alpx_recurrent_step": (_c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_int, _c_ptr,
                                     _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                     _c_ptr, _c_size, _c_int, _c_int, _c_int, _c_int, _c_int,
                                     _c_float, _c_int, _c_ptr]),
    "alpx_set_override": (_c_int, [_c_int, _c_int]),
    "alpx_get_override": (_c_int, [_c_int]),
    "alpx_timing_enable": (_c_int, [_c_int]),
    "alpx_timing_read": (_c_int, [_c_int, ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_int64)]),
}

# alpx_timed_kernel ids
(T_KV_APPEND, T_DECODE, T_DECODE_COMBINE, T_PREFILL, T_GDN_CHUNK, T_GDN_STEP, T_AUX, T_LAYER,
 T_RECURRENT_STEP) = range(9)

# alpx_row_norm modes
NORM_L2, NORM_RMS, NORM_RMS_GATE = 0, 1, 2

# alpx_override ids and the ALPX_OVERRIDE_PREFILL_KERNEL values
(OVERRIDE_DECODE_GENERIC, OVERRIDE_PREFILL_GENERIC, OVERRIDE_PREFILL_KERNEL,
 OVERRIDE_GDN_SEQUENTIAL, OVERRIDE_RECURRENT_UNFUSED) = range(5)
PREFILL_KERNELS = {"auto": 0, "single": 1, "pair": 2, "shared": 3}


def set_override(which: int, value: int) -> int:
    """Sets a kernel-choice override of the library (tests and A/B timing;
    the library reads the environment only once, at load) and returns the
    previous value."""
    previous = lib().alpx_set_override(int(which), int(value))
    if previous < 0:
        check(previous)
    return previous


def get_override(which: int) -> int:
    value = lib().alpx_get_override(int(which))
    if value < 0:
        check(value)
    return value


def timing_enable(on: bool) -> None:
    check(lib().alpx_timing_enable(1 if on else 0))


def timing_read(kernel: int) -> tuple[float, int]:
    """(summed milliseconds, launches) recorded for ``kernel`` since enable."""
    total = ctypes.c_double()
    count = ctypes.c_int64()
    check(lib().alpx_timing_read(int(kernel), ctypes.byref(total), ctypes.byref(count)))
    return total.value, count.value


class AlpxUnavailable(RuntimeError):
    """The library is not built, fails to load, or no gfx950 device exists."""


class AlpxError(RuntimeError):
    """A HIP runtime failure reported by the library."""

    def __init__(self, message: str, status: int) -> None:
        super().__init__(message)
        self.status = status


class AlpxUnsupported(ValueError):
    """Shape/dtype outside what the kernels cover (status ALPX_EUNSUPPORTED)."""


_lib = None


def lib():
    """Load libalpx.so once, bind every signature and check the ABI version."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise AlpxUnavailable(
            f"{LIB_PATH} is not built (run __graft_entry__.build() or make -C csrc)")
    try:
        handle = ctypes.CDLL(LIB_PATH)
    except OSError as exc:  # pragma: no cover - depends on the image
        raise AlpxUnavailable(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = handle.alpx_abi_version()
    if version != ABI_VERSION:
        raise AlpxUnavailable(f"libalpx ABI {version} != expected {ABI_VERSION}")
    _lib = handle
    return handle


def last_error() -> str:
    return lib().alpx_last_error().decode("utf-8", "replace")


def check(status: int) -> None:
    """Map a library status to the reference's exception types."""
    if status == OK:
        return
    message = last_error()
    if status in (EINVAL, ERANGE):
        raise ValueError(message)
    if status == EUNSUPPORTED:
        raise AlpxUnsupported(message)
    raise AlpxError(message, status)


def device_arch(index: int) -> str:
    buf = ctypes.create_string_buffer(256)
    check(lib().alpx_device_arch(int(index), buf, len(buf)))
    return buf.value.decode()


_dtype_codes: dict = {}


def host_device_pointer(host_address: int):
    """Device address of page-locked host memory, or None when the runtime
    does not map it (alpx_host_device_pointer)."""
    dev = ctypes.c_void_p()
    if lib().alpx_host_device_pointer(host_address, ctypes.byref(dev)) != OK or not dev.value:
        return None
    return dev.value


def dtype_code(torch, dtype) -> int:
    code = _dtype_codes.get(dtype)
    if code is not None:
        return code
    if not _dtype_codes:
        _dtype_codes.update({torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16})
        if dtype in _dtype_codes:
            return _dtype_codes[dtype]
    raise TypeError(f"unsupported dtype {dtype}")


_raw_stream = None


def current_stream(index: int) -> int:
    """hipStream_t of torch's current stream on device ``index`` (an int)."""
    global _raw_stream
    if _raw_stream is None:
        import torch
        _raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", False)
    if _raw_stream is not False:
        return _raw_stream(index)
    import torch
    return int(torch.cuda.current_stream(index).cuda_stream)


def stream_handle(torch, device) -> int:
    """hipStream_t of torch's current stream on ``device`` (a torch.device,
    an index or a device string).  Uses torch's raw stream query (no Stream
    object per call) when this torch build has it."""
    global _raw_stream
    index = getattr(device, "index", device)
    if _raw_stream is None:
        _raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", False)
    if _raw_stream is not False and (index is None or type(index) is int):
        return _raw_stream(torch.cuda.current_device() if index is None else index)
    return int(torch.cuda.current_stream(device).cuda_stream)


_workspaces: dict = {}
# Workspaces replaced by a larger one stay allocated until the process ends:
# a HIP graph captured while one of them was current keeps its address in
# its kernel arguments, and replays of that graph still write there.  Were
# the buffer returned to torch's caching allocator, those replays would
# overwrite whatever tensor torch handed the memory to next.  Each
# replacement at least doubles, so the retired buffers together hold less
# than the current workspace.
_retired: dict = {}


def workspace(torch, device, nbytes: int):
    """A grow-only scratch workspace per device, owned by this module.
    Calls that share it are ordered on one stream (the reference's
    one-caller-at-a-time contract, serve.py:326).  A graph that captures a
    call keeps using the workspace that was current at capture time, so
    graphs should be captured after the largest workspace a process needs
    has been sized (one eager call of each shape), though a later growth
    never frees the buffer a graph holds."""
    key = _device_keys.get(device)
    if key is None:
        key = _device_keys.setdefault(device, str(device))
    buf = _workspaces.get(key)
    if buf is None or _workspace_bytes[key] < nbytes:
        size = max(int(nbytes), 256)
        if buf is not None:
            _retired.setdefault(key, []).append(buf)
            # at least double, so the retired buffers together stay below
            # the current one (a decode loop asks for a little more as its
            # split count grows with the length)
            size = max(size, 2 * _workspace_bytes[key])
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = buf
        _workspace_bytes[key] = buf.numel()
    return buf


_device_keys: dict = {}     # device (object or string) -> str(device)
_workspace_bytes: dict = {}  # str(device) -> bytes of _workspaces[str(device)]
