"""CPU checks of the C-ABI boundary: the library loads, exports every symbol
the header declares, and rejects contract violations before touching the
GPU (no compute calls are made here)."""

import ctypes
import importlib
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "alpx.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(alpx_\w+)\s*\(", text)))


def test_header_symbols_exported(pkg):
    lib = pkg._lib.lib()
    names = _declared()
    assert "alpx_decode_gqa" in names and "alpx_kv_append" in names
    for name in names:
        assert hasattr(lib, name), name
        assert name in pkg._lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.alpx_abi_version() == pkg._lib.ABI_VERSION


def test_header_abi_version_matches_binding(pkg):
    m = re.search(r"#define ALPX_ABI_VERSION (\d+)", open(HEADER).read())
    assert int(m.group(1)) == pkg._lib.ABI_VERSION


def test_null_buffers_rejected_without_gpu(pkg):
    lib = pkg._lib.lib()
    rc = lib.alpx_kv_append(None, None, None, None, 0, 8, 1, 1, 4, 4, 1, 0, None, None)
    assert rc == pkg._lib.EINVAL and "null" in pkg._lib.last_error()
    rc = lib.alpx_decode_gqa(None, None, None, None, 4, None, None, None, 0, 1, 4, 2, 64, 64,
                             128, 0, 64, 128, 0, 64, 0.125, 0, 0, None)
    assert rc == pkg._lib.EINVAL
    with pytest.raises(ValueError):
        pkg._lib.check(rc)
    # the allocation-free variant validates before it looks up its scratch
    rc = lib.alpx_decode_gqa_noalloc(None, None, None, None, 4, None, None, 1, 4, 2, 64, 64,
                                     128, 0, 64, 128, 0, 64, 0.125, 0, 0, None)
    assert rc == pkg._lib.EINVAL and "null" in pkg._lib.last_error()
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    rc = lib.alpx_decode_gqa_noalloc(fake, fake, fake, None, 4, None, fake, 1, 6, 4, 64, 64,
                                     256, 0, 64, 256, 0, 64, 0.125, 1, 1, None)
    assert rc == pkg._lib.EINVAL and "multiple of KV heads" in pkg._lib.last_error()


def test_host_device_pointer_rejects_null_without_gpu(pkg):
    lib = pkg._lib.lib()
    dev = ctypes.c_void_p()
    assert lib.alpx_host_device_pointer(None, ctypes.byref(dev)) == pkg._lib.EINVAL
    assert "null" in pkg._lib.last_error()
    assert lib.alpx_host_device_pointer(ctypes.c_void_p(64), None) == pkg._lib.EINVAL


def test_gated_prefill_rejects_null_gate_without_gpu(pkg):
    lib = pkg._lib.lib()
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    rc = lib.alpx_prefill_causal_gated(fake, fake, fake, None, fake, None, 0, 4, 8, 4, 2, 64, 64,
                                       128, 128, 4, 0, 0, 0.125, 2, 2, None)
    assert rc == pkg._lib.EINVAL and "null gate" in pkg._lib.last_error()


def test_range_and_shape_errors_without_gpu(pkg):
    lib = pkg._lib.lib()
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    rc = lib.alpx_prefill_append(fake, None, fake, fake, fake, None, fake, None, 0, 4, 16, 8, 2,
                                 64, 64, 0, 0, 0.125, 2, 2, None)
    assert rc == pkg._lib.EINVAL and "null" in pkg._lib.last_error()
    rc = lib.alpx_prefill_append(fake, fake, fake, fake, fake, None, fake, None, 0, 4, 16, 8, 2,
                                 64, 64, 13, 0, 0.125, 2, 2, None)
    assert rc == pkg._lib.ERANGE and "exceeds capacity" in pkg._lib.last_error()
    rc = lib.alpx_kv_append(fake, fake, fake, fake, 1, 8, 1, 1, 4, 4, 2, 7, None, None)
    assert rc == pkg._lib.ERANGE and "exceeds capacity" in pkg._lib.last_error()
    rc = lib.alpx_decode_gqa(fake, fake, fake, None, 4, None, fake, fake, 1 << 20, 1, 6, 4, 64,
                             64, 256, 0, 64, 256, 0, 64, 0.125, 1, 1, None)
    assert rc == pkg._lib.EINVAL and "multiple of KV heads" in pkg._lib.last_error()
    rc = lib.alpx_decode_gqa(fake, fake, fake, None, 4, None, fake, fake, 16, 1, 8, 4, 64,
                             64, 256, 0, 64, 256, 0, 64, 0.125, 1, 1, None)
    assert rc == pkg._lib.EINVAL and "workspace" in pkg._lib.last_error()
    rc = lib.alpx_decode_gqa(fake, fake, fake, None, 4, None, fake, fake, 1 << 20, 1, 8, 4,
                             512, 512, 256, 0, 64, 256, 0, 64, 0.125, 1, 1, None)
    assert rc == pkg._lib.EUNSUPPORTED


def test_decode_workspace_sizes(pkg):
    lib = pkg._lib.lib()
    assert lib.alpx_decode_workspace_bytes(16, 32, 8, 128, 8192) > 0
    assert lib.alpx_decode_workspace_bytes(16, 30, 8, 128, 8192) == 0  # not a multiple
    # grows with the number of partial slots, never below the 1-slot size
    one = 3 * 256
    assert lib.alpx_decode_workspace_bytes(1, 1, 1, 64, 1) >= one


def test_workspace_growth_is_geometric_and_caches_are_bounded(pkg):
    # the facade's grow-only workspace (host memory stands in for a device
    # here): small growth steps, as a decode loop's lengthening plan asks
    # for, at least double the buffer, so the retired buffers kept for
    # captured graphs hold less than the current one
    import torch
    lib = pkg._lib
    dev = torch.device("cpu")
    key = str(dev)
    try:
        for n in range(1000, 60000, 700):
            buf = lib.workspace(torch, dev, n)
            assert buf.numel() >= n
        held = sum(b.numel() for b in lib._retired.get(key, []))
        assert held < lib._workspace_bytes[key]
        assert len(lib._retired.get(key, [])) <= 7
        # the decode call's workspace-size cache, asked with a new length
        # per token as a decode loop does, stays within its bound (the call
        # is only packed here, never launched)
        ops = importlib.import_module(pkg.__name__ + "._ops")
        ops._decode_ws_bytes.clear()
        q = torch.zeros((1, 8, 64))
        kc = torch.zeros((3000, 1, 2, 64))
        for length in range(1, ops._DECODE_WS_CACHE_MAX + 200):
            ops._decode_call(q, kc, kc, length=length, k_strides=(128, 128, 64),
                             v_strides=(128, 128, 64), batch=1, kv_heads=2)
            assert len(ops._decode_ws_bytes) <= ops._DECODE_WS_CACHE_MAX
    finally:
        importlib.import_module(pkg.__name__ + "._ops")._decode_ws_bytes.clear()
        lib._workspaces.pop(key, None)
        lib._workspace_bytes.pop(key, None)
        lib._retired.pop(key, None)
        lib._device_keys.pop(dev, None)


def test_facade_validation_mirrors_reference(pkg):
    import importlib

    import torch
    m = importlib.import_module(pkg.__name__ + ".qwen35_rocm_ops")
    cap = m.RocmCapability(True, "injected", 0, "gfx950")
    ops = m.Qwen35RocmOps(_capability=cap)
    t = torch.zeros(2, 2, 2)
    with pytest.raises(TypeError, match="must remain on the ROCm device"):
        ops.attention_append_(torch.zeros(4, 2, 2, 2), torch.zeros(4, 2, 2, 2), 0, t, t)
    with pytest.raises(TypeError, match="must be a PyTorch tensor"):
        ops.online_attention([1.0], t, t, length=1)
    with pytest.raises(m.Qwen35RocmUnavailable):
        m.Qwen35RocmOps(_capability=m.RocmCapability(False, "no device"))
    with pytest.raises(ValueError, match="positive integer"):
        ops.zeros((0, 2))


def test_layer_prefill_without_query_buffer_refusals_without_gpu(pkg):
    """alpx_attention_layer_prefill with query_out = NULL (the prefill forms
    the query heads itself) refuses what that form cannot do -- fp32, rotary
    sections that are not whole groups of 32, a head_dim it has no kernel
    for, a workspace too small for the rotation table -- before any launch."""
    L = pkg._lib
    lib = L.lib()
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    sec = (ctypes.c_int * 4)(11, 11, 10, 0)   # R = 32
    odd = (ctypes.c_int * 4)(10, 10, 10, 0)   # R = 30

    def call(dtype, sections, head_dim=256, ws=fake, ws_bytes=1 << 20, tokens=64):
        return lib.alpx_attention_layer_prefill(
            fake, fake, fake, fake, fake, None, fake, fake, fake, ws, ws_bytes, dtype, dtype,
            4096, 1, 0, tokens, 16, 2, head_dim, 0, sections, 1e7, 1e-6, 0.0625, None)

    assert call(L.F32, sec) == L.EUNSUPPORTED and "without query_out" in L.last_error()
    assert call(L.BF16, odd) == L.EUNSUPPORTED and "multiple of 32" in L.last_error()
    assert call(L.F16, sec, head_dim=96) == L.EUNSUPPORTED and "head_dim" in L.last_error()
    # 64 tokens x 32 pairs x 8 bytes = 16 KiB of rotation table
    assert call(L.BF16, sec, ws_bytes=16383) == L.EINVAL
    assert "16384 needed" in L.last_error()
    assert call(L.BF16, sec, ws=None) == L.EINVAL and "workspace" in L.last_error()

    def paged(dtype, sections, page=64, position=0, ws_bytes=1 << 20, head_dim=128):
        return lib.alpx_attention_layer_prefill_paged(
            fake, fake, fake, fake, fake, fake, fake, fake, 4, page, 8, 0, fake, fake, ws_bytes,
            dtype, 64, 16, 2, head_dim, position, sections, 1e7, 1e-6, 0.0625, None)

    assert paged(L.BF16, sec, page=32) == L.EINVAL and "power of two" in L.last_error()
    assert paged(L.BF16, sec, position=200) == L.ERANGE and "capacity" in L.last_error()
    assert paged(L.F32, sec) == L.EUNSUPPORTED and "fp16/bf16" in L.last_error()
    assert paged(L.BF16, odd) == L.EUNSUPPORTED and "multiple of 32" in L.last_error()
    assert paged(L.BF16, sec, ws_bytes=100) == L.EINVAL and "16384 needed" in L.last_error()


def test_layer_entry_points_validate_without_gpu(pkg):
    lib = pkg._lib.lib()
    L = pkg._lib
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    sec = (ctypes.c_int * 4)(11, 11, 10, 0)
    bad = (ctypes.c_int * 4)(0, 0, 0, 0)
    assert lib.alpx_row_norm(None, None, None, None, 4, 8, 0, 0, 1e-6, 0, 0, 0, None) == L.EINVAL
    assert lib.alpx_row_norm(fake, None, None, fake, 4, 8, 0, 0, 1e-6, 1, 0, 0, None) == L.EINVAL
    assert "weight" in L.last_error()
    assert lib.alpx_row_norm(fake, fake, None, fake, 4, 8, 0, 0, 1e-6, 2, 0, 0, None) == L.EINVAL
    assert "gate" in L.last_error()
    assert lib.alpx_row_norm(fake, None, None, fake, 4, 8, 0, 0, 0.0, 0, 0, 0, None) == L.EINVAL
    assert "epsilon" in L.last_error()
    assert lib.alpx_conv_step(None, fake, fake, fake, 1, 4, 4, 4, 1, 0, 0, None) == L.EINVAL
    assert lib.alpx_recurrent_parameters(fake, fake, fake, fake, fake, fake, 7, 2, None) == L.EINVAL
    assert "value heads" in L.last_error()
    assert lib.alpx_imrope(fake, fake, fake, 0, 4, 1, 64, bad, 1e4, 1.0, 0, 0, None) == L.EINVAL
    assert "rotary pair" in L.last_error()
    assert lib.alpx_imrope(fake, fake, fake, 0, 4, 1, 32, sec, 1e4, 1.0, 0, 0, None) == L.EINVAL
    assert "shorter" in L.last_error()
    rc = lib.alpx_attention_prologue(fake, fake, fake, fake, fake, fake, fake, fake, fake, 2, 64, 1,
                                     16, 2, 256, 256, 64, None, sec, 1e7, 1e-6, None)
    assert rc == L.ERANGE and "exceeds capacity" in L.last_error()
    rc = lib.alpx_attention_prologue(fake, fake, fake, fake, fake, fake, fake, fake, fake, 2, 64, 1,
                                     15, 2, 256, 256, 0, None, sec, 1e7, 1e-6, None)
    assert rc == L.EINVAL and "multiple of KV heads" in L.last_error()
    f9 = (fake,) * 9
    rc = lib.alpx_prefill_causal_paged(fake, fake, fake, fake, 4, 32, 8, 0, None, fake, 8, 64,
                                       8, 2, 128, 56, 0, 0, 0.0884, 2, None)
    assert rc == L.EINVAL and "power of two" in L.last_error()
    rc = lib.alpx_prefill_causal_paged(fake, fake, fake, fake, 4, 64, 8, 0, None, fake, 8, 264,
                                       8, 2, 128, 256, 0, 0, 0.0884, 2, None)
    assert rc == L.ERANGE and "exceeds capacity" in L.last_error()
    rc = lib.alpx_prefill_causal_paged(fake, fake, fake, None, 4, 64, 8, 0, None, fake, 8, 64,
                                       8, 2, 128, 56, 0, 0, 0.0884, 2, None)
    assert rc == L.EINVAL and "null block table" in L.last_error()
    rc = lib.alpx_prefill_causal_paged(fake, fake, fake, fake, 4, 64, 8, 0, None, fake, 8, 64,
                                       8, 2, 128, 56, 0, 0, 0.0884, 0, None)
    assert rc == L.EUNSUPPORTED and "paged" in L.last_error()
    rc = lib.alpx_attention_layer_step(*f9, 1 << 20, 2, 2, 64, 1, 16, 2, 256, 64, None, sec, 1e7,
                                       1e-6, 0.0625, None)
    assert rc == L.ERANGE and "exceeds capacity" in L.last_error()
    rc = lib.alpx_attention_layer_step(*f9[:8], None, 1 << 20, 2, 2, 64, 1, 16, 2, 256, 10,
                                       None, sec, 1e7, 1e-6, 0.0625, None)
    assert rc == L.EINVAL and "null" in L.last_error()
    rc = lib.alpx_attention_layer_step(*f9, 1 << 20, 2, 2, 64, 1, 16, 2, 256, 10, None, bad, 1e7,
                                       1e-6, 0.0625, None)
    assert rc == L.EINVAL and "rotary pair" in L.last_error()
    rc = lib.alpx_attention_layer_step(*f9, 16, 2, 2, 64, 1, 16, 2, 256, 10, None, sec, 1e7, 1e-6,
                                       0.0625, None)
    assert rc == L.EINVAL and "workspace" in L.last_error()
    # fp32 caches and widths outside {64, 128, 256} have no fused kernel
    rc = lib.alpx_attention_layer_step(*f9, 1 << 20, 0, 0, 64, 1, 16, 2, 256, 10, None, sec, 1e7,
                                       1e-6, 0.0625, None)
    assert rc == L.EUNSUPPORTED and "fused attention step" in L.last_error()
    rc = lib.alpx_attention_layer_step(*f9, 1 << 20, 2, 2, 64, 1, 16, 2, 96, 10, None, sec, 1e7,
                                       1e-6, 0.0625, None)
    assert rc == L.EUNSUPPORTED and "fused attention step" in L.last_error()
    # paged state transfer: table, page size and range checks
    rc = lib.alpx_kv_export_paged(fake, fake, None, 2, 4, 32, 8, fake, fake, 2, 2, 64, 64, 0, 0,
                                  8, None)
    assert rc == L.EINVAL and "null block table" in L.last_error()
    rc = lib.alpx_kv_import_paged(fake, fake, fake, fake, fake, 2, 4, 48, 8, 2, 2, 64, 64, 0, 0,
                                  8, None)
    assert rc == L.EINVAL and "power of two" in L.last_error()
    rc = lib.alpx_kv_export_paged(fake, fake, fake, 2, 4, 32, 8, fake, fake, 2, 2, 64, 64, 1, 100,
                                  40, None)
    assert rc == L.ERANGE and "exceed" in L.last_error()
    rc = lib.alpx_kv_export_paged(fake, fake, fake, 2, 4, 32, 8, fake, fake, 2, 2, 64, 64, 2, 0,
                                  8, None)
    assert rc == L.EINVAL and "batch_index" in L.last_error()
    # paged layer step: pool geometry, capacity, table and fused-shape checks
    f7 = (fake,) * 7
    rc = lib.alpx_attention_layer_step_paged(*f7, fake, 4, 16, 8, fake, fake, 1 << 20, 2, 2, 1, 16,
                                             2, 256, 10, None, sec, 1e7, 1e-6, 0.0625, None)
    assert rc == L.EINVAL and "power of two" in L.last_error()
    rc = lib.alpx_attention_layer_step_paged(*f7, fake, 4, 64, 8, fake, fake, 1 << 20, 2, 2, 1, 16,
                                             2, 256, 256, None, sec, 1e7, 1e-6, 0.0625, None)
    assert rc == L.ERANGE and "exceeds capacity" in L.last_error()
    rc = lib.alpx_attention_layer_step_paged(*f7, None, 4, 64, 8, fake, fake, 1 << 20, 2, 2, 1, 16,
                                             2, 256, 10, None, sec, 1e7, 1e-6, 0.0625, None)
    assert rc == L.EINVAL and "null" in L.last_error()
    rc = lib.alpx_attention_layer_step_paged(*f7, fake, 0, 64, 8, fake, fake, 1 << 20, 2, 2, 1, 16,
                                             2, 256, 10, None, sec, 1e7, 1e-6, 0.0625, None)
    assert rc == L.EINVAL and "sizes must be positive" in L.last_error()
    rc = lib.alpx_attention_layer_step_paged(*f7, fake, 4, 64, 8, fake, fake, 1 << 20, 0, 0, 1, 16,
                                             2, 256, 10, None, sec, 1e7, 1e-6, 0.0625, None)
    assert rc == L.EUNSUPPORTED and "fused attention step" in L.last_error()
    assert lib.alpx_recurrent_step_workspace_bytes(1, 16, 32, 128, 128) > 0
    assert lib.alpx_recurrent_step_workspace_bytes(1, 0, 32, 128, 128) == 0
    rc = lib.alpx_recurrent_step(fake, fake, 4, 1, fake, 4, fake, fake, fake, fake, fake, fake,
                                 fake, fake, fake, 16, 1, 16, 32, 128, 128, 1e-6, 0, None)
    assert rc == L.EINVAL and "workspace" in L.last_error()
    rc = lib.alpx_recurrent_step(fake, fake, 4, 1, fake, 4, fake, fake, fake, fake, fake, fake,
                                 fake, fake, fake, 1 << 30, 1, 16, 30, 128, 128, 1e-6, 0, None)
    assert rc == L.EINVAL and "multiple of key heads" in L.last_error()
    assert lib.alpx_silu(None, fake, 4, 0, 0, None) == L.EINVAL


def test_overrides_read_once_and_set_by_hook_without_gpu(pkg, monkeypatch):
    """Kernel-choice overrides come from the environment once, at load, and
    afterwards only from alpx_set_override: a variable set later changes
    nothing, and the hook validates its arguments."""
    L = pkg._lib
    lib = L.lib()
    before = lib.alpx_gdn_chunk_uses_mfma(L.BF16, 1024, 16, 32, 128, 128)
    monkeypatch.setenv("ALPX_GDN_SEQUENTIAL", "1")
    assert lib.alpx_gdn_chunk_uses_mfma(L.BF16, 1024, 16, 32, 128, 128) == before == 1
    prev = L.set_override(L.OVERRIDE_PREFILL_KERNEL, L.PREFILL_KERNELS["pair"])
    try:
        assert L.get_override(L.OVERRIDE_PREFILL_KERNEL) == 2
    finally:
        assert L.set_override(L.OVERRIDE_PREFILL_KERNEL, prev) == 2
    assert lib.alpx_set_override(99, 0) == L.EINVAL and "unknown override" in L.last_error()
    assert lib.alpx_set_override(L.OVERRIDE_GDN_SEQUENTIAL, 2) == L.EINVAL
    assert "out of range" in L.last_error()
    assert lib.alpx_get_override(-1) == L.EINVAL


def test_gdn_chunk_form_predicate_without_gpu(pkg, override):
    """alpx_gdn_chunk_uses_mfma: bf16 and fp32 inputs with key_dim 64 / 128
    / 256 and value_dim a multiple of 16 run the chunked kernels; phase B's
    unsigned 24 x 24-bit token offsets need token x row < 2^32, so longer
    calls run token by token instead of wrapping."""
    L = pkg._lib
    f = L.lib().alpx_gdn_chunk_uses_mfma
    assert f(L.BF16, 1024, 16, 32, 128, 128) == 1
    assert f(L.F32, 1024, 16, 32, 128, 128) == 1
    assert f(L.F16, 1024, 16, 32, 128, 128) == 0
    assert f(L.BF16, 1024, 16, 32, 100, 128) == 0
    assert f(L.BF16, 1024, 16, 32, 128, 40) == 0
    assert f(L.BF16, 1024, 16, 24, 128, 128) == 0
    assert f(L.BF16, 0, 16, 32, 128, 128) == 0
    # the wider row here is the value row, 32 x 128 = 2^12 elements
    assert f(L.BF16, (1 << 20) - 1, 16, 32, 128, 128) == 1
    assert f(L.BF16, 1 << 20, 16, 32, 128, 128) == 0
    # the key row: 2^14 x 256 = 2^22 elements, at most 1023 tokens
    assert f(L.F32, 1023, 1 << 14, 1 << 14, 256, 16) == 1
    assert f(L.F32, 1024, 1 << 14, 1 << 14, 256, 16) == 0
    override("gdn_sequential", 1)
    assert f(L.BF16, 1024, 16, 32, 128, 128) == 0


def test_layer_prefill_query_buffer_checks_workspace_first_without_gpu(pkg):
    """The query-buffer form of alpx_attention_layer_prefill refuses, before
    its prologue launch writes the caches, a call whose prefill leaves the
    MFMA kernels -- a cache of 2 GiB or more per tensor, an fp32 cache --
    without a large enough split-K workspace; the form without a query
    buffer refuses the 2 GiB cache outright."""
    L = pkg._lib
    lib = L.lib()
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    sec = (ctypes.c_int * 4)(11, 11, 10, 0)
    # 16 sequences x 2 heads x 256 dims of bf16: 16 KiB per cache row, so
    # 131072 rows make 2 GiB
    cap = 131072

    def call(query_out, ws, ws_bytes, dtype=L.BF16, position=cap - 64):
        return lib.alpx_attention_layer_prefill(
            fake, fake, fake, fake, fake, query_out, fake, fake, fake, ws, ws_bytes, dtype, dtype,
            cap, 16, 3, 64, 16, 2, 256, position, sec, 1e7, 1e-6, 0.0625, None)

    assert call(fake, None, 0) == L.EINVAL and "null workspace" in L.last_error()
    need = lib.alpx_prefill_workspace_bytes(64, 16, 2, 256, cap)
    assert need > 0
    assert call(fake, fake, need - 1) == L.EINVAL and f"{need} bytes" in L.last_error()
    assert call(None, fake, 1 << 20) == L.EUNSUPPORTED and "2 GiB" in L.last_error()
    assert call(fake, None, 0, dtype=L.F32, position=0) == L.EINVAL
    assert "workspace" in L.last_error()
