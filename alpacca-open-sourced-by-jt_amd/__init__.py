"""MI355X (gfx950) attention path for alpaccaroo.

A hipcc-built shared library (``libalpx.so``, sources in ``csrc/``, C-ABI in
``include/alpx.h``) with hand-written kernels for KV-cache append, split-K
GQA decode, causal prefill and the gated delta-rule recurrence, behind
drop-in facades that mirror the reference's entry points:

* ``qwen35_rocm_ops.Qwen35RocmOps`` -- alpaccaroo/qwen35_rocm_ops.py
* ``qwen35_kernels`` -- alpaccaroo/qwen35_kernels.py
* ``kernels.attention_decode`` -- alpaccaroo/kernels.py
* ``cuda.attention_batch`` -- the prefill seam of alpaccaroo/cuda.py
* ``qwen35_ops`` -- list-in/list-out adapters of alpaccaroo/qwen35_ops.py

PyTorch-ROCm tensors serve only as device buffers and streams.
"""

from . import _lib  # noqa: F401

__all__ = ["_lib"]
