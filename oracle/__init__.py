"""CPU oracle for the MI355X attention path -- TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the reference algorithms that the HIP
library replaces (alpaccaroo, mounted read-only as the reference tree):

* ``oracle.attention`` -- KV append, GQA decode (two-pass and online forms),
  causal prefill, the ROCm ``online_attention`` contract and the sigmoid
  output gate.
* ``oracle.gdn`` -- the gated delta-rule (GDN) recurrence, token-sequential,
  plus the GDN input preparation (L2 normalisation, beta/decay).
* ``oracle.layer`` -- the Qwen3.5 layer primitives on either side of the
  kernels: causal convolution step, SiLU, L2 / RMS / gated RMS norms, the
  recurrent parameters, IMROPE, the query/gate split, and the composed
  attention prologue and recurrent-layer step.
* ``oracle.rope`` -- the llama "norm" (adjacent-pair) rotary embedding used
  to build prefill inputs.
* ``oracle.inputs`` -- seeded synthetic inputs for the five benchmark
  configurations and exact bf16/fp16 rounding helpers.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or as the
timed CPU baseline.  The product path (the ``alpacca-open-sourced-by-jt_amd``
package and its HIP library) never imports it and has no CPU fallback.

Parity pinning.  The reference ships no tests, golden vectors or fixtures
for this path, so every oracle function is pinned by closed forms,
invariants and special cases in ``tests/test_oracle.py`` (each test names
the mistake it would catch).  No function of this package is left
"parity unpinned".
"""

from . import attention, gdn, inputs, layer, rope  # noqa: F401

__all__ = ["attention", "gdn", "inputs", "layer", "rope"]
