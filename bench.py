#!/usr/bin/env python3
"""Benchmark of the MI355X attention path; prints ONE JSON line.

Headline (``value``): GQA decode attention at 8K context -- BASELINE config
C2, uniform-8192 variant: 16 sequences x 8192 cached rows, 32 query / 8 KV
heads, head_dim 128, fp16 cache in the ROCm layout [8192, 16, 8, 128] --
reported as algorithmic HBM GB/s (K + V bytes of every valid row, plus q and
o) per decode step, whole step (split + combine) timed.  ``roofline`` covers
the dominant kernel (the split-K pass), timed with HIP events recorded by
the library on its launch stream over the timed region.  ``extra`` carries
the other configs (C1 fp32 decode, C4 gated bf16 decode, ...).
``cpu_baseline`` times the NumPy oracle (the reference's two-pass llama
algorithm, fp32) on the same C2 workload on this host.

``roofline.traffic`` (HBM bytes per split launch) comes from two rocprofv3
counter runs of ``bench.py --pmc-probe`` (FETCH_SIZE, then WRITE_SIZE), each
scaled by what the counter reads for a plain copy of known size in the same
run; ``bench.py --traffic-summary FETCH_DIR WRITE_DIR`` turns the two runs
into the summary under profiles/ that this script reads.

Inputs are synthetic N(0, 1) (seeded), generated on the device.
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
PACKAGE = "alpacca-open-sourced-by-jt_amd"

METRIC = ("decode attn HBM GB/s (% of peak) @8K ctx; "
          "prefill attn TFLOP/s (% MFMA peak)")
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "pmc_traffic_decode_split_c2_f16.md")
C2_SHAPE = dict(batch=16, ctx=8192, hq=32, hkv=8, d=128)
SPLIT_KERNEL = "decode_split_mfma"
COPY_KERNEL = "kv_append_kernel"


def _mod(name):
    return importlib.import_module(f"{PACKAGE}.{name}")


def _timed_steps(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


def _kernel_avg_ms(lib, kernel):
    total, count = lib.timing_read(kernel)
    return (total / count) if count else float("nan")


def bench_decode(torch, ops, lib, *, batch, ctx, hq, hkv, d, dtype, gate, steps, warmup,
                 seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = torch.device("cuda")
    q = torch.randn((batch, hq, d), generator=g, device=dev).to(dtype)
    K = torch.randn((ctx, batch, hkv, d), generator=g, device=dev).to(dtype)
    V = torch.randn((ctx, batch, hkv, d), generator=g, device=dev).to(dtype)
    gt = torch.randn((batch, hq, d), generator=g, device=dev).to(dtype) if gate else None
    fn = lambda: ops.online_attention(q, K, V, length=ctx, gate=gt)  # noqa: E731
    # Timed region 1: the K steps as a caller runs them (value, ms_per_step).
    ms = _timed_steps(torch, fn, steps, warmup)
    # Timed region 2: the same K steps with the library's HIP-event brackets
    # on the launch stream, for per-kernel durations (roofline).  Event
    # records cost a few microseconds each, so region 1 excludes them.
    lib.timing_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    ev_ms = (time.perf_counter() - t0) / steps * 1e3
    split_ms = _kernel_avg_ms(lib, lib.T_DECODE)
    comb_ms = _kernel_avg_ms(lib, lib.T_DECODE_COMBINE)
    lib.timing_enable(False)
    es = q.element_size()
    kv_bytes = 2 * ctx * batch * hkv * d * es
    q_bytes = batch * hq * d * es
    step_bytes = kv_bytes + q_bytes * (3 if gate else 2)  # + gate + o
    return {
        "ms_per_step": ms,
        "gbs": step_bytes / (ms * 1e-3) / 1e9,
        "split_ms": split_ms,
        "combine_ms": comb_ms,
        "ms_per_step_with_events": ev_ms,
        "split_alg_bytes": kv_bytes + q_bytes,
        "split_gbs": (kv_bytes + q_bytes) / (split_ms * 1e-3) / 1e9,
        "step_bytes": step_bytes,
        "tensors": (q, K, V),
    }


def bench_prefill(torch, ops, lib, *, steps, warmup, seed=3):
    """C3: causal prefill of a 2048-token bf16 chunk whose K/V were appended
    at rows 2048..4095 of a [4096, 1, 8, 128] cache; 32 query heads.  The
    step is the prefill attention call; FLOPs count causal-valid pairs only."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = torch.device("cuda")
    tq, prefix, hq, hkv, d = 2048, 2048, 32, 8, 128
    K = torch.randn((prefix + tq, 1, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    V = torch.randn((prefix + tq, 1, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((tq, hq, d), generator=g, device=dev).to(torch.bfloat16)
    fn = lambda: ops.attention_prefill(q, K, V, position=prefix)  # noqa: E731
    ms = _timed_steps(torch, fn, steps, warmup)
    lib.timing_enable(True)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    k_ms = _kernel_avg_ms(lib, lib.T_PREFILL)
    lib.timing_enable(False)
    # the same rows in a paged pool: 256-row pages in shuffled order
    page, n_pages = 256, (prefix + tq) // 256
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(seed))
    kp = torch.empty((n_pages, page, hkv, d), dtype=K.dtype, device=dev)
    vp = torch.empty_like(kp)
    kp[perm.to(dev)] = K.view(n_pages, page, hkv, d)
    vp[perm.to(dev)] = V.view(n_pages, page, hkv, d)
    table = perm.to(torch.int32).view(1, n_pages).to(dev)
    fp = lambda: ops.paged_attention_prefill(q, kp, vp, table, position=prefix)  # noqa: E731
    _timed_steps(torch, fp, 3, 2)
    lib.timing_enable(True)
    for _ in range(steps):
        fp()
    torch.cuda.synchronize()
    pk_ms = _kernel_avg_ms(lib, lib.T_PREFILL)
    lib.timing_enable(False)
    pairs = sum(prefix + i + 1 for i in range(tq))  # 6,292,480
    flops = 4 * d * hq * pairs                      # QK^T and PV, 2 FLOP per MAC
    return {"ms_per_step": ms, "kernel_ms": k_ms, "flops": flops,
            "tflops": flops / (ms * 1e-3) / 1e12, "kernel_tflops": flops / (k_ms * 1e-3) / 1e12,
            "paged_kernel_ms": pk_ms}


def bench_gdn(torch, ops, lib, *, steps, warmup, seed=5):
    """C5: gated delta rule, 16 q/k heads, 32 v heads, Dk = Dv = 128, fp32
    state; a 1024-token chunked prefill, then 256 single-token decode steps.
    Prefill FLOPs follow the chunked form (2 C^2 (3 Dk + 2 Dv) + 6 C Dk Dv per
    head-chunk); decode bytes are the state read + write plus q/k/v/o."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = torch.device("cuda")
    T, hk, hv, dk, dv, C = 1024, 16, 32, 128, 128, 64
    q = torch.nn.functional.normalize(torch.randn((1, T, hk, dk), generator=g, device=dev), dim=-1)
    k = torch.nn.functional.normalize(torch.randn((1, T, hk, dk), generator=g, device=dev), dim=-1)
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    v = torch.randn((1, T, hv, dv), generator=g, device=dev).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn((1, T, hv), generator=g, device=dev))
    a = torch.rand((hv,), generator=g, device=dev) * 2 - 1
    gl = (-torch.exp(a) * torch.nn.functional.softplus(
        torch.randn((1, T, hv), generator=g, device=dev))).contiguous()
    S = torch.zeros((1, hv, dv, dk), dtype=torch.float32, device=dev)
    fn = lambda: ops.gated_delta_net_chunk_(S, q, k, v, beta, gl)  # noqa: E731
    ms = _timed_steps(torch, fn, steps, warmup)
    lib.timing_enable(True)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    k_ms = _kernel_avg_ms(lib, lib.T_GDN_CHUNK)
    lib.timing_enable(False)
    head_chunks = hv * (T // C)
    flops = head_chunks * (2 * C * C * (3 * dk + 2 * dv) + 6 * C * dk * dv)
    # decode: 256 steps on the carried state
    q1, k1, v1 = q[:, 0].contiguous(), k[:, 0].contiguous(), v[:, 0].contiguous()
    b1, g1 = beta[:, 0].contiguous(), gl[:, 0].contiguous()
    step = lambda: ops.gated_delta_net_step_(S, q1, k1, v1, b1, g1)  # noqa: E731
    n_dec = 256
    dec_ms = _timed_steps(torch, step, n_dec, 16)
    lib.timing_enable(True)
    for _ in range(n_dec):
        step()
    torch.cuda.synchronize()
    dk_ms = _kernel_avg_ms(lib, lib.T_GDN_STEP)
    lib.timing_enable(False)
    step_bytes = 2 * hv * dv * dk * 4 + (2 * hk * dk + 2 * hv * dv) * 2
    return {"prefill_ms": ms, "prefill_kernel_ms": k_ms, "prefill_flops": flops,
            "prefill_tflops": flops / (k_ms * 1e-3) / 1e12,
            "decode_us_per_step": dec_ms * 1e3, "decode_kernel_us": dk_ms * 1e3,
            "decode_step_bytes": step_bytes,
            "decode_kernel_gbs": step_bytes / (dk_ms * 1e-3) / 1e9}


def bench_layers(torch, ops, lib, *, steps, warmup, seed=6):
    """The two fused Qwen3.5 decode-step paths around the kernels.

    * Attention layer at the C4 geometry (4 sequences, 16 q / 2 kv heads,
      head_dim 256, bf16 cache of 32768 rows): prologue (query/gate split,
      Q/K RMSNorm, IMROPE, append at row 32767) inside the split-K launch
      over 32768 rows, then the combine with the sigmoid gate (two
      launches; ``kernel_us`` is their HIP-event sum).  The three-launch
      path (prologue kernel, split, combine) is timed beside it.  Bytes per
      step: the K/V rows read (as C4) plus the prologue's projection reads
      and cache writes.
    * Recurrent layer at the C5 geometry (16 k / 32 v heads, Dk = Dv = 128,
      conv kernel 4, batch 1): conv + SiLU + split + Q/K L2 + beta/decay,
      GDN step, gated RMSNorm (two launches; ``kernel_us`` is their
      HIP-event span).  Bytes per step: state read + write, conv history
      read + write, conv weights, projections in, output out."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = torch.device("cuda")
    bf = torch.bfloat16
    b, hq, hkv, d, ctx = 4, 16, 2, 256, 32768
    K = torch.randn((ctx, b, hkv, d), generator=g, device=dev).to(bf)
    V = torch.randn((ctx, b, hkv, d), generator=g, device=dev).to(bf)
    qg = torch.randn((b, hq * 2 * d), generator=g, device=dev).to(bf)
    kn = torch.randn((b, hkv * d), generator=g, device=dev).to(bf)
    vn = torch.randn((b, hkv * d), generator=g, device=dev).to(bf)
    qw = torch.rand((d,), generator=g, device=dev) + 0.5
    kw = torch.rand((d,), generator=g, device=dev) + 0.5

    rope = dict(sections=(11, 11, 10, 0), frequency_base=10000000.0, epsilon=1e-6)

    def attn_step():
        return ops.attention_layer_step_(qg, kn, vn, qw, kw, K, V, position=ctx - 1, **rope)

    def attn_three_launches():
        q, gate, _ = ops.attention_prologue_(qg, kn, vn, qw, kw, K, V, position=ctx - 1, **rope)
        return ops.online_attention(q, K, V, length=ctx, gate=gate)

    a_ms = _timed_steps(torch, attn_step, steps, warmup)
    a3_ms = _timed_steps(torch, attn_three_launches, steps, warmup)
    lib.timing_enable(True)
    for _ in range(steps):
        attn_step()
    torch.cuda.synchronize()
    ak_ms = _kernel_avg_ms(lib, lib.T_DECODE) + _kernel_avg_ms(lib, lib.T_DECODE_COMBINE)
    lib.timing_enable(False)
    es = 2
    a_bytes = (2 * ctx * b * hkv * d * es + (hq * 2 * d + 2 * hkv * d) * b * es
               + 2 * b * hkv * d * es + 2 * b * hq * d * es + b * hq * d * es)

    bsz, hk, hv, dk, dv, kern = 1, 16, 32, 128, 128, 4
    chn = 2 * hk * dk + hv * dv
    ws = ops.initialize_recurrent_workspace(batch_size=bsz, convolution_kernel=kern,
                                            convolution_channels=chn, value_heads=hv,
                                            value_dimension=dv, key_dimension=dk)
    mixed = torch.randn((bsz, chn), generator=g, device=dev)
    cw = torch.randn((kern, chn), generator=g, device=dev) * 0.5
    gate = torch.randn((bsz, hv * dv), generator=g, device=dev)
    bl = torch.randn((bsz, hv), generator=g, device=dev)
    al = torch.randn((bsz, hv), generator=g, device=dev)
    dt = torch.randn((hv,), generator=g, device=dev)
    ssm = -torch.exp(torch.rand((hv,), generator=g, device=dev) * 2 - 1)
    nw = torch.rand((dv,), generator=g, device=dev) + 0.5

    def rec_step():
        return ops.recurrent_layer_step_(ws, mixed, cw, gate, bl, al, dt, ssm, nw,
                                         key_heads=hk, key_dimension=dk, epsilon=1e-6)

    r_ms = _timed_steps(torch, rec_step, steps, warmup)
    lib.timing_enable(True)
    for _ in range(steps):
        rec_step()
    torch.cuda.synchronize()
    rk_ms = _kernel_avg_ms(lib, lib.T_RECURRENT_STEP)
    lib.timing_enable(False)
    r_bytes = (2 * bsz * hv * dv * dk * 4 + 2 * bsz * (kern - 1) * chn * 4 + kern * chn * 4
               + bsz * chn * 4 + 2 * bsz * hv * dv * 4 + 2 * bsz * hv * 4 + 2 * hv * 4 + dv * 4)
    return {
        "attention_layer_c4": {
            "us_per_step": round(a_ms * 1e3, 2),
            "kernel_us": round(ak_ms * 1e3, 2),
            "three_launch_us_per_step": round(a3_ms * 1e3, 2),
            "step_bytes": a_bytes,
            "step_gbs": round(a_bytes / (a_ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(a_bytes / (a_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "recurrent_layer_c5": {
            "us_per_step": round(r_ms * 1e3, 2),
            "kernel_us": round(rk_ms * 1e3, 2),
            "step_bytes": r_bytes,
            "kernel_gbs": round(r_bytes / (rk_ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(r_bytes / (rk_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
    }


def bench_paged(torch, ops, lib, c2, *, steps, warmup, seed=8):
    """C2 through a paged pool: the same 16 x 8192 fp16 rows in 256-row pages
    assigned in shuffled order; the step is the paged split + combine."""
    q, K, V = c2["tensors"]
    batch, hkv, d, ctx, page = 16, 8, 128, 8192, 256
    max_pages = ctx // page
    g = torch.Generator(device="cpu").manual_seed(seed)
    perm = torch.randperm(batch * max_pages, generator=g).to(torch.int32)
    table = perm.reshape(batch, max_pages).to(q.device)
    pw = ops.initialize_paged_attention_workspace(num_pages=batch * max_pages, page_size=page,
                                                  kv_heads=hkv, key_dimension=d,
                                                  value_dimension=d, dtype=q.dtype)
    _mod("_ops").kv_append_paged(pw.key_pages, pw.value_pages, table, K, V, position=0)
    fn = lambda: ops.paged_online_attention(q, pw.key_pages, pw.value_pages, table,  # noqa: E731
                                            length=ctx)
    ms = _timed_steps(torch, fn, steps, warmup)
    lib.timing_enable(True)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    split_ms = _kernel_avg_ms(lib, lib.T_DECODE)
    lib.timing_enable(False)
    return {"c2_paged_256_rows": {
        "ms_per_step": round(ms, 5), "gbs": round(c2["step_bytes"] / (ms * 1e-3) / 1e9, 1),
        "split_ms": round(split_ms, 5),
        "split_gbs": round(c2["split_alg_bytes"] / (split_ms * 1e-3) / 1e9, 1),
        "vs_contiguous_step": round(c2["ms_per_step"] / ms, 3)}}


def bench_layer_prefill(torch, ops, lib, *, steps, warmup, seed=7):
    """The chunked Qwen3.5 layer prefill against the device's own
    token-by-token path (the reference's prefill is token-sequential).

    * Attention layer, Qwen3.5 head geometry (16 q / 2 kv heads, head_dim
      256, bf16), one sequence: a 2048-token chunk at position 2048 of a
      4096-row cache -- chunk prologue + causal prefill + sigmoid gate.
      FLOPs count causal-valid pairs (4 D Hq per pair).  Token path: 2048
      attention-layer decode steps (prologue in the split-K launch, gated
      combine).
    * Recurrent layer, C5 geometry (16 k / 32 v heads, Dk = Dv = 128, conv
      kernel 4): a 1024-token chunk -- chunk prep + chunked GDN + gated
      RMSNorm.  Token path: 1024 fused recurrent-layer steps."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = torch.device("cuda")
    bf = torch.bfloat16
    hq, hkv, d, prefix, T = 16, 2, 256, 2048, 2048
    sec, base, eps = (11, 11, 10, 0), 10000000.0, 1e-6
    K = torch.randn((prefix + T, 1, hkv, d), generator=g, device=dev).to(bf)
    V = torch.randn((prefix + T, 1, hkv, d), generator=g, device=dev).to(bf)
    qg = torch.randn((T, hq * 2 * d), generator=g, device=dev).to(bf)
    kn = torch.randn((T, hkv * d), generator=g, device=dev).to(bf)
    vn = torch.randn((T, hkv * d), generator=g, device=dev).to(bf)
    qw = torch.rand((d,), generator=g, device=dev) + 0.5
    kw = torch.rand((d,), generator=g, device=dev) + 0.5
    chunk = lambda: ops.attention_layer_prefill_(  # noqa: E731
        qg, kn, vn, qw, kw, K, V, position=prefix, sections=sec, frequency_base=base,
        epsilon=eps)
    a_ms = _timed_steps(torch, chunk, max(3, steps // 5), 2)

    def tokens_attn():
        for t in range(T):
            ops.attention_layer_step_(qg[t:t + 1], kn[t:t + 1], vn[t:t + 1], qw, kw, K, V,
                                      position=prefix + t, sections=sec, frequency_base=base,
                                      epsilon=eps)

    at_ms = _timed_steps(torch, tokens_attn, 2, 1)
    pairs = sum(prefix + i + 1 for i in range(T))
    a_flops = 4 * d * hq * pairs

    hk, hv, dk, dv, kern, R = 16, 32, 128, 128, 4, 1024
    chn = 2 * hk * dk + hv * dv
    ws = ops.initialize_recurrent_workspace(batch_size=1, convolution_kernel=kern,
                                            convolution_channels=chn, value_heads=hv,
                                            value_dimension=dv, key_dimension=dk)
    mixed = torch.randn((R, chn), generator=g, device=dev)
    cw = torch.randn((kern, chn), generator=g, device=dev) * 0.5
    gate = torch.randn((R, hv * dv), generator=g, device=dev)
    bl = torch.randn((R, hv), generator=g, device=dev)
    al = torch.randn((R, hv), generator=g, device=dev)
    dt = torch.randn((hv,), generator=g, device=dev)
    ssm = -torch.exp(torch.rand((hv,), generator=g, device=dev) * 2 - 1)
    nw = torch.rand((dv,), generator=g, device=dev) + 0.5
    rchunk = lambda: ops.recurrent_layer_prefill_(  # noqa: E731
        ws, mixed, cw, gate, bl, al, dt, ssm, nw, key_heads=hk, key_dimension=dk, epsilon=eps)
    r_ms = _timed_steps(torch, rchunk, max(3, steps // 5), 2)

    def tokens_rec():
        for t in range(R):
            ops.recurrent_layer_step_(ws, mixed[t:t + 1], cw, gate[t:t + 1], bl[t:t + 1],
                                      al[t:t + 1], dt, ssm, nw, key_heads=hk, key_dimension=dk,
                                      epsilon=eps)

    rt_ms = _timed_steps(torch, tokens_rec, 2, 1)
    return {
        "attention_layer_prefill_qwen35_2k_on_2k": {
            "chunk_ms": round(a_ms, 4), "token_path_ms": round(at_ms, 3),
            "speedup": round(at_ms / a_ms, 1), "flops": a_flops,
            "chunk_tflops": round(a_flops / (a_ms * 1e-3) / 1e12, 1)},
        "recurrent_layer_prefill_c5_1024": {
            "chunk_ms": round(r_ms, 4), "token_path_ms": round(rt_ms, 3),
            "speedup": round(rt_ms / r_ms, 1)},
    }


def cpu_baseline_c2(q, K, V, batch, hkv, d, budget_s=12.0):
    """Time the oracle's two-pass llama decode (fp32, model.py:1246-1252) on
    the C2 workload; returns GB/s of algorithmic bytes and the sample."""
    import numpy as np
    from oracle import attention as A
    try:
        from threadpoolctl import threadpool_info
        blas = [i for i in threadpool_info() if i.get("user_api") == "blas"]
        cores = max(int(i.get("num_threads", 1)) for i in blas) if blas else 1
    except Exception:  # pragma: no cover
        cores = 1
    qh = q.float().cpu().numpy()
    # llama layout: one contiguous (t, n_kv, hd) fp32 cache per sequence
    Kh = [np.ascontiguousarray(K[:, b].float().cpu().numpy()) for b in range(batch)]
    Vh = [np.ascontiguousarray(V[:, b].float().cpu().numpy()) for b in range(batch)]
    group = qh.shape[1] // hkv
    scale = 1.0 / math.sqrt(d)
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        for b in range(batch):
            A.attention_decode_twopass(qh[b], Kh[b], Vh[b], group, scale, acc=np.float32)
        times.append(time.perf_counter() - t0)
    step_s = statistics.median(times)
    es = 2  # algorithmic bytes are counted at the workload's fp16 storage size
    ctx = Kh[0].shape[0]
    step_bytes = 2 * ctx * batch * hkv * d * es + 2 * qh.size * es
    return {
        "value": step_bytes / step_s / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"full C2 uniform-8192 step (16 sequences, NumPy two-pass fp32 "
                   f"oracle), median of {len(times)} runs, {step_s * 1e3:.1f} ms/step"),
    }


def _c2_tensors(torch, seed=2):
    g = torch.Generator(device="cuda").manual_seed(seed)
    b, c, hq, hkv, d = (C2_SHAPE[k] for k in ("batch", "ctx", "hq", "hkv", "d"))
    q = torch.randn((b, hq, d), generator=g, device="cuda").half()
    K = torch.randn((c, b, hkv, d), generator=g, device="cuda").half()
    V = torch.randn((c, b, hkv, d), generator=g, device="cuda").half()
    return q, K, V


def pmc_probe(torch, ops, steps) -> int:
    """Workload for the counter runs: 3 plain copies of known size (the
    library's append kernel writing a whole C2-sized K and V cache: it reads
    and writes 2 x 268,435,456 bytes per launch), then ``steps`` C2 decode
    steps.  Prints the copy's byte count for the summary step."""
    q, K, V = _c2_tensors(torch)
    Kc, Vc = torch.empty_like(K), torch.empty_like(V)
    ops_mod = _mod("_ops")
    for _ in range(3):
        ops_mod.kv_append(Kc, Vc, K, V, position=0)
    for _ in range(steps):
        ops.online_attention(q, K, V, length=C2_SHAPE["ctx"])
    torch.cuda.synchronize()
    copy_bytes = 2 * K.numel() * K.element_size()
    print(json.dumps({"copy_kernel": COPY_KERNEL, "copy_read_bytes": copy_bytes,
                      "copy_write_bytes": copy_bytes, "split_kernel": SPLIT_KERNEL,
                      "decode_steps": steps}))
    return 0


def _counter_means(run_dir, counter):
    """Mean per-dispatch value of ``counter`` for the copy and split kernels
    in one rocprofv3 CSV run directory (rows of one dispatch are summed)."""
    import csv
    import glob
    files = glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {run_dir}")
    per = {COPY_KERNEL: {}, SPLIT_KERNEL: {}}
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] != counter:
                    continue
                for key, acc in per.items():
                    if key in r["Kernel_Name"]:
                        did = (f, r["Dispatch_Id"])
                        acc[did] = acc.get(did, 0.0) + float(r["Counter_Value"])
    out = {}
    for key, acc in per.items():
        if not acc:
            raise SystemExit(f"{counter}: no dispatch of {key} in {run_dir}")
        out[key] = (statistics.mean(acc.values()), len(acc))
    return out


def traffic_summary(fetch_dir, write_dir) -> int:
    """Print the profiles/ summary (markdown) from the two counter runs."""
    copy_bytes = 2 * C2_SHAPE["ctx"] * C2_SHAPE["batch"] * C2_SHAPE["hkv"] * C2_SHAPE["d"] * 2
    fetch = _counter_means(fetch_dir, "FETCH_SIZE")
    write = _counter_means(write_dir, "WRITE_SIZE")
    f_scale = copy_bytes / (fetch[COPY_KERNEL][0] * 1024.0)
    w_scale = copy_bytes / (write[COPY_KERNEL][0] * 1024.0)
    fetch_b = fetch[SPLIT_KERNEL][0] * 1024.0 * f_scale
    write_b = write[SPLIT_KERNEL][0] * 1024.0 * w_scale
    b, c, hq, hkv, d = (C2_SHAPE[k] for k in ("batch", "ctx", "hq", "hkv", "d"))
    alg = 2 * c * b * hkv * d * 2 + b * hq * d * 2
    rec = {"kernel": SPLIT_KERNEL + "<f16,128>", "workload": "C2 uniform 8192, fp16",
           "traffic_bytes_per_launch": round(fetch_b + write_b),
           "fetch_bytes_per_launch": round(fetch_b), "write_bytes_per_launch": round(write_b),
           "alg_bytes_per_launch": alg,
           "traffic_over_alg": round((fetch_b + write_b) / alg, 4),
           "fetch_scale": round(f_scale, 5), "write_scale": round(w_scale, 5)}
    print("# HBM traffic of the decode split kernel (C2 uniform-8192, fp16)\n")
    print("Counter runs (one rocprofv3 run per counter, from the repository root):\n")
    print("```")
    for ctr, dname in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        print(f"rocprofv3 --pmc {ctr} --output-format csv -d {dname} -o run -- "
              "python3 bench.py --pmc-probe")
    print(f"python3 bench.py --traffic-summary {fetch_dir} {write_dir}")
    print("```\n")
    print("| kernel | counter | mean KiB / dispatch | dispatches |")
    print("|---|---|---|---|")
    for ctr, res in (("FETCH_SIZE", fetch), ("WRITE_SIZE", write)):
        for key in (COPY_KERNEL, SPLIT_KERNEL):
            print(f"| {key} | {ctr} | {res[key][0]:.1f} | {res[key][1]} |")
    print(f"\nCalibration: the copy moves {copy_bytes} bytes each way per launch; "
          f"scale = known bytes / (counter KiB x 1024): fetch {f_scale:.4f}, "
          f"write {w_scale:.4f}.\n")
    print("traffic_json: " + json.dumps(rec))
    return 0


def _measured_traffic():
    """Bytes per split launch from the committed counter summary, or None."""
    try:
        with open(TRAFFIC_FILE) as fh:
            for line in fh:
                if line.startswith("traffic_json: "):
                    return json.loads(line[len("traffic_json: "):])
    except OSError:
        return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--workloads", default="c4,c3,c5,c1,layers,lprefill,paged",
                    help="comma list of secondary workloads to run "
                         "(c1, c3, c4, c5, layers, lprefill, paged)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run the counter-run workload (copy calibration + C2 steps)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two rocprofv3 counter runs of --pmc-probe")
    args = ap.parse_args()
    if args.traffic_summary:
        return traffic_summary(*args.traffic_summary)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the path has no multi-GPU component in this build)", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    lib = _mod("_lib")
    ops = _mod("qwen35_rocm_ops").Qwen35RocmOps()
    steps, warmup = args.steps, args.warmup
    if args.pmc_probe:
        return pmc_probe(torch, ops, 5)

    # headline: C2 uniform-8192 fp16
    c2 = bench_decode(torch, ops, lib, batch=16, ctx=8192, hq=32, hkv=8, d=128,
                      dtype=torch.float16, gate=False, steps=steps, warmup=warmup, seed=2)
    extra = {}
    wl = set(args.workloads.split(",")) if not args.only_headline or "--workloads" in " ".join(sys.argv) else set()
    if "c4" in wl:
        c4 = bench_decode(torch, ops, lib, batch=4, ctx=32768, hq=16, hkv=2, d=256,
                          dtype=torch.bfloat16, gate=True, steps=steps, warmup=warmup, seed=4)
        c4.pop("tensors")
        extra["c4_gated_decode_bf16_32k"] = {
            "gbs": round(c4["gbs"], 1), "frac_hbm": round(c4["gbs"] / HBM_PEAK_GBS, 4),
            "ms_per_step": round(c4["ms_per_step"], 4),
            "split_kernel_gbs": round(c4["split_gbs"], 1),
            "split_ms": round(c4["split_ms"], 4), "combine_ms": round(c4["combine_ms"], 4)}
    if "c3" in wl:
        c3 = bench_prefill(torch, ops, lib, steps=steps, warmup=warmup)
        extra["c3_prefill_bf16_2k_on_2k"] = {
            "tflops": round(c3["tflops"], 1),
            "frac_mfma_bf16": round(c3["tflops"] / BF16_PEAK_TFLOPS, 4),
            "ms_per_step": round(c3["ms_per_step"], 4),
            "kernel_ms": round(c3["kernel_ms"], 4),
            "kernel_tflops": round(c3["kernel_tflops"], 1),
            "flops_per_step": c3["flops"],
            "paged_256_rows_kernel_ms": round(c3["paged_kernel_ms"], 4),
            "paged_vs_contiguous_kernel": round(c3["kernel_ms"] / c3["paged_kernel_ms"], 3)}
    if "c5" in wl:
        c5 = bench_gdn(torch, ops, lib, steps=steps, warmup=warmup)
        extra["c5_gdn_bf16"] = {
            "prefill_1024_ms": round(c5["prefill_ms"], 4),
            "prefill_kernel_ms": round(c5["prefill_kernel_ms"], 4),
            "prefill_kernel_tflops": round(c5["prefill_tflops"], 1),
            "prefill_frac_mfma_bf16": round(c5["prefill_tflops"] / BF16_PEAK_TFLOPS, 4),
            "prefill_flops_chunked": c5["prefill_flops"],
            "decode_us_per_step": round(c5["decode_us_per_step"], 2),
            "decode_kernel_us": round(c5["decode_kernel_us"], 2),
            "decode_kernel_gbs": round(c5["decode_kernel_gbs"], 1),
            "decode_frac_hbm": round(c5["decode_kernel_gbs"] / HBM_PEAK_GBS, 4)}
    if "c1" in wl:
        c1 = bench_decode(torch, ops, lib, batch=1, ctx=512, hq=32, hkv=8, d=64,
                          dtype=torch.float32, gate=False, steps=steps, warmup=warmup, seed=1)
        c1.pop("tensors")
        extra["c1_decode_fp32_512"] = {
            "us_per_step": round(c1["ms_per_step"] * 1e3, 2),
            "split_us": round(c1["split_ms"] * 1e3, 2),
            "combine_us": round(c1["combine_ms"] * 1e3, 2)}
    if "layers" in wl:
        extra.update(bench_layers(torch, ops, lib, steps=steps, warmup=warmup))
    if "paged" in wl:
        extra.update(bench_paged(torch, ops, lib, c2, steps=steps, warmup=warmup))
    if "lprefill" in wl:
        extra.update(bench_layer_prefill(torch, ops, lib, steps=steps, warmup=warmup))
    extra["c2_combine_ms"] = round(c2["combine_ms"], 5)

    cpu = None
    if not args.no_cpu:
        q, K, V = c2["tensors"]
        cpu = cpu_baseline_c2(q, K, V, 16, 8, 128)
    c2.pop("tensors")

    traffic = _measured_traffic()
    if traffic:
        extra["traffic_source"] = {k: traffic[k] for k in (
            "fetch_bytes_per_launch", "write_bytes_per_launch", "traffic_over_alg",
            "fetch_scale", "write_scale")}
        extra["traffic_source"]["file"] = os.path.relpath(TRAFFIC_FILE, ROOT)
    line = {
        "metric": METRIC,
        "value": round(c2["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(c2["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic N(0,1), seeded, generated on device",
        "config": {
            "workload": "C2 GQA decode, uniform 8192-row fp16 cache, 16 seqs, 32q/8kv heads, "
                        "head_dim 128, ROCm layout [8192,16,8,128], split-K + combine",
            "batch": 16, "ctx": 8192, "q_heads": 32, "kv_heads": 8, "head_dim": 128,
            "frac_of_hbm_peak": round(c2["gbs"] / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "kernel": "decode_split_mfma<f16,128>",
            "bound": "hbm",
            "achieved": round(c2["split_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(c2["split_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic["traffic_bytes_per_launch"] if traffic else None,
            "avg_launch_ms": round(c2["split_ms"], 5),
            "alg_bytes_per_launch": c2["split_alg_bytes"],
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
