"""GPU parity over seeded random geometry: decode (contiguous and paged),
causal prefill (rows in the cache, and append + prefill in one call) and the
chunked GDN, each against the oracle.

The fixed-shape tests pin the BASELINE configurations and the edge cases
one by one; these draw the shape of every call from a fixed seed -- dtype,
head dims (the MFMA widths 64 / 128 / 256 and widths that take the generic
kernels), GQA group, batch, cache capacity and length, ragged lengths, the
fused gate, windows, custom scales, output dtype, page size, chunk
remainders, nonzero GDN states -- so that plan choices (one round, several
rounds, skew, balanced, split-K fallback, paired or single prefill, token-
sequential GDN) meet shapes nobody picked by hand.  Every case is named in
its test id and printed before its GPU call.  Bars: fp32 1e-4; fp16 / bf16
2e-2; GDN state 1e-4 against fp64; KV rows and paged-vs-contiguous outputs
bit for bit.
"""

import importlib
import math

import numpy as np
import pytest

from oracle import attention as A
from oracle import gdn as G
from oracle import inputs as I

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "f16": 2e-2, "bf16": 2e-2}


def _mod(name):
    return importlib.import_module("alpacca-open-sourced-by-jt_amd." + name)


@pytest.fixture(scope="module")
def ops(gpu):
    return _mod("qwen35_rocm_ops").Qwen35RocmOps()


def _td(torch, name):
    return {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[name]


def _dev(torch, arr, dtype, device):
    # values are already rounded to dtype, so the cast is exact
    return torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float32)).to(device).to(
        _td(torch, dtype))


def _normal(rng, shape, dtype):
    return I.round_to(rng.standard_normal(shape), dtype).astype(np.float32)


def _pick(rng, values):
    return values[int(rng.integers(len(values)))]


# ---------------------------------------------------------------- case lists

def _decode_cases(n=64):
    rng = np.random.default_rng(9100)
    cases = []
    for i in range(n):
        dtype = _pick(rng, ["f32", "f16", "bf16", "f16", "bf16"])
        d = _pick(rng, [64, 128, 256, 128, 80, 40])
        dv = d if rng.random() < 0.8 else _pick(rng, [32, 48, 128])
        hkv = int(rng.integers(1, 5))
        group = _pick(rng, [1, 2, 4, 5, 8, 12])
        batch = int(rng.integers(1, 7))
        cap = int(rng.integers(1, 2049 if d == 256 else 3073))
        length = int(rng.integers(max(1, cap // 2), cap + 1))
        c = dict(seed=9100 + i, dtype=dtype, d=d, dv=dv, hkv=hkv, hq=hkv * group, batch=batch,
                 cap=cap, length=length, ragged=bool(rng.random() < 0.5),
                 gated=bool(rng.random() < 0.35),
                 scale=None if rng.random() < 0.7 else round(float(rng.uniform(0.02, 0.25)), 4),
                 out32=bool(dtype != "f32" and rng.random() < 0.3))
        c["id"] = (f"dec{i:02d}-{dtype}-d{d}x{dv}-q{c['hq']}kv{hkv}-B{batch}-L{length}of{cap}"
                   f"{'-ragged' if c['ragged'] else ''}{'-gate' if c['gated'] else ''}"
                   f"{'-s' if c['scale'] else ''}{'-o32' if c['out32'] else ''}")
        cases.append(c)
    return cases


def _paged_cases(n=16):
    rng = np.random.default_rng(9150)
    cases = []
    for i in range(n):
        dtype = _pick(rng, ["f16", "bf16", "f32"])
        d = _pick(rng, [64, 128, 256, 80])
        page = _pick(rng, [32, 64, 128, 256])
        hkv = int(rng.integers(1, 4))
        group = _pick(rng, [1, 4, 8])
        batch = int(rng.integers(1, 5))
        pages = int(rng.integers(1, max(2, 2049 // page)))
        cap = pages * page
        length = int(rng.integers(1, cap + 1))
        c = dict(seed=9150 + i, dtype=dtype, d=d, page=page, hkv=hkv, hq=hkv * group,
                 batch=batch, cap=cap, length=length, gated=bool(rng.random() < 0.3))
        c["id"] = (f"pg{i:02d}-{dtype}-d{d}-p{page}-q{c['hq']}kv{hkv}-B{batch}-L{length}of{cap}"
                   f"{'-gate' if c['gated'] else ''}")
        cases.append(c)
    return cases


def _prefill_cases(n=48):
    rng = np.random.default_rng(9200)
    cases = []
    for i in range(n):
        dtype = _pick(rng, ["bf16", "f16", "bf16", "f16", "f32"])
        d = _pick(rng, [64, 128, 256, 128, 80])
        hkv = int(rng.integers(1, 4 if d == 256 else 5))
        group = _pick(rng, [1, 2, 4, 5, 8])
        tokens = int(rng.integers(1, 401))
        position = int(rng.integers(0, 1501))
        cap = position + tokens + int(rng.integers(0, 65))
        batch = int(rng.integers(1, 4))
        window = 0 if rng.random() < 0.7 else int(rng.integers(1, position + tokens + 1))
        c = dict(seed=9200 + i, dtype=dtype, d=d, hkv=hkv, hq=hkv * group, tokens=tokens,
                 position=position, cap=cap, batch=batch, bi=int(rng.integers(batch)),
                 window=window, gated=bool(rng.random() < 0.3),
                 scale=None if rng.random() < 0.7 else round(float(rng.uniform(0.03, 0.2)), 4))
        c["id"] = (f"pre{i:02d}-{dtype}-d{d}-q{c['hq']}kv{hkv}-T{tokens}at{position}-B{batch}"
                   f"{'-w%d' % window if window else ''}{'-gate' if c['gated'] else ''}"
                   f"{'-s' if c['scale'] else ''}")
        cases.append(c)
    return cases


def _append_cases(n=16):
    rng = np.random.default_rng(9250)
    cases = []
    for i in range(n):
        dtype = _pick(rng, ["bf16", "f16", "f32"])
        d = _pick(rng, [64, 128, 256, 80])
        hkv = int(rng.integers(1, 4))
        group = _pick(rng, [1, 4, 8])
        tokens = int(rng.integers(1, 301))
        position = int(rng.integers(0, 1201))
        c = dict(seed=9250 + i, dtype=dtype, d=d, hkv=hkv, hq=hkv * group, tokens=tokens,
                 position=position, cap=position + tokens + int(rng.integers(0, 33)))
        c["id"] = f"app{i:02d}-{dtype}-d{d}-q{c['hq']}kv{hkv}-T{tokens}at{position}"
        cases.append(c)
    return cases


def _gdn_cases(n=40):
    rng = np.random.default_rng(9300)
    cases = []
    for i in range(n):
        dtype = _pick(rng, ["bf16", "f32", "bf16", "f32", "f16"])
        dk = _pick(rng, [64, 128, 256, 128, 40])
        dv = _pick(rng, [16, 32, 64, 128, 256, 24])
        hk = int(rng.integers(1, 4))
        hv = hk * int(rng.integers(1, 4))
        batch = int(rng.integers(1, 4))
        tokens = int(rng.integers(1, 261))
        tokens = max(1, min(tokens, 3000 // (batch * hv)))
        c = dict(seed=9300 + i, dtype=dtype, dk=dk, dv=dv, hk=hk, hv=hv, batch=batch,
                 tokens=tokens, s0=bool(rng.random() < 0.6))
        c["id"] = (f"gdn{i:02d}-{dtype}-k{dk}v{dv}-hk{hk}hv{hv}-B{batch}-T{tokens}"
                   f"{'-s0' if c['s0'] else ''}")
        cases.append(c)
    return cases


DECODE = _decode_cases()
PAGED = _paged_cases()
PREFILL = _prefill_cases()
APPEND = _append_cases()
GDN = _gdn_cases()


def _err(out, ref):
    return float(np.abs(out.float().cpu().numpy() - ref).max())


# ---------------------------------------------------------------- decode

@pytest.mark.parametrize("c", DECODE, ids=[c["id"] for c in DECODE])
def test_random_decode_against_oracle(gpu, ops, c):
    import torch
    print("random decode:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    dt, B = c["dtype"], c["batch"]
    q = _normal(rng, (B, c["hq"], c["d"]), dt)
    K = _normal(rng, (c["cap"], B, c["hkv"], c["d"]), dt)
    V = _normal(rng, (c["cap"], B, c["hkv"], c["dv"]), dt)
    lens = rng.integers(1, c["length"] + 1, B).astype(np.int32) if c["ragged"] else None
    gate = _normal(rng, (B, c["hq"], c["dv"]), dt) if c["gated"] else None
    out = ops.online_attention(
        _dev(torch, q, dt, gpu), _dev(torch, K, dt, gpu), _dev(torch, V, dt, gpu),
        length=c["length"], scale=c["scale"],
        seq_lens=None if lens is None else torch.from_numpy(lens).to(gpu),
        gate=None if gate is None else _dev(torch, gate, dt, gpu),
        out_dtype=torch.float32 if c["out32"] else None)
    torch.cuda.synchronize()
    ref = A.online_attention(q, K, V, c["length"], scale=c["scale"], seq_lens=lens)
    if gate is not None:
        ref = A.sigmoid_gate(ref, gate)
    assert out.shape == (B, c["hq"], c["dv"])
    assert out.dtype == (torch.float32 if c["out32"] else _td(torch, dt))
    err = _err(out, ref)
    print(f"  max abs error {err:.3g} (bar {TOL[dt]:g})", flush=True)
    assert err <= TOL[dt], (c["id"], err)


@pytest.mark.parametrize("c", PAGED, ids=[c["id"] for c in PAGED])
def test_random_paged_decode_equals_contiguous_and_oracle(gpu, ops, c):
    import torch
    print("random paged decode:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    dt, B, d, page, cap = c["dtype"], c["batch"], c["d"], c["page"], c["cap"]
    td = _td(torch, dt)
    max_pages = cap // page
    num_pages = B * max_pages + 2
    perm = rng.permutation(num_pages)[:B * max_pages].reshape(B, max_pages)
    table = torch.from_numpy(perm.astype(np.int32)).to(gpu)
    K = _normal(rng, (cap, B, c["hkv"], d), dt)
    V = _normal(rng, (cap, B, c["hkv"], d), dt)
    q = _normal(rng, (B, c["hq"], d), dt)
    lens = rng.integers(1, c["length"] + 1, B).astype(np.int32)
    gate = _normal(rng, (B, c["hq"], d), dt) if c["gated"] else None
    Kd, Vd = _dev(torch, K, dt, gpu), _dev(torch, V, dt, gpu)
    pw = ops.initialize_paged_attention_workspace(num_pages=num_pages, page_size=page,
                                                  kv_heads=c["hkv"], key_dimension=d,
                                                  value_dimension=d, dtype=td)
    _mod("_ops").kv_append_paged(pw.key_pages, pw.value_pages, table, Kd, Vd, position=0)
    qd = _dev(torch, q, dt, gpu)
    ld = torch.from_numpy(lens).to(gpu)
    gd = None if gate is None else _dev(torch, gate, dt, gpu)
    got = ops.paged_online_attention(qd, pw.key_pages, pw.value_pages, table, length=c["length"],
                                     seq_lens=ld, gate=gd)
    want = ops.online_attention(qd, Kd, Vd, length=c["length"], seq_lens=ld, gate=gd)
    torch.cuda.synchronize()
    assert torch.equal(got, want), c["id"]
    ref = A.online_attention(q, K, V, c["length"], seq_lens=lens)
    if gate is not None:
        ref = A.sigmoid_gate(ref, gate)
    err = _err(got, ref)
    print(f"  max abs error {err:.3g} (bar {TOL[dt]:g})", flush=True)
    assert err <= TOL[dt], (c["id"], err)


# ---------------------------------------------------------------- prefill

@pytest.mark.parametrize("c", PREFILL, ids=[c["id"] for c in PREFILL])
def test_random_prefill_against_oracle(gpu, ops, c):
    import torch
    print("random prefill:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    dt, d, T, pos = c["dtype"], c["d"], c["tokens"], c["position"]
    K = _normal(rng, (c["cap"], c["batch"], c["hkv"], d), dt)
    V = _normal(rng, (c["cap"], c["batch"], c["hkv"], d), dt)
    q = _normal(rng, (T, c["hq"], d), dt)
    gate = _normal(rng, (T, c["hq"], d), dt) if c["gated"] else None
    out = ops.attention_prefill(_dev(torch, q, dt, gpu), _dev(torch, K, dt, gpu),
                                _dev(torch, V, dt, gpu), position=pos, batch_index=c["bi"],
                                scale=c["scale"], window=c["window"],
                                gate=None if gate is None else _dev(torch, gate, dt, gpu))
    torch.cuda.synchronize()
    scale = c["scale"] if c["scale"] is not None else 1.0 / math.sqrt(d)
    ref = A.attention_batch(q, K[:pos + T, c["bi"]], V[:pos + T, c["bi"]], pos + np.arange(T),
                            c["hq"] // c["hkv"], scale, window=c["window"])
    if gate is not None:
        ref = A.sigmoid_gate(ref, gate)
    assert out.shape == (T, c["hq"], d)
    err = _err(out, ref)
    print(f"  max abs error {err:.3g} (bar {TOL[dt]:g})", flush=True)
    assert err <= TOL[dt], (c["id"], err)


@pytest.mark.parametrize("c", APPEND, ids=[c["id"] for c in APPEND])
def test_random_append_prefill_against_oracle(gpu, ops, c):
    import torch
    print("random append + prefill:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    dt, d, T, pos, hkv = c["dtype"], c["d"], c["tokens"], c["position"], c["hkv"]
    K = _normal(rng, (c["cap"], 1, hkv, d), dt)
    V = _normal(rng, (c["cap"], 1, hkv, d), dt)
    kn = _normal(rng, (T, hkv, d), dt)
    vn = _normal(rng, (T, hkv, d), dt)
    q = _normal(rng, (T, c["hq"], d), dt)
    kc, vc = _dev(torch, K, dt, gpu), _dev(torch, V, dt, gpu)
    out, end = ops.append_prefill_attention_(_dev(torch, q, dt, gpu), _dev(torch, kn, dt, gpu),
                                             _dev(torch, vn, dt, gpu), kc, vc, position=pos)
    torch.cuda.synchronize()
    assert end == pos + T
    K[pos:pos + T, 0], V[pos:pos + T, 0] = kn, vn
    bits = torch.int32 if dt == "f32" else torch.int16
    assert torch.equal(kc.view(bits), _dev(torch, K, dt, gpu).view(bits)), c["id"]
    assert torch.equal(vc.view(bits), _dev(torch, V, dt, gpu).view(bits)), c["id"]
    ref = A.attention_batch(q, K[:pos + T, 0], V[:pos + T, 0], pos + np.arange(T),
                            c["hq"] // hkv, 1.0 / math.sqrt(d))
    err = _err(out, ref)
    print(f"  max abs error {err:.3g} (bar {TOL[dt]:g})", flush=True)
    assert err <= TOL[dt], (c["id"], err)


# ---------------------------------------------------------------- GDN

@pytest.mark.parametrize("c", GDN, ids=[c["id"] for c in GDN])
def test_random_chunked_gdn_against_fp64_scan(gpu, ops, c):
    import torch
    print("random chunked GDN:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])
    dt, B, T, hk, hv, dk, dv = (c["dtype"], c["batch"], c["tokens"], c["hk"], c["hv"], c["dk"],
                                c["dv"])
    q, k = G.normalize_qk(rng.standard_normal((B, T, hk, dk)),
                          rng.standard_normal((B, T, hk, dk)), 1e-6)
    q, k = I.round_to(q, dt).astype(np.float32), I.round_to(k, dt).astype(np.float32)
    v = _normal(rng, (B, T, hv, dv), dt)
    beta = rng.uniform(0, 1, (B, T, hv)).astype(np.float32)
    g = (-np.exp(rng.uniform(-1, 1, hv)) * np.log1p(np.exp(rng.standard_normal((B, T, hv))))
         ).astype(np.float32)
    s0 = ((rng.standard_normal((B, hv, dv, dk)) * 0.3) if c["s0"]
          else np.zeros((B, hv, dv, dk))).astype(np.float32)
    S = torch.from_numpy(s0).to(gpu)
    out = ops.gated_delta_net_chunk_(S, _dev(torch, q, dt, gpu), _dev(torch, k, dt, gpu),
                                     _dev(torch, v, dt, gpu), torch.from_numpy(beta).to(gpu),
                                     torch.from_numpy(g).to(gpu))
    torch.cuda.synchronize()
    assert out.shape == (B, T, hv, dv)
    tol = 1e-4 if dt == "f32" else 2e-2
    for b in range(B):
        ref_state = s0[b].astype(np.float64)
        ref = G.gdn_scan(ref_state, q[b], k[b], v[b], beta[b], g[b])
        err_o = _err(out[b], ref)
        err_s = float(np.abs(S[b].cpu().numpy() - ref_state).max())
        print(f"  sequence {b}: output {err_o:.3g} (bar {tol:g}), state {err_s:.3g} (bar 1e-4)",
              flush=True)
        assert err_o <= tol, (c["id"], b, err_o)
        assert err_s <= 1e-4, (c["id"], b, err_s)
