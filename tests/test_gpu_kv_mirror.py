"""GPU tests of ``kernels.DeviceKVMirror``: the NumPy-facing llama decode
drop-in (kernels.attention_decode, kernels.py:1183-1200) keeping the host
cache rows on the device between calls (the reference's device tier,
cuda.py:1881-1900).

A decode loop over a growing host cache -- a bulk prefill, then one row per
token -- must give the two-pass NumPy oracle's output (model.py:1246-1252)
to 1e-4 on every token (fp32 cache; 2e-2 for an fp16 host cache), also after
host rows are rewritten and reported with ``invalidate`` and after the host
cache is cut back and regrown.
"""

import importlib

import numpy as np
import pytest

from oracle import attention as A

pytestmark = pytest.mark.gpu


def _kernels():
    return importlib.import_module("alpacca-open-sourced-by-jt_amd.kernels")


def _check(kern, mirror, rng, K, V, t, group, n_kv, hd, tol):
    q = rng.standard_normal(n_kv * group * hd).astype(np.float32)
    inv = 1.0 / np.sqrt(hd)
    got = kern.attention_decode(q, K[:t], V[:t], group, inv, mirror=mirror)
    qq = q.astype(K.dtype).astype(np.float32)  # the query in the cache dtype
    ref = A.attention_decode_twopass(qq, K[:t].astype(np.float32), V[:t].astype(np.float32),
                                     group, inv)
    assert got.shape == (n_kv * group, hd)
    err = float(np.abs(got - ref).max())
    assert err <= tol, (t, err)


@pytest.mark.parametrize("dtype,tol", [(np.float32, 1e-4), (np.float16, 2e-2)])
def test_mirror_decode_loop_matches_oracle(gpu, dtype, tol):
    kern = _kernels()
    rng = np.random.default_rng(21)
    cap, n_kv, hd, group = 1024, 8, 128, 4
    print(f"kv mirror loop: cap={cap} n_kv={n_kv} hd={hd} group={group} {np.dtype(dtype)}",
          flush=True)
    K = np.zeros((cap, n_kv, hd), dtype=dtype)
    V = np.zeros((cap, n_kv, hd), dtype=dtype)
    mirror = kern.DeviceKVMirror(cap, n_kv, hd, dtype=dtype)
    t = 300  # prefill rows: one bulk upload, then one row per token
    K[:t] = rng.standard_normal((t, n_kv, hd))
    V[:t] = rng.standard_normal((t, n_kv, hd))
    _check(kern, mirror, rng, K, V, t, group, n_kv, hd, tol)
    for _ in range(12):
        K[t] = rng.standard_normal((n_kv, hd))
        V[t] = rng.standard_normal((n_kv, hd))
        t += 1
        _check(kern, mirror, rng, K, V, t, group, n_kv, hd, tol)
    assert mirror.valid_upto == t
    # rewrite rows 100.. on the host and report it
    K[100:t] = rng.standard_normal((t - 100, n_kv, hd))
    V[100:t] = rng.standard_normal((t - 100, n_kv, hd))
    mirror.invalidate(100)
    _check(kern, mirror, rng, K, V, t, group, n_kv, hd, tol)
    # cut the host cache back to 200 rows and grow it with new rows
    t = 200
    _check(kern, mirror, rng, K, V, t, group, n_kv, hd, tol)
    for _ in range(3):
        K[t] = rng.standard_normal((n_kv, hd))
        V[t] = rng.standard_normal((n_kv, hd))
        t += 1
        _check(kern, mirror, rng, K, V, t, group, n_kv, hd, tol)
    # one row at the very end of the capacity
    K[:cap] = rng.standard_normal((cap, n_kv, hd))
    V[:cap] = rng.standard_normal((cap, n_kv, hd))
    mirror.invalidate(0)
    _check(kern, mirror, rng, K, V, cap, group, n_kv, hd, tol)


def test_mirror_rejects_bad_calls(gpu):
    kern = _kernels()
    mirror = kern.DeviceKVMirror(16, 2, 64)
    K = np.zeros((17, 2, 64), np.float32)
    q = np.zeros(4 * 64, np.float32)
    with pytest.raises(ValueError, match="capacity"):
        kern.attention_decode(q, K, K, 2, 0.125, mirror=mirror)
    with pytest.raises(ValueError, match="matching the mirror"):
        kern.attention_decode(q, K[:4, :1], K[:4, :1], 2, 0.125, mirror=mirror)


def _random_mirror_cases(n=8):
    rng = np.random.default_rng(9990)
    pick = lambda vals: vals[int(rng.integers(len(vals)))]  # noqa: E731
    return [dict(seed=9990 + i, dtype=pick(["f32", "f32", "f16"]), cap=int(rng.integers(32, 1500)),
                 n_kv=int(rng.integers(1, 9)), hd=pick([32, 64, 80, 128, 256]),
                 group=pick([1, 2, 4, 5, 8]), ops=int(rng.integers(10, 25)))
            for i in range(n)]


MIRROR_CASES = _random_mirror_cases()


@pytest.mark.parametrize("c", MIRROR_CASES, ids=[
    f"mirror{i}-{c['dtype']}-cap{c['cap']}-kv{c['n_kv']}x{c['group']}-hd{c['hd']}-ops{c['ops']}"
    for i, c in enumerate(MIRROR_CASES)])
def test_random_mirror_operation_sequences(gpu, c):
    """Seeded random sequences of host-cache operations through one mirror
    -- bulk growth (a prefill), single-token growth, host rewrites reported
    with ``invalidate``, cut-backs and regrowth, and a second query group
    size on the same mirror -- each followed by a decode checked against the
    two-pass oracle on the host rows (1e-4 fp32, 2e-2 fp16 caches)."""
    kern = _kernels()
    rng = np.random.default_rng(c["seed"])
    dtype = np.float16 if c["dtype"] == "f16" else np.float32
    tol = 2e-2 if c["dtype"] == "f16" else 1e-4
    cap, n_kv, hd, group = c["cap"], c["n_kv"], c["hd"], c["group"]
    print(f"random mirror: {c}", flush=True)
    K = np.zeros((cap, n_kv, hd), dtype=dtype)
    V = np.zeros((cap, n_kv, hd), dtype=dtype)
    mirror = kern.DeviceKVMirror(cap, n_kv, hd, dtype=dtype)
    t = 0
    for _ in range(c["ops"]):
        op = rng.integers(5) if t > 0 else 0
        if op == 0 and t < cap:          # bulk growth
            n = int(rng.integers(1, min(200, cap - t) + 1))
            K[t:t + n] = rng.standard_normal((n, n_kv, hd))
            V[t:t + n] = rng.standard_normal((n, n_kv, hd))
            t += n
        elif op == 1 and t < cap:        # one token
            K[t] = rng.standard_normal((n_kv, hd))
            V[t] = rng.standard_normal((n_kv, hd))
            t += 1
        elif op == 2:                    # host rewrite from pos, reported
            pos = int(rng.integers(0, t))
            K[pos:t] = rng.standard_normal((t - pos, n_kv, hd))
            V[pos:t] = rng.standard_normal((t - pos, n_kv, hd))
            mirror.invalidate(pos)
        elif op == 3:                    # cut back (rows past t rewritten on regrowth)
            t = int(rng.integers(1, t + 1))
        g = group if rng.random() < 0.8 else 1  # a second group size on the same mirror
        _check(kern, mirror, rng, K, V, t, g, n_kv, hd, tol)
