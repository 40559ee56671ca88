"""GPU parity of the ``qwen35_ops`` list-in / list-out drop-in
(qwen35_ops.py:309-472) against the oracle's scalar fsum restatements.

The device computes in float32 on float32-rounded inputs, so the bar is
the fp32 one: max abs error <= 1e-4.  The drop-in must also leave its
inputs untouched and return fresh Python lists.
"""

import copy
import importlib
import math

import numpy as np
import pytest

from oracle import attention as A
from oracle import gdn as G

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def q35(gpu):
    return importlib.import_module("alpacca-open-sourced-by-jt_amd.qwen35_ops")


def _worst(a, b):
    return float(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64)).max())


def _f32_lists(arr):
    return np.asarray(arr, dtype=np.float32).astype(np.float64).tolist()


@pytest.mark.parametrize("dv,dk", [(128, 128), (16, 24), (3, 5)])
def test_gated_delta_net_step(q35, dv, dk):
    rng = np.random.default_rng(dv * 100 + dk)
    state = _f32_lists(rng.standard_normal((dv, dk)) * 0.3)
    q = rng.standard_normal(dk)
    k = rng.standard_normal(dk)
    q, k = _f32_lists(q / np.linalg.norm(q)), _f32_lists(k / np.linalg.norm(k))
    v = _f32_lists(rng.standard_normal(dv))
    beta, log_decay = float(np.float32(0.7)), float(np.float32(-0.2))
    before = copy.deepcopy((state, q, k, v))
    out, new = q35.gated_delta_net_step(state, q, k, v, beta=beta, log_decay=log_decay)
    assert (state, q, k, v) == before  # inputs not mutated
    assert isinstance(out, list) and isinstance(new, list) and isinstance(new[0], list)
    assert len(out) == dv and len(new) == dv and len(new[0]) == dk
    ref_out, ref_new = G.gdn_step_scalar(state, q, k, v, beta, log_decay)
    assert _worst(out, ref_out) <= TOL
    assert _worst(new, ref_new) <= TOL


def test_gated_delta_net_scan(q35):
    rng = np.random.default_rng(5)
    dv, dk, t = 32, 64, 40
    state = _f32_lists(rng.standard_normal((dv, dk)) * 0.1)
    qs = rng.standard_normal((t, dk))
    ks = rng.standard_normal((t, dk))
    qs = _f32_lists(qs / np.linalg.norm(qs, axis=1, keepdims=True))
    ks = _f32_lists(ks / np.linalg.norm(ks, axis=1, keepdims=True))
    vs = _f32_lists(rng.standard_normal((t, dv)))
    betas = _f32_lists(1.0 / (1.0 + np.exp(-rng.standard_normal(t))))
    gs = _f32_lists(-np.exp(rng.uniform(-1, 1, t)) * np.log1p(np.exp(rng.standard_normal(t))))
    before = copy.deepcopy(state)
    outs, final = q35.gated_delta_net_scan(state, qs, ks, vs, betas, gs)
    assert state == before
    assert len(outs) == t and len(outs[0]) == dv
    ref = state
    worst = 0.0
    for i in range(t):
        o, ref = G.gdn_step_scalar(ref, qs[i], ks[i], vs[i], betas[i], gs[i])
        worst = max(worst, _worst(outs[i], o))
    assert worst <= TOL
    assert _worst(final, ref) <= TOL
    # an empty chunk returns the state unchanged
    outs0, same = q35.gated_delta_net_scan(state, [], [], [], [], [])
    assert outs0 == [] and same == state


@pytest.mark.parametrize("hq,hkv,d,dv,t", [(32, 8, 64, 64, 50), (6, 2, 5, 3, 7), (4, 4, 16, 8, 1)])
def test_causal_gqa_step(q35, hq, hkv, d, dv, t):
    rng = np.random.default_rng(hq * 7 + t)
    q = _f32_lists(rng.standard_normal((hq, d)))
    K = _f32_lists(rng.standard_normal((t, hkv, d)))
    V = _f32_lists(rng.standard_normal((t, hkv, dv)))
    before = copy.deepcopy((q, K, V))
    out = q35.causal_gqa_step(q, K, V)
    assert (q, K, V) == before
    assert len(out) == hq and len(out[0]) == dv
    assert _worst(out, A.causal_gqa_step_scalar(q, K, V)) <= TOL
    out2 = q35.causal_gqa_step(q, K, V, scale=0.3)
    assert _worst(out2, A.causal_gqa_step_scalar(q, K, V, scale=0.3)) <= TOL


def test_causal_gqa_step_one_token_returns_its_value_row(q35):
    """A one-row cache gives every query head exactly its KV head's value
    row (softmax over one key is 1), whatever the scores."""
    rng = np.random.default_rng(1)
    q = _f32_lists(rng.standard_normal((8, 32)) * 50)
    K = _f32_lists(rng.standard_normal((1, 2, 32)))
    V = _f32_lists(rng.standard_normal((1, 2, 16)))
    out = q35.causal_gqa_step(q, K, V)
    for h in range(8):
        assert _worst(out[h], V[0][h // 4]) <= 1e-6
    assert all(math.isfinite(x) for row in out for x in row)


# ------------------------------------------------ seeded random geometry

def _random_q35_cases():
    rng = np.random.default_rng(9900)
    pick = lambda vals: vals[int(rng.integers(len(vals)))]  # noqa: E731
    steps = [dict(kind="step", seed=9900 + i, dv=int(rng.integers(1, 129)),
                  dk=int(rng.integers(1, 129))) for i in range(10)]
    scans = [dict(kind="scan", seed=9920 + i, dv=pick([8, 24, 32, 64]),
                  dk=pick([64, 128, 40, 7]), t=int(rng.integers(0, 81))) for i in range(8)]
    gqas = []
    for i in range(10):
        hkv = int(rng.integers(1, 5))
        gqas.append(dict(kind="gqa", seed=9940 + i, hkv=hkv, hq=hkv * pick([1, 2, 4, 5]),
                         d=pick([3, 16, 64, 100, 128]), dv=pick([5, 16, 64, 128]),
                         t=int(rng.integers(1, 301)), scale=pick([None, 0.05, 0.3])))
    for c in steps + scans + gqas:
        c["id"] = "-".join([c["kind"]] + [f"{k}{v}" for k, v in c.items()
                                          if k not in ("seed", "kind")])
    return steps + scans + gqas


Q35_CASES = _random_q35_cases()


@pytest.mark.parametrize("c", Q35_CASES, ids=[c["id"] for c in Q35_CASES])
def test_random_list_adapters_against_scalar_oracle(q35, c):
    """Seeded random sizes of the three list adapters (GDN step, GDN scan --
    chunked kernels where the key width allows, token by token otherwise --
    and the causal GQA step with and without a custom scale) against the
    oracle's scalar fsum forms at the fp32 bar; inputs untouched."""
    print("random qwen35_ops:", c["id"], flush=True)
    rng = np.random.default_rng(c["seed"])

    def unit_rows(n, d):
        x = rng.standard_normal((n, d))
        return _f32_lists(x / np.linalg.norm(x, axis=1, keepdims=True))

    if c["kind"] == "step":
        dv, dk = c["dv"], c["dk"]
        state = _f32_lists(rng.standard_normal((dv, dk)) * 0.3)
        q, k = unit_rows(1, dk)[0], unit_rows(1, dk)[0]
        v = _f32_lists(rng.standard_normal(dv))
        beta = float(np.float32(rng.uniform(0, 1)))
        g = float(np.float32(-rng.uniform(0, 1.5)))
        before = copy.deepcopy((state, q, k, v))
        out, new = q35.gated_delta_net_step(state, q, k, v, beta=beta, log_decay=g)
        assert (state, q, k, v) == before
        ref_out, ref_new = G.gdn_step_scalar(state, q, k, v, beta, g)
        assert _worst(out, ref_out) <= TOL and _worst(new, ref_new) <= TOL
    elif c["kind"] == "scan":
        dv, dk, t = c["dv"], c["dk"], c["t"]
        state = _f32_lists(rng.standard_normal((dv, dk)) * 0.2)
        qs, ks = unit_rows(t, dk), unit_rows(t, dk)
        vs = _f32_lists(rng.standard_normal((t, dv)))
        betas = _f32_lists(rng.uniform(0, 1, t))
        gs = _f32_lists(-np.exp(rng.uniform(-1, 1, t)) * np.log1p(np.exp(rng.standard_normal(t))))
        before = copy.deepcopy(state)
        outs, final = q35.gated_delta_net_scan(state, qs, ks, vs, betas, gs)
        assert state == before and len(outs) == t
        ref, worst = state, 0.0
        for i in range(t):
            o, ref = G.gdn_step_scalar(ref, qs[i], ks[i], vs[i], betas[i], gs[i])
            worst = max(worst, _worst(outs[i], o))
        assert worst <= TOL and _worst(final, ref) <= TOL
    else:
        q = _f32_lists(rng.standard_normal((c["hq"], c["d"])))
        K = _f32_lists(rng.standard_normal((c["t"], c["hkv"], c["d"])))
        V = _f32_lists(rng.standard_normal((c["t"], c["hkv"], c["dv"])))
        before = copy.deepcopy((q, K, V))
        out = q35.causal_gqa_step(q, K, V, scale=c["scale"])
        assert (q, K, V) == before
        assert _worst(out, A.causal_gqa_step_scalar(q, K, V, scale=c["scale"])) <= TOL
