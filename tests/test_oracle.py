"""Pins the CPU oracle with closed forms, invariants and special cases.

The reference ships no tests or golden vectors for this path, so each
oracle function is checked here against facts that mathematics fixes.
Every test names the plausible mistake it catches.  No GPU is needed.
"""

import math

import numpy as np
import pytest

from oracle import attention as A
from oracle import gdn as G
from oracle import inputs as I
from oracle import rope as R


def _rng(seed=0):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ decode

def test_decode_length_one_returns_value_row():
    # softmax over one key is 1: catches a missing normalisation / wrong V row
    rng = _rng(1)
    q = rng.standard_normal((8, 16))
    K = rng.standard_normal((1, 2, 16))
    V = rng.standard_normal((1, 2, 16))
    out = A.attention_decode_twopass(q, K, V, 4, 0.25)
    np.testing.assert_allclose(out[:4], np.repeat(V[0, 0:1], 4, 0), atol=1e-14)
    np.testing.assert_allclose(out[4:], np.repeat(V[0, 1:2], 4, 0), atol=1e-14)


def test_decode_gqa_contiguous_head_map():
    # kv head j holds constant V rows c_j: head h must return c_{h // group};
    # catches the modulo map (h % n_kv) that GDN uses instead
    rng = _rng(2)
    n_head, n_kv, hd, t = 8, 4, 8, 5
    q = rng.standard_normal((n_head, hd))
    K = rng.standard_normal((t, n_kv, hd))
    V = np.zeros((t, n_kv, hd))
    for j in range(n_kv):
        V[:, j, :] = 10.0 * j + 1.0
    out = A.attention_decode_twopass(q, K, V, n_head // n_kv, 0.3)
    for h in range(n_head):
        np.testing.assert_allclose(out[h], 10.0 * (h // 2) + 1.0, atol=1e-12)


def test_decode_two_keys_sigmoid_closed_form_pins_scale():
    # two keys: weight of key 0 is sigmoid((s0 - s1) * scale); catches a
    # missing or squared 1/sqrt(d) scale and swapped weights
    d = 64
    q = np.zeros((1, d)); q[0, 0] = 3.0
    K = np.zeros((2, 1, d)); K[0, 0, 0] = 2.0; K[1, 0, 0] = -1.0
    V = np.zeros((2, 1, d)); V[0, 0, :] = 1.0; V[1, 0, :] = -2.0
    scale = 1.0 / math.sqrt(d)
    w0 = 1.0 / (1.0 + math.exp(-(6.0 - (-3.0)) * scale))
    expect = w0 * 1.0 + (1.0 - w0) * (-2.0)
    for fn in (lambda: A.attention_decode_twopass(q, K, V, 1, scale),
               lambda: A.full_attention_decode_online(q, K, V)):
        np.testing.assert_allclose(fn()[0], expect, atol=1e-13)


def test_decode_equal_keys_give_mean_value():
    rng = _rng(3)
    K = np.repeat(rng.standard_normal((1, 2, 8)), 7, axis=0)
    V = rng.standard_normal((7, 2, 8))
    q = rng.standard_normal((4, 8))
    out = A.attention_decode_twopass(q, K, V, 2, 0.5)
    np.testing.assert_allclose(out[0], V[:, 0].mean(0), atol=1e-13)
    np.testing.assert_allclose(out[3], V[:, 1].mean(0), atol=1e-13)


def test_decode_shift_and_permutation_invariance():
    # adding u with q.u const shifts every score equally (no-op); permuting
    # positions is a no-op: catches position-dependent indexing errors
    rng = _rng(4)
    q = rng.standard_normal((2, 6))
    K = rng.standard_normal((9, 1, 6))
    V = rng.standard_normal((9, 1, 6))
    base = A.attention_decode_twopass(q, K, V, 2, 0.4)
    perm = rng.permutation(9)
    np.testing.assert_allclose(
        A.attention_decode_twopass(q, K[perm], V[perm], 2, 0.4), base, atol=1e-12)
    # u orthogonal to both query heads -> every score unchanged
    u = rng.standard_normal(6)
    qq = q.T
    u -= qq @ np.linalg.lstsq(qq, u, rcond=None)[0]
    np.testing.assert_allclose(
        A.attention_decode_twopass(q, K + u, V, 2, 0.4), base, atol=1e-12)


def test_decode_online_equals_twopass_and_scalar():
    # three independently written forms (online loop, two-pass matmul,
    # exact fsum scalar loops) agree on random data
    rng = _rng(5)
    q = rng.standard_normal((6, 8))
    K = rng.standard_normal((11, 3, 8))
    V = rng.standard_normal((11, 3, 5))
    a = A.attention_decode_twopass(q, K, V, 2, 1 / math.sqrt(8))
    b = A.full_attention_decode_online(q, K, V)
    c = np.array(A.causal_gqa_step_scalar(q, K.tolist(), V.tolist()))
    np.testing.assert_allclose(a, b, atol=1e-12)
    np.testing.assert_allclose(a, c, atol=1e-12)


def test_decode_huge_score_selects_row():
    q = np.zeros((1, 4)); q[0, 1] = 100.0
    K = np.zeros((5, 1, 4)); K[3, 0, 1] = 100.0
    V = np.arange(20, dtype=float).reshape(5, 1, 4)
    out = A.attention_decode_twopass(q, K, V, 1, 1.0)
    np.testing.assert_allclose(out[0], V[3, 0], atol=1e-12)


def test_online_attention_ragged_lengths():
    # sequence b must read only its first seq_lens[b] rows: rows past the
    # length hold huge values that would dominate if read
    rng = _rng(6)
    C, B, Hkv, D = 10, 3, 2, 4
    Kc = rng.standard_normal((C, B, Hkv, D))
    Vc = rng.standard_normal((C, B, Hkv, D))
    lens = np.array([3, 10, 1])
    for b, n in enumerate(lens):
        Vc[n:, b] = 1e6
    q = rng.standard_normal((B, 4, D))
    out = A.online_attention(q, Kc, Vc, length=C, seq_lens=lens)
    assert np.abs(out).max() < 100
    np.testing.assert_allclose(out[2], np.repeat(Vc[0, 2], 2, axis=0), atol=1e-12)


# ------------------------------------------------------------------ prefill

@pytest.mark.parametrize("prefix", [0, 5])
def test_prefill_row_sees_exactly_prefix_plus_one_keys(prefix):
    # equal keys + one-hot values: row t averages the first prefix+t+1 rows;
    # catches the off-by-one (< vs <=) causal mask
    t_q, n_kv, group, hd = 6, 2, 2, 16
    total = prefix + t_q
    K = np.ones((total, n_kv, hd))
    V = np.zeros((total, n_kv, hd))
    for j in range(total):
        V[j, :, j] = 1.0
    q = _rng(7).standard_normal((t_q, n_kv * group, hd))
    out = A.full_attention_prefill(q, K, V, prefix_length=prefix)
    for t in range(t_q):
        n = prefix + t + 1
        expect = np.zeros(hd); expect[:n] = 1.0 / n
        np.testing.assert_allclose(out[t, 0], expect, atol=1e-13)
        np.testing.assert_allclose(out[t, 3], expect, atol=1e-13)


def test_prefill_last_row_equals_decode_and_rows_match_truncated_decode():
    rng = _rng(8)
    prefix, t_q, n_kv, group, hd = 4, 5, 2, 3, 8
    K = rng.standard_normal((prefix + t_q, n_kv, hd))
    V = rng.standard_normal((prefix + t_q, n_kv, hd))
    q = rng.standard_normal((t_q, n_kv * group, hd))
    out = A.full_attention_prefill(q, K, V, prefix)
    for t in range(t_q):
        n = prefix + t + 1
        dec = A.full_attention_decode_online(q[t], K[:n], V[:n])
        np.testing.assert_allclose(out[t], dec, atol=1e-12)


def test_prefill_window_and_kv_start():
    # window w: row at position p sees keys p-w+1..p; kv_start shifts key
    # positions; a row with no visible key returns zeros
    rng = _rng(9)
    K = np.ones((8, 1, 4))
    V = np.zeros((8, 1, 8))
    for j in range(8):
        V[j, 0, j] = 1.0
    q = rng.standard_normal((3, 1, 4))
    out = A.attention_batch(q, K, V, np.array([5, 7, 1]), 1, 0.5, window=3,
                            kv_start=2)
    # key j has position j+2. Row p=5 sees positions 3,4,5 -> j=1,2,3
    np.testing.assert_allclose(out[0, 0], np.eye(8)[[1, 2, 3]].mean(0), atol=1e-13)
    np.testing.assert_allclose(out[1, 0], np.eye(8)[[3, 4, 5]].mean(0), atol=1e-13)
    np.testing.assert_allclose(out[2, 0], 0.0)


# ------------------------------------------------------------------ append

def test_append_bit_exact_and_untouched_rows():
    rng = _rng(10)
    kc = rng.standard_normal((6, 2, 3, 4)).astype(np.float32)
    vc = rng.standard_normal((6, 2, 3, 5)).astype(np.float32)
    before_k, before_v = kc.copy(), vc.copy()
    k = rng.standard_normal((2, 3, 4)).astype(np.float32)
    v = rng.standard_normal((2, 3, 5)).astype(np.float32)
    assert A.attention_append(kc, vc, 4, k, v) == 5
    assert np.array_equal(kc[4].view(np.uint32), k.view(np.uint32))
    assert np.array_equal(vc[4].view(np.uint32), v.view(np.uint32))
    mask = np.ones(6, bool); mask[4] = False
    assert np.array_equal(kc[mask], before_k[mask])
    assert np.array_equal(vc[mask], before_v[mask])
    with pytest.raises(ValueError, match="exceeds capacity"):
        A.attention_append(kc, vc, 6, k, v)
    with pytest.raises(ValueError, match="does not match cache token shape"):
        A.attention_append(kc, vc, 1, k[:, :2], v)


def test_ragged_append_positions():
    kc = np.zeros((8, 2, 1, 2)); vc = np.zeros((8, 2, 1, 2))
    k = np.arange(12, dtype=float).reshape(3, 2, 1, 2)
    A.ragged_append(kc, vc, [1, 4], k, -k)
    assert np.array_equal(kc[1:4, 0], k[:, 0]) and np.array_equal(kc[4:7, 1], k[:, 1])
    assert not kc[[0, 4, 5, 6, 7], 0].any() and not kc[[0, 1, 2, 3, 7], 1].any()
    with pytest.raises(ValueError):
        A.ragged_append(kc, vc, [6, 0], k, k)


# ------------------------------------------------------------------ gate

def test_sigmoid_gate_closed_forms():
    g = np.array([0.0, 1000.0, -1000.0, 2.0, -2.0])
    s = A.stable_sigmoid(g)
    assert s[0] == 0.5 and s[1] == 1.0 and s[2] == 0.0
    np.testing.assert_allclose(s[3] + s[4], 1.0, atol=1e-15)
    np.testing.assert_allclose(s[3], 1 / (1 + math.exp(-2.0)), atol=1e-15)
    np.testing.assert_allclose(A.sigmoid_gate(np.full(5, 3.0), g), 3.0 * s)


# ------------------------------------------------------------------ GDN

def _gdn_inputs(rng, hv=4, hk=2, dv=6, dk=5):
    state = rng.standard_normal((hv, dv, dk))
    q = rng.standard_normal((hk, dk))
    k = rng.standard_normal((hk, dk))
    v = rng.standard_normal((hv, dv))
    beta = rng.uniform(0, 1, hv)
    g = -rng.uniform(0, 2, hv)
    return state, q, k, v, beta, g


def test_gdn_beta_zero_is_pure_decay():
    rng = _rng(11)
    state, q, k, v, beta, g = _gdn_inputs(rng)
    s0 = state.copy()
    out = G.gdn_step(state, q, k, v, np.zeros(4), g)
    for h in range(4):
        np.testing.assert_allclose(state[h], math.exp(g[h]) * s0[h], atol=1e-13)
        np.testing.assert_allclose(out[h], state[h] @ q[h % 2] / math.sqrt(5), atol=1e-13)


def test_gdn_unit_beta_orthonormal_key_overwrites_memory():
    # g = 0, beta = 1, ||k|| = 1: after the update S k == v exactly (delta
    # rule writes v under key k); catches a sign error in (v - S k)
    rng = _rng(12)
    state, q, k, v, beta, g = _gdn_inputs(rng)
    k = np.linalg.qr(rng.standard_normal((5, 5)))[0][:2]
    G.gdn_step(state, q, k, v, np.ones(4), np.zeros(4))
    for h in range(4):
        np.testing.assert_allclose(state[h] @ k[h % 2], v[h], atol=1e-12)


def test_gdn_rank_one_from_zero_state_and_modulo_head_map():
    # from S = 0: S = beta v k^T and o = beta v (k . q) / sqrt(dk), with
    # value head h reading key head h % Hk (not h // group)
    rng = _rng(13)
    _, q, k, v, beta, g = _gdn_inputs(rng)
    state = np.zeros((4, 6, 5))
    out = G.gdn_step(state, q, k, v, beta, g)
    for h in range(4):
        kh = h % 2
        np.testing.assert_allclose(state[h], beta[h] * np.outer(v[h], k[kh]), atol=1e-13)
        np.testing.assert_allclose(
            out[h], beta[h] * v[h] * (k[kh] @ q[kh]) / math.sqrt(5), atol=1e-13)
    assert G.key_head_for_value_head(5, 2) == 1


def test_gdn_vectorised_equals_scalar_reference_form():
    rng = _rng(14)
    state, q, k, v, beta, g = _gdn_inputs(rng)
    s_vec = state.copy()
    out = G.gdn_step(s_vec, q, k, v, beta, g)
    for h in range(4):
        o, new = G.gdn_step_scalar(state[h].tolist(), q[h % 2], k[h % 2], v[h],
                                   beta[h], g[h])
        np.testing.assert_allclose(out[h], o, atol=1e-12)
        np.testing.assert_allclose(s_vec[h], np.array(new), atol=1e-12)
    with pytest.raises(ValueError):
        G.gdn_step_scalar(state[0].tolist(), q[0], k[0], v[0], 1.5, -0.1)
    with pytest.raises(ValueError):
        G.gdn_step_scalar(state[0].tolist(), q[0], k[0], v[0], 0.5, 0.1)


def test_gdn_scan_composes_steps():
    rng = _rng(15)
    T = 4
    state = rng.standard_normal((2, 3, 3))
    qs = rng.standard_normal((T, 1, 3)); ks = rng.standard_normal((T, 1, 3))
    vs = rng.standard_normal((T, 2, 3))
    bs = rng.uniform(0, 1, (T, 2)); gs = -rng.uniform(0, 1, (T, 2))
    s1 = state.copy()
    outs = G.gdn_scan(s1, qs, ks, vs, bs, gs)
    s2 = state.copy()
    for t in range(T):
        np.testing.assert_allclose(outs[t], G.gdn_step(s2, qs[t], ks[t], vs[t], bs[t], gs[t]))
    np.testing.assert_allclose(s1, s2)


def test_gdn_prep_closed_forms():
    q = np.array([[3.0, 4.0], [0.0, 0.0]])
    qn, kn = G.normalize_qk(q, q, 1e-6)
    np.testing.assert_allclose(qn[0], [0.6, 0.8], atol=1e-7)
    assert np.all(qn[1] == 0.0)
    beta, g = G.beta_decay(np.array([0.0, 50.0, -50.0]), np.array([0.0, 30.0, -30.0]),
                           np.zeros(3), np.array([-1.0, -2.0, -0.5]))
    np.testing.assert_allclose(beta, [0.5, 1.0, math.exp(-50.0)], rtol=1e-6)
    np.testing.assert_allclose(g, [-math.log(2.0), -60.0, -0.5 * math.log1p(math.exp(-30.0))],
                               rtol=1e-6)


# ------------------------------------------------------------------ helpers

def test_bf16_rounding_is_rne_and_exact():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 1e-40, np.inf],
                 dtype=np.float32)
    r = I.round_to(x, "bf16")
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7 -> even (1.0);
    # 1 + 3*2^-8 ties between 1+2^-7 and 1+2^-6 -> even (1 + 2^-6)
    assert r[0] == 1.0 and r[1] == 1.0 and r[2] == 1.0 + 2 ** -6
    assert r[3] == -2.5 and r[5] == np.inf
    assert np.array_equal(I.round_to(r, "bf16"), r)


def test_rope_rotation_properties():
    cos, sin = R.rope_tables(16, 8, 500000.0)
    v = _rng(16).standard_normal((3, 2, 8)).astype(np.float32)
    out = R.rope_norm_batch(v, np.array([0, 5, 15]), cos, sin)
    np.testing.assert_allclose(out[0], v[0], atol=0)  # position 0 is identity
    np.testing.assert_allclose(np.linalg.norm(out, axis=-1),
                               np.linalg.norm(v, axis=-1), rtol=1e-5)
    # pair 0 rotates by angle = position (inv_freq[0] = 1)
    a, b = v[1, 0, 0], v[1, 0, 1]
    np.testing.assert_allclose(out[1, 0, 0], a * math.cos(5) - b * math.sin(5), rtol=1e-5)


def test_config_generators_small():
    c1 = I.c1_decode_fp32(ctx=16)
    assert c1["q"].shape == (32, 64) and c1["K"].shape == (16, 8, 64)
    c2 = I.c2_decode_fp16(batch=3, capacity=64, lo=8, hi=64)
    assert c2["K"].shape == (64, 3, 8, 128) and np.all(c2["seq_lens"] <= 64)
    assert np.array_equal(c2["K"], c2["K"].astype(np.float16).astype(np.float32))
    c5 = I.c5_gdn_bf16(tokens=4)
    np.testing.assert_allclose(np.linalg.norm(c5["q"], axis=-1), 1.0, atol=1e-2)
    assert np.all(c5["g"] <= 0) and np.all((c5["beta"] > 0) & (c5["beta"] < 1))


def test_paged_rows_gather_through_the_block_table():
    # identity table = contiguous slicing; a shuffled table reorders pages;
    # rows cross a page boundary at multiples of the page size
    rng = np.random.default_rng(4)
    size, hkv, d = 4, 2, 3
    pages = rng.standard_normal((6, size, hkv, d))
    ident = np.array([[0, 1, 2], [3, 4, 5]])
    np.testing.assert_array_equal(A.paged_rows(pages, ident, 0, 10),
                                  pages[:3].reshape(12, hkv, d)[:10])
    table = np.array([[5, 0, 3], [1, 2, 4]])
    got = A.paged_rows(pages, table, 0, 9)
    np.testing.assert_array_equal(got[:4], pages[5])
    np.testing.assert_array_equal(got[4:8], pages[0])
    np.testing.assert_array_equal(got[8], pages[3, 0])
    assert A.paged_rows(pages, table, 1, 0).shape == (0, hkv, d)
