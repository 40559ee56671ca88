"""Pins the Qwen3.5 layer-primitive oracle (oracle/layer.py) with closed
forms, hand-derived tables and independent textbook restatements.  Each
test names the plausible mistake it catches.  No GPU is needed."""

import math

import numpy as np
import pytest

from oracle import gdn as G
from oracle import layer as L


def _rng(seed=0):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ SiLU

def test_silu_closed_values_and_no_overflow():
    # silu(x) = x / (1 + e^-x): catches sigmoid-only (no x factor) and the
    # one-branch form that overflows for large negative x
    np.testing.assert_allclose(L.silu([0.0, 1.0, -1.0]),
                               [0.0, 1.0 / (1.0 + math.exp(-1.0)), -1.0 / (1.0 + math.e)],
                               rtol=1e-15)
    big = L.silu([-1000.0, 1000.0])
    assert np.all(np.isfinite(big)) and abs(big[0]) < 1e-300 and big[1] == 1000.0


# ------------------------------------------------------------------ norms

def test_l2_normalize_345_and_epsilon_is_a_floor():
    np.testing.assert_allclose(L.l2_normalize([3.0, 4.0], 1e-6), [0.6, 0.8], rtol=1e-15)
    # max(||x||, eps), not ||x|| + eps: a norm below eps divides by eps
    np.testing.assert_allclose(L.l2_normalize([1e-8, 0.0], 1e-6), [1e-2, 0.0], rtol=1e-12)
    np.testing.assert_allclose(L.l2_normalize([0.0, 0.0], 1e-6), [0.0, 0.0])


def test_rms_norm_uses_the_mean_and_the_weight():
    # [3, 4]: mean square 12.5 (a sum would give 25); weight applied per column
    out = L.rms_norm([3.0, 4.0], [1.0, 2.0], 0.0 + 1e-300)
    den = math.sqrt(12.5)
    np.testing.assert_allclose(out, [3.0 / den, 8.0 / den], rtol=1e-14)


def test_rms_norm_epsilon_inside_the_root():
    # constant vector c: c / sqrt(c^2 + eps); catches eps added outside the root
    c, eps = 0.01, 1e-4
    out = L.rms_norm(np.full(8, c), np.ones(8), eps)
    np.testing.assert_allclose(out, c / math.sqrt(c * c + eps), rtol=1e-14)


def test_gated_rms_norm_gate_is_silu_not_sigmoid():
    # gate 2: factor silu(2) = 2 / (1 + e^-2) = 1.7616 (sigmoid would be 0.8808)
    x = np.array([1.0, -2.0, 0.5])
    w = np.array([1.0, 1.0, 1.0])
    base = L.rms_norm(x, w, 1e-6)
    out = L.gated_rms_norm(x, w, np.full(3, 2.0), 1e-6)
    np.testing.assert_allclose(out, base * (2.0 / (1.0 + math.exp(-2.0))), rtol=1e-14)
    np.testing.assert_allclose(L.gated_rms_norm(x, w, np.zeros(3), 1e-6), 0.0)


# ------------------------------------------------------------------ conv

def test_conv_step_tap_order_and_history_shift():
    # one-hot taps: tap 0 must read the OLDEST history row and tap K-1 the
    # current sample; catches a reversed window
    k, c = 4, 3
    hist = np.arange(1.0, 1.0 + (k - 1) * c).reshape(k - 1, c)
    cur = np.array([100.0, 200.0, 300.0])
    for t0 in range(k):
        w = np.zeros((k, c))
        w[t0] = 1.0
        out, new_hist = L.conv_step(cur, w, hist)
        expect = cur if t0 == k - 1 else hist[t0]
        np.testing.assert_array_equal(out, expect)
        np.testing.assert_array_equal(new_hist, np.vstack((hist[1:], cur[None])))


def test_conv_step_layouts_agree_and_silu_applies_after_the_sum():
    rng = _rng(1)
    k, c = 4, 16
    w = rng.standard_normal((k, c))
    hist = rng.standard_normal((2, k - 1, c))
    cur = rng.standard_normal((2, c))
    a, ha = L.conv_step(cur, w, hist)
    b, hb = L.conv_step(cur, w.T, hist, layout="ck")
    np.testing.assert_allclose(a, b, rtol=1e-15)
    np.testing.assert_array_equal(ha, hb)
    s, _ = L.conv_step(cur, w, hist, apply_silu=True)
    np.testing.assert_allclose(s, L.silu(a), rtol=1e-15)
    # depthwise: each channel only sees itself (a dense mix would break this)
    direct = np.einsum("btc,tc->bc", np.concatenate((hist, cur[:, None]), axis=1), w)
    np.testing.assert_allclose(a, direct, rtol=1e-13)


# ------------------------------------------------------- recurrent params

def test_recurrent_parameters_closed_values_and_head_broadcast():
    # beta(0) = 1/2; softplus(0) = ln 2; per-head dt_bias / ssm_a broadcast
    # over the batch axis (catches indexing them by the batch)
    bl = np.array([[0.0, 0.0, 50.0], [-50.0, 0.0, 0.0]])
    al = np.array([[0.0, 1.0, 50.0], [0.0, -1.0, -40.0]])
    dt = np.array([0.0, -1.0, 0.0])
    ssm = np.array([-1.0, -2.0, -0.5])
    beta, g = L.recurrent_parameters(bl, al, dt, ssm)
    np.testing.assert_allclose(beta[0, 0], 0.5, rtol=1e-15)
    np.testing.assert_allclose(beta[0, 2], 1.0, rtol=1e-15)
    assert 0.0 < beta[1, 0] < 1e-21
    np.testing.assert_allclose(g[0, 0], -math.log(2.0), rtol=1e-15)
    np.testing.assert_allclose(g[0, 1], -2.0 * math.log(2.0), rtol=1e-15)  # 1 + (-1) = 0
    np.testing.assert_allclose(g[1, 1], -2.0 * math.log1p(math.exp(-2.0)), rtol=1e-14)
    np.testing.assert_allclose(g[0, 2], -0.5 * 50.0, rtol=1e-15)  # no overflow at 50
    np.testing.assert_allclose(g[1, 2], -0.5 * math.log1p(math.exp(-40.0)), rtol=1e-12)
    # agrees with the single-token qwen35_beta_decay oracle
    b1, g1 = G.beta_decay(bl[0], al[0], dt, ssm)
    np.testing.assert_allclose(beta[0], b1, rtol=1e-6)
    np.testing.assert_allclose(g[0], g1, rtol=1e-6)


# ---------------------------------------------------------------- IMROPE

def test_imrope_lane_schedule_hand_table():
    # derived by hand from the rule text (sector % 3 picks T/H/W while the
    # section allows, else E): pins the test order and the 3 * section bound
    assert [L.imrope_lane(p, (2, 1, 1, 1)) for p in range(5)] == [0, 1, 2, 0, 3]
    assert [L.imrope_lane(p, (11, 11, 10, 0)) for p in range(32)] == [p % 3 for p in range(32)]
    assert [L.imrope_lane(p, (1, 0, 0, 3)) for p in range(4)] == [0, 3, 3, 3]
    # the schedule repeats with period sum(sections)
    assert L.imrope_lane(37, (2, 1, 1, 1)) == L.imrope_lane(2, (2, 1, 1, 1))


def _neox_textbook(x, pos, base, rot_dims):
    """Independent rotate-half formulation of NeoX RoPE on the leading
    rot_dims coordinates: x * cos + rotate_half(x) * sin."""
    half = rot_dims // 2
    inv = base ** (-np.arange(half) * 2.0 / rot_dims)
    ang = np.concatenate([pos * inv, pos * inv])
    xr = x[..., :rot_dims]
    rh = np.concatenate([-xr[..., half:], xr[..., :half]], axis=-1)
    out = x.copy()
    out[..., :rot_dims] = xr * np.cos(ang) + rh * np.sin(ang)
    return out


def test_imrope_text_lanes_equal_textbook_neox_rope():
    # sections (11, 11, 10, 0) give every pair a T/H/W lane, and text lanes
    # (p, p, p, 0) make them all p: IMROPE must equal plain NeoX RoPE on the
    # first 64 coordinates and copy the rest (catches adjacent pairing
    # (2i, 2i+1), a wrong exponent, and rotating the tail)
    rng = _rng(3)
    x = rng.standard_normal((3, 256))
    for pos in (0, 1, 777, 32767):
        got = L.imrope(x, L.text_lanes(pos), (11, 11, 10, 0), 10000000.0)
        np.testing.assert_allclose(got, _neox_textbook(x, float(pos), 10000000.0, 64),
                                   rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(L.imrope(x, L.text_lanes(0), (11, 11, 10, 0), 1e7), x)


def test_imrope_per_lane_positions_and_norm():
    # distinct lane positions: pair p must turn by lanes[lane(p)] only
    rng = _rng(4)
    sections = (2, 1, 1, 1)
    x = rng.standard_normal((2, 12))
    lanes = np.array([[3.0, 5.0, 7.0, 11.0], [0.0, 2.0, 0.0, 9.0]])
    got = L.imrope(x, lanes, sections, 100.0, scale=0.5)
    for r in range(2):
        for p in range(5):
            lane = L.imrope_lane(p, sections)
            th = lanes[r, lane] * 0.5 * 100.0 ** (-2.0 * p / 10)
            a, b = x[r, p], x[r, p + 5]
            np.testing.assert_allclose(got[r, p], a * math.cos(th) - b * math.sin(th), rtol=1e-13)
            np.testing.assert_allclose(got[r, p + 5], a * math.sin(th) + b * math.cos(th),
                                       rtol=1e-12, atol=1e-14)
            np.testing.assert_allclose(got[r, p] ** 2 + got[r, p + 5] ** 2, a * a + b * b,
                                       rtol=1e-12)
        np.testing.assert_array_equal(got[r, 10:], x[r, 10:])


# ------------------------------------------------------ split / composites

def test_split_query_gate_interleaved_per_head():
    # per head: D query values then D gate values (not all queries first)
    p = np.arange(2 * 3 * 2 * 4).reshape(2, 3 * 2 * 4)
    q, g = L.split_query_gate(p, 3, 4)
    assert q.shape == (2, 3, 4) and g.shape == (2, 3, 4)
    np.testing.assert_array_equal(q[0, 1], [8, 9, 10, 11])
    np.testing.assert_array_equal(g[0, 1], [12, 13, 14, 15])
    np.testing.assert_array_equal(g[1, 2], 24 + np.array([20, 21, 22, 23]))


def test_attention_prologue_at_position_zero_is_norm_and_split():
    # position 0: IMROPE is the identity, so q / k are exactly the per-head
    # RMS norms and the gate is the raw second half of each head block
    rng = _rng(5)
    b, hq, hkv, d = 2, 4, 2, 16
    qg = rng.standard_normal((b, hq * 2 * d))
    k = rng.standard_normal((b, hkv * d))
    v = rng.standard_normal((b, hkv * d))
    qw = rng.uniform(0.5, 1.5, d)
    kw = rng.uniform(0.5, 1.5, d)
    q, g, kr, vv = L.attention_prologue(qg, k, v, qw, kw, 1e-6, np.zeros(b), (2, 2, 2, 0), 1e6)
    qs, gs = L.split_query_gate(qg, hq, d)
    np.testing.assert_allclose(q, L.rms_norm(qs, qw, 1e-6), rtol=1e-14)
    np.testing.assert_array_equal(g, gs)
    np.testing.assert_allclose(kr, L.rms_norm(k.reshape(b, hkv, d), kw, 1e-6), rtol=1e-14)
    np.testing.assert_array_equal(vv, v.reshape(b, hkv, d))


def test_recurrent_layer_step_zero_beta_only_decays_the_state():
    # beta ~ 0 (logit -60): the state must only decay by exp(g) per head and
    # the history must shift; catches beta / decay wired to the wrong heads
    rng = _rng(6)
    hk, hv, dk, dv, kk = 2, 4, 8, 8, 4
    chn = 2 * hk * dk + hv * dv
    mixed = rng.standard_normal((1, chn))
    w = rng.standard_normal((kk, chn))
    hist = rng.standard_normal((1, kk - 1, chn))
    state = rng.standard_normal((1, hv, dv, dk))
    s0 = state.copy()
    al = rng.standard_normal((1, hv))
    dt = rng.standard_normal(hv)
    ssm = -np.exp(rng.uniform(-1, 1, hv))
    out, new_hist = L.recurrent_layer_step(
        mixed, w, hist, rng.standard_normal((1, hv * dv)), np.full((1, hv), -60.0), al, dt, ssm,
        np.ones(dv), state, key_heads=hk, key_dim=dk, value_heads=hv, value_dim=dv, eps=1e-6)
    _, g = L.recurrent_parameters(np.zeros((1, hv)), al, dt, ssm)
    np.testing.assert_allclose(state[0], s0[0] * np.exp(g[0])[:, None, None], rtol=1e-12,
                               atol=1e-15)
    np.testing.assert_array_equal(new_hist[0], np.vstack((hist[0, 1:], mixed)))
    assert out.shape == (1, hv * dv) and np.all(np.isfinite(out))


def test_recurrent_layer_step_matches_composed_reference_chain():
    # the composite follows qwen35_numpy.py:63-131 step by step: conv+SiLU,
    # split q | k | v, normalize_qk, beta_decay, gdn_step, gated RMS
    rng = _rng(7)
    hk, hv, dk, dv, kk = 2, 4, 8, 6, 3
    chn = 2 * hk * dk + hv * dv
    mixed = rng.standard_normal((1, chn))
    w = rng.standard_normal((kk, chn))
    hist = rng.standard_normal((1, kk - 1, chn))
    state = rng.standard_normal((1, hv, dv, dk)) * 0.1
    gate = rng.standard_normal((1, hv * dv))
    bl, al = rng.standard_normal((1, hv)), rng.standard_normal((1, hv))
    dt, ssm, nw = rng.standard_normal(hv), -np.exp(rng.uniform(-1, 1, hv)), rng.uniform(0.5, 1.5, dv)
    st2 = state[0].copy()
    out, _ = L.recurrent_layer_step(mixed, w, hist, gate, bl, al, dt, ssm, nw, state,
                                    key_heads=hk, key_dim=dk, value_heads=hv, value_dim=dv,
                                    eps=1e-6)
    act = L.conv_step(mixed[0], w, hist[0], apply_silu=True)[0]
    q = act[:hk * dk].reshape(hk, dk)
    k = act[hk * dk:2 * hk * dk].reshape(hk, dk)
    v = act[2 * hk * dk:].reshape(hv, dv)
    qn, kn = G.normalize_qk(q, k, 1e-6)
    beta, g = G.beta_decay(bl[0], al[0], dt, ssm)
    o = G.gdn_step(st2, qn, kn, v, beta, g)
    expect = L.gated_rms_norm(o, nw, gate[0].reshape(hv, dv), 1e-6).reshape(-1)
    # the single-token helpers round to float32; the composite stays in float64
    np.testing.assert_allclose(out[0], expect, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(state[0], st2, rtol=1e-4, atol=1e-5)


def test_conv_history_length_is_checked():
    with pytest.raises(ValueError):
        L.conv_step(np.zeros(3), np.zeros((4, 3)), np.zeros((2, 3)))


# ------------------------------------------------------- chunked prefill

def _attn_layer_inputs(rng, tokens, hq, hkv, d, dv):
    qg = rng.standard_normal((tokens, hq * 2 * d))
    k = rng.standard_normal((tokens, hkv * d))
    v = rng.standard_normal((tokens, hkv * dv))
    qn = 1.0 + 0.1 * rng.standard_normal(d)
    kn = 1.0 + 0.1 * rng.standard_normal(d)
    return qg, k, v, qn, kn


def test_attention_layer_prefill_equals_the_batched_causal_form():
    # The token-sequential chain (one decode per token) equals one causal
    # prefill over the cache of the rotated queries: token t sees exactly
    # the rows 0 .. position + t.  Catches an off-by-one in the visible
    # range or a query rotated at the wrong position.
    from oracle import attention as A
    rng = _rng(11)
    tokens, hq, hkv, d, dv, position = 9, 4, 2, 16, 16, 5
    sections, base, eps = (3, 3, 2, 0), 10000.0, 1e-6
    qg, k, v, qn, kn = _attn_layer_inputs(rng, tokens, hq, hkv, d, dv)
    kc = np.zeros((position + tokens + 3, hkv, d))
    vc = np.zeros((position + tokens + 3, hkv, dv))
    kc[:position] = rng.standard_normal((position, hkv, d))
    vc[:position] = rng.standard_normal((position, hkv, dv))
    out = L.attention_layer_prefill(qg, k, v, qn, kn, eps, position, sections, base, kc, vc)
    q, g = L.split_query_gate(qg, hq, d)
    lanes = L.text_lanes(np.arange(position, position + tokens))[:, None, :]
    qr = L.imrope(L.rms_norm(q, qn, eps), lanes, sections, base)
    att = A.full_attention_prefill(qr, kc[:position + tokens], vc[:position + tokens],
                                   prefix_length=position)
    np.testing.assert_allclose(out, A.sigmoid_gate(att, g), rtol=1e-12, atol=1e-12)
    # the appended rows are the rotated keys and raw values at their positions
    kr = L.imrope(L.rms_norm(k.reshape(tokens, hkv, d), kn, eps), lanes, sections, base)
    np.testing.assert_allclose(kc[position:position + tokens], kr, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(vc[position:position + tokens], v.reshape(tokens, hkv, dv))
    assert not kc[position + tokens:].any()


def _extended_conv(mixed, conv_w, history):
    # the chunk-form convolution: token t convolves rows t .. t + K - 1 of
    # E = [history; mixed]; the new history is E's last K - 1 rows
    e = np.concatenate((history, mixed), axis=0)
    kernel = conv_w.shape[0]
    out = np.stack([np.sum(e[t:t + kernel] * conv_w, axis=0) for t in range(mixed.shape[0])])
    return L.silu(out), e[e.shape[0] - (kernel - 1):]


def test_recurrent_layer_prefill_equals_chunk_form():
    # The token-sequential chain equals the chunk form the device runs:
    # convolution over E = [history; x], one GDN scan, one gated norm.
    # Catches a window shifted by one row, a stale history row, or taps in
    # reverse order -- and, with T < K - 1, a history that keeps old rows.
    rng = _rng(12)
    hk, hv, dk, dv, kernel, eps = 2, 4, 8, 8, 4, 1e-6
    c = 2 * hk * dk + hv * dv
    for tokens in (7, 2):
        mixed = rng.standard_normal((tokens, c))
        conv_w = rng.standard_normal((kernel, c))
        hist = rng.standard_normal((kernel - 1, c))
        gate = rng.standard_normal((tokens, hv * dv))
        bl, al = rng.standard_normal((tokens, hv)), rng.standard_normal((tokens, hv))
        dtb, ssm = rng.standard_normal(hv), -np.exp(rng.uniform(-1, 1, hv))
        nw = 1.0 + 0.1 * rng.standard_normal(dv)
        s0 = 0.1 * rng.standard_normal((hv, dv, dk))
        st = s0.copy()
        out, new_hist = L.recurrent_layer_prefill(
            mixed, conv_w, hist, gate, bl, al, dtb, ssm, nw, st, key_heads=hk, key_dim=dk,
            value_heads=hv, value_dim=dv, eps=eps)
        act, want_hist = _extended_conv(mixed, conv_w, hist)
        np.testing.assert_array_equal(new_hist, want_hist)
        w = hk * dk
        q = L.l2_normalize(act[:, :w].reshape(tokens, hk, dk), eps)
        k = L.l2_normalize(act[:, w:2 * w].reshape(tokens, hk, dk), eps)
        v = act[:, 2 * w:].reshape(tokens, hv, dv)
        beta, g = L.recurrent_parameters(bl, al, dtb, ssm)
        s2 = s0.copy()
        o = G.gdn_scan(s2, q, k, v, beta, g)
        want = L.gated_rms_norm(np.asarray(o), nw, gate.reshape(tokens, hv, dv), eps)
        np.testing.assert_allclose(out, want.reshape(tokens, -1), rtol=1e-11, atol=1e-12)
        np.testing.assert_allclose(st, s2, rtol=1e-11, atol=1e-13)
