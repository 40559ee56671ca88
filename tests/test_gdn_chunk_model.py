"""The chunked GDN algorithm of the HIP kernels equals the reference's
token-sequential recurrence (oracle.gdn.gdn_scan) on the CPU."""

import numpy as np
import pytest

from oracle import gdn as G
from oracle import inputs as I
from tests import gdn_chunk_model as CM


def test_blocked_unit_lower_inverse():
    rng = np.random.default_rng(0)
    B = np.tril(rng.standard_normal((64, 64)) * 0.3, -1)
    T = CM.invert_unit_lower(B)
    np.testing.assert_allclose(T @ (np.eye(64) + B), np.eye(64), atol=1e-10)


@pytest.mark.parametrize("chunk", [16, 64])
def test_chunked_equals_sequential(chunk):
    c = I.c5_gdn_bf16(tokens=128, hk=2, hv=4, dk=32, dv=24)
    rng = np.random.default_rng(1)
    s0 = rng.standard_normal((4, 24, 32)) * 0.1
    s_seq = s0.copy()
    ref = G.gdn_scan(s_seq, c["q"], c["k"], c["v"], c["beta"], c["g"])
    s_chk = s0.copy()
    out = CM.gdn_chunked(s_chk, c["q"], c["k"], c["v"], c["beta"], c["g"], chunk=chunk)
    np.testing.assert_allclose(out, ref, atol=1e-10)
    np.testing.assert_allclose(s_chk, s_seq, atol=1e-10)


def test_chunked_c5_shape_slice():
    # C5 head geometry (Dk = Dv = 128, 16 key heads / 32 value heads) on a
    # 2-chunk prefix with 4 value heads
    c = I.c5_gdn_bf16(tokens=128)
    v = c["v"][:, :4]
    s_seq = np.zeros((4, 128, 128))
    ref = G.gdn_scan(s_seq, c["q"], c["k"], v, c["beta"][:, :4], c["g"][:, :4])
    s_chk = np.zeros((4, 128, 128))
    out = CM.gdn_chunked(s_chk, c["q"], c["k"], v, c["beta"][:, :4], c["g"][:, :4])
    np.testing.assert_allclose(out, ref, atol=1e-9)
    np.testing.assert_allclose(s_chk, s_seq, atol=1e-9)


def test_folded_form_equals_delta_form():
    # The P / W form phase B computes against the textbook chunk step with
    # Delta = T diag(beta) X^T, on one chunk with a nonzero state and decays
    c = I.c5_gdn_bf16(tokens=64, hk=1, hv=1, dk=32, dv=24)
    rng = np.random.default_rng(2)
    S = rng.standard_normal((24, 32)) * 0.3
    q = c["q"][:, 0].astype(np.float64)
    k = c["k"][:, 0].astype(np.float64)
    v = c["v"][:, 0].astype(np.float64)
    beta = c["beta"][:, 0].astype(np.float64)
    Gc, T, P, W = CM.chunk_prep(q, k, beta, c["g"][:, 0].astype(np.float64))
    o1, s1 = CM.chunk_apply(S, q, k, v, Gc, P, W)
    o2, s2 = CM.chunk_apply_delta(S, q, k, v, beta, Gc, T)
    np.testing.assert_allclose(o1, o2, atol=1e-12)
    np.testing.assert_allclose(s1, s2, atol=1e-12)


def test_stored_tiles_cover_p_and_w():
    # Phase A stores only the six 16 x 32 tiles of P and W that can be
    # nonzero; every other tile is exactly zero (P and W are causal).
    c = I.c5_gdn_bf16(tokens=64, hk=1, hv=1, dk=32, dv=24)
    q = c["q"][:, 0].astype(np.float64)
    k = c["k"][:, 0].astype(np.float64)
    beta = c["beta"][:, 0].astype(np.float64)
    _, _, P, W = CM.chunk_prep(q, k, beta, c["g"][:, 0].astype(np.float64))
    live = set(CM.live_tiles())
    assert len(live) == 6
    for mat in (P, W):
        for mt in range(4):
            for ks in range(2):
                tile = mat[16 * mt:16 * mt + 16, 32 * ks:32 * ks + 32]
                if (mt, ks) not in live:
                    assert not tile.any()
        assert np.abs(np.triu(mat, 1)).max() == 0.0
