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


def test_folded_delta_equals_ub_w_form():
    # Delta = T X (what phase B computes) against Ub V - W S^T formed
    # separately, on one chunk with a nonzero state
    c = I.c5_gdn_bf16(tokens=64, hk=1, hv=1, dk=32, dv=24)
    rng = np.random.default_rng(2)
    S = rng.standard_normal((24, 32)) * 0.3
    k = c["k"][:, 0].astype(np.float64)
    v = c["v"][:, 0].astype(np.float64)
    beta = c["beta"][:, 0].astype(np.float64)
    Gc, T = CM.chunk_prep(k, beta, c["g"][:, 0].astype(np.float64))
    X = beta[:, None] * (v - np.exp(Gc)[:, None] * (k @ S.T))
    np.testing.assert_allclose(T @ X, CM.delta_ub_w(S, k, v, beta, Gc, T), atol=1e-12)
