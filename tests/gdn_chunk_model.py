"""NumPy model of the chunked gated delta-rule algorithm the HIP kernels use.

This is the kernel's algorithm written out on the CPU (not the reference's,
which is token-sequential); ``tests/test_gdn_chunk_model.py`` checks it
against the sequential oracle so the derivation is pinned before it is
trusted on the GPU.

Per value head with state S (Dv x Dk) entering a chunk of C tokens, with
cumulative log decay Gc[t] = g_0 + ... + g_t (within the chunk),
gamma = exp(Gc) and scale = 1 / sqrt(Dk):

  A[t, i]  = exp(Gc[t] - Gc[i]) * (k_t . k_i)      for i < t   (else 0)
  M[t, i]  = exp(Gc[t] - Gc[i]) * (q_t . k_i)      for i <= t  (else 0)
  T        = (I + diag(beta) A)^-1                 (unit lower triangular)
  P        = scale M T diag(beta)                  (C x C, causal)
  W        = diag(gamma[C-1] / gamma) T diag(beta) (C x C, causal)

are state-independent (phase A, per head and chunk in parallel); phase B
carries the chunk-to-chunk dependency:

  X^T      = V - diag(gamma) K S^T                 (C x Dv)
  O        = scale diag(gamma) Q S^T + P X^T
  Y^T      = W X^T
  S_next^T = gamma[C-1] S^T + K^T Y^T

This is the textbook chunked delta rule (``chunk_apply_delta``: Delta =
T diag(beta) X^T, O = scale (diag(gamma) Q S^T + M Delta), S_next =
gamma[C-1] S + (diag(gamma[C-1] / gamma) Delta)^T K) with T folded into P
and W, so phase B holds no C x C inverse and its chain is X^T, Y^T and the
state update.
"""

from __future__ import annotations

import math

import numpy as np


def invert_unit_lower(B, block=16):
    """(I + B)^-1 for strictly lower-triangular B by 16x16 diagonal blocks
    (forward substitution) combined with the block recursion
    T_ij = -T_ii sum_{j<=k<i} B_ik T_kj, as the kernel does."""
    n = B.shape[0]
    T = np.zeros_like(B)
    nb = n // block
    for b in range(nb):
        s = slice(b * block, (b + 1) * block)
        Bd = B[s, s]
        Td = np.zeros((block, block), dtype=B.dtype)
        for t in range(block):
            Td[t] = -(Bd[t, :t] @ Td[:t])
            Td[t, t] = 1.0
        T[s, s] = Td
    for i in range(1, nb):
        si = slice(i * block, (i + 1) * block)
        for j in range(i - 1, -1, -1):
            sj = slice(j * block, (j + 1) * block)
            acc = np.zeros((block, block), dtype=B.dtype)
            for k in range(j, i):
                sk = slice(k * block, (k + 1) * block)
                acc += B[si, sk] @ T[sk, sj]
            T[si, sj] = -(T[si, si] @ acc)
    return T


def chunk_prep(q, k, beta, g):
    """State-independent per-chunk quantities (phase A).  q, k [C, Dk];
    beta, g [C].  Returns Gc, T, P, W."""
    Gc = np.cumsum(g)
    decay = np.exp(Gc[:, None] - Gc[None, :])
    C, dk = k.shape
    lower = np.tril(np.ones((C, C), dtype=bool), -1)
    causal = np.tril(np.ones((C, C), dtype=bool))
    A = np.where(lower, decay * (k @ k.T), 0.0)
    M = np.where(causal, decay * (q @ k.T), 0.0)
    T = invert_unit_lower(beta[:, None] * A)
    P = (M @ T) * beta[None, :] / math.sqrt(dk)
    W = np.exp(Gc[-1] - Gc)[:, None] * T * beta[None, :]
    return Gc, T, P, W


def chunk_apply(S, q, k, v, Gc, P, W):
    """Carry the state through one chunk (phase B); returns (outputs [C, Dv], S_next)."""
    dk = q.shape[1]
    XT = v - np.exp(Gc)[:, None] * (k @ S.T)
    O = np.exp(Gc)[:, None] * (q @ S.T) / math.sqrt(dk) + P @ XT
    YT = W @ XT
    S_next = (math.exp(Gc[-1]) * S.T + k.T @ YT).T
    return O, S_next


def chunk_apply_delta(S, q, k, v, beta, Gc, T):
    """The textbook chunk step with Delta = T diag(beta) X^T (cross-check of
    the folded P / W form)."""
    dk = q.shape[1]
    C = q.shape[0]
    X = beta[:, None] * (v - np.exp(Gc)[:, None] * (k @ S.T))
    Delta = T @ X
    causal = np.tril(np.ones((C, C), dtype=bool))
    M = np.where(causal, np.exp(Gc[:, None] - Gc[None, :]) * (q @ k.T), 0.0)
    O = (np.exp(Gc)[:, None] * (q @ S.T) + M @ Delta) / math.sqrt(dk)
    tail = np.exp(Gc[-1] - Gc)
    S_next = math.exp(Gc[-1]) * S + (tail[:, None] * Delta).T @ k
    return O, S_next


def live_tiles(C=64):
    """(m tile, k step) pairs of the 16 x 32 A-operand tiles of a causal C x C
    matrix that can hold a nonzero (the ones phase A stores)."""
    return [(mt, ks) for mt in range(C // 16) for ks in range(C // 32) if 32 * ks <= 16 * mt + 15]


def gdn_chunked(state, q, k, v, beta, g, chunk=64):
    """Chunked GDN over T tokens for every value head.  state [Hv, Dv, Dk]
    (updated in place); q, k [T, Hk, Dk]; v [T, Hv, Dv]; beta, g [T, Hv].
    T must be a multiple of ``chunk``."""
    t_count = q.shape[0]
    hv = state.shape[0]
    hk = q.shape[1]
    out = np.zeros((t_count, hv, state.shape[1]))
    for h in range(hv):
        kh = h % hk
        S = state[h].astype(np.float64)
        for c0 in range(0, t_count, chunk):
            s = slice(c0, c0 + chunk)
            qc, kc = q[s, kh].astype(np.float64), k[s, kh].astype(np.float64)
            bc = beta[s, h].astype(np.float64)
            Gc, _, P, W = chunk_prep(qc, kc, bc, g[s, h].astype(np.float64))
            O, S = chunk_apply(S, qc, kc, v[s, h].astype(np.float64), Gc, P, W)
            out[s, h] = O
        state[h] = S
    return out
