"""NumPy model of the chunked gated delta-rule algorithm the HIP kernels use.

This is the kernel's algorithm written out on the CPU (not the reference's,
which is token-sequential); ``tests/test_gdn_chunk_model.py`` checks it
against the sequential oracle so the derivation is pinned before it is
trusted on the GPU.

Per value head with state S (Dv x Dk) entering a chunk of C tokens, with
cumulative log decay Gc[t] = g_0 + ... + g_t (within the chunk) and
gamma = exp(Gc):

  A[t, i]  = exp(Gc[t] - Gc[i]) * (k_t . k_i)      for i < t   (else 0)
  T        = (I + diag(beta) A)^-1                 (unit lower triangular)
  X        = diag(beta) (V - diag(gamma) K S^T)    (C x Dv)
  Delta    = T X                                   (C x Dv; row t = delta_t)
  M[t, i]  = exp(Gc[t] - Gc[i]) * (q_t . k_i)      for i <= t  (else 0)
  O        = (diag(gamma) Q S^T + M Delta) / sqrt(Dk)
  S_next   = gamma[C-1] S + (diag(exp(Gc[C-1] - Gc)) Delta)^T K

The state-independent part (Gc, T, M) is computed per (head, chunk) in
parallel (phase A); the rest carries the chunk-to-chunk dependency (phase B)
and is independent across the Dv rows of S.  Delta = T X is the familiar
Ub V - W S^T with Ub = T diag(beta) and W = T diag(beta gamma) K
(``delta_ub_w``), folded so that phase B reads T instead of Ub and W.
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


def chunk_prep(k, beta, g):
    """State-independent per-chunk quantities (phase A).  k [C, Dk]; beta, g [C]."""
    Gc = np.cumsum(g)
    decay = np.exp(Gc[:, None] - Gc[None, :])
    C = k.shape[0]
    lower = np.tril(np.ones((C, C), dtype=bool), -1)
    A = np.where(lower, decay * (k @ k.T), 0.0)
    T = invert_unit_lower(beta[:, None] * A)
    return Gc, T


def delta_ub_w(S, k, v, beta, Gc, T):
    """Delta in the unfolded form Ub V - W S^T (cross-check of T X)."""
    Ub = T * beta[None, :]
    W = Ub @ (np.exp(Gc)[:, None] * k)
    return Ub @ v - W @ S.T


def chunk_apply(S, q, k, v, beta, Gc, T):
    """Carry the state through one chunk (phase B); returns (outputs [C, Dv], S_next)."""
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
            Gc, T = chunk_prep(kc, bc, g[s, h].astype(np.float64))
            O, S = chunk_apply(S, qc, kc, v[s, h].astype(np.float64), bc, Gc, T)
            out[s, h] = O
        state[h] = S
    return out
