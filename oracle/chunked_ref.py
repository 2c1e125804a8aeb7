"""Chunked (WY / UT) form of the gated-delta recurrence, float64.

TEST INFRASTRUCTURE ONLY (same import rule as ``gated_delta_ref``).

The reference has no chunk-parallel form: its prefill runs the sequential
recurrence (``model/qwen3_5/_gated_delta_metal.py:64-87``, and the ops path
``model/qwen3_5/gated_delta.py:93-109``). This module restates the algebra the
GPU prefill kernel uses, so that a test can show it equals the sequential
oracle on identical inputs; the GPU kernel is then checked against both.

Per value head and chunk of C tokens with start state S0 (Dv x Dk), log-decay
l_i = sum_{j<=i} log g_j, decay ratio G_ij = exp(l_i - l_j):

    A   = strict_lower(diag(beta) (K K^T) o G)
    Tb  = (I + A)^-1 diag(beta)
    R   = V - diag(exp(l)) K S0^T
    D   = Tb R                                      (the per-token deltas)
    Y   = diag(exp(l)) Q S0^T + lower(Q K^T o G) D
    S_C = exp(l_C) S0 + (diag(exp(l_C - l)) D)^T K
"""

from __future__ import annotations

import numpy as np

from .gated_delta_ref import repeat_heads


def chunk_step(q, k, v, log_g, beta, state):
    """One chunk for all value heads. q/k ``(C, Hv, Dk)`` (already repeated),
    v ``(C, Hv, Dv)``, log_g/beta ``(C, Hv)``, state ``(Hv, Dv, Dk)``."""

    Q = q.transpose(1, 0, 2)
    K = k.transpose(1, 0, 2)
    V = v.transpose(1, 0, 2)
    l = np.cumsum(log_g.T, axis=1)  # (H, C)
    bt = beta.T
    C = Q.shape[1]
    diff = l[:, :, None] - l[:, None, :]
    lower = np.tril(np.ones((C, C), dtype=bool))
    strict = np.tril(np.ones((C, C), dtype=bool), -1)
    decay = np.where(lower, np.exp(np.where(lower, diff, 0.0)), 0.0)
    KK = K @ K.transpose(0, 2, 1)
    A = np.where(strict, bt[:, :, None] * KK * decay, 0.0)
    eye = np.eye(C)
    T = np.linalg.solve(eye[None] + A, np.broadcast_to(eye, A.shape))
    Tb = T * bt[:, None, :]
    gam = np.exp(l)
    R = V - gam[:, :, None] * (K @ state.transpose(0, 2, 1))
    D = Tb @ R
    P = (Q @ K.transpose(0, 2, 1)) * decay
    Y = gam[:, :, None] * (Q @ state.transpose(0, 2, 1)) + P @ D
    w = np.exp(l[:, -1:] - l)
    new_state = np.exp(l[:, -1])[:, None, None] * state + (w[:, :, None] * D).transpose(0, 2, 1) @ K
    return Y.transpose(1, 0, 2), new_state


def chunked_scan(q, k, v, g, beta, state, chunk=64):
    """Same contract as ``gated_delta_scan_ops`` (single sequence, q/k at
    their own head count), computed chunk by chunk."""

    q, k, v, g, beta, state = (np.asarray(t, dtype=np.float64) for t in (q, k, v, g, beta, state))
    repeat = v.shape[-2] // q.shape[-2]
    q = repeat_heads(q, repeat)
    k = repeat_heads(k, repeat)
    with np.errstate(divide="ignore"):
        log_g = np.log(g)
    log_g = np.maximum(log_g, -1e4)
    ys = []
    for c0 in range(0, q.shape[0], chunk):
        sl = slice(c0, c0 + chunk)
        y, state = chunk_step(q[sl], k[sl], v[sl], log_g[sl], beta[sl], state)
        ys.append(y)
    return np.concatenate(ys), state
