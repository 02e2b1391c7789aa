"""The chunkwise (WY/UT) form of the gated delta rule, forward and backward, in float64 numpy: the decomposition
the chunked HIP design implements, kernel by kernel, so its equations can be checked against the oracle on the CPU.

Per value head and chunk of C steps (positions i < C; a partial last chunk is padded with k = q = v = 0, beta = 0,
log-decay 0), with S0 the state at the chunk start (rows = value index):
  G_i = sum_{j<=i} a_j,  gam_i = exp(G_i),  E_ij = exp(G_i - G_j)
  A = strict_lower(diag(beta) (E * K K^T)),  T = (I + A)^-1,  Tb = T diag(beta)              [prep]
  KS = K S0^T,  R = V - diag(gam) KS,  Delta = Tb R                                          [state pass]
  Y = diag(gam) Q S0^T + P Delta,  P = lower_incl(E * Q K^T)
  S_C = gam_{C-1} S0 + Delta^T diag(exp(G_{C-1} - G)) K
Delta's rows are the per-step delta_t = beta_t (v_t - u_t) of the recurrence (reference src/delta_grad.cpp:14).
Backward, with dS_C the cotangent of the chunk's end state (the next chunk's start):
  dDelta = P^T dY + D K dS_C^T,  D = diag(exp(G_{C-1} - G));  dR = Tb^T dDelta;  dV = dR                [bwd state]
  dS0 = gam_{C-1} dS_C + (diag(gam) dY)^T Q - (diag(gam) dR)^T K
  dQ = diag(gam) dY S0 + (dP * M) K,  dP = dY Delta^T                                               [bwd grads]
  dK = -diag(gam) dR S0 + D Delta dS_C + (dP * M)^T Q + (dKK + dKK^T) K
  dTb = dDelta R^T;  dbeta_j = sum_i dTb_ij T_ij + sum_j' dA_jj' G_jj';  dA = -T^T (dTb diag(beta)) T^T (strict lower)
  dKK = strict_lower(diag(beta) dA * E);  dG from every exp(.) factor;  da_t = sum_{i >= t} dG_i
"""
from __future__ import annotations

import numpy as np

# The matrix product every equation below uses: numpy's own (float64 inputs give float64 products), or a replacement
# with the same signature, such as an emulation of the kernels' MFMA arithmetic on float32 inputs.
MM = None


def mm(x, y):
    return x @ y if MM is None else MM(x, y)


def prep(K, beta, a):
    C = K.shape[0]
    G = np.cumsum(a)
    E = np.exp(G[:, None] - G[None, :])
    KK = mm(K, K.T)
    A = np.tril(beta[:, None] * E * KK, -1)
    T = np.linalg.inv(np.eye(C, dtype=A.dtype) + A)
    return G, E, KK, A, T, T * beta[None, :]


def chunk_fwd(K, Q, V, beta, a, S0):
    G, E, KK, A, T, Tb = prep(K, beta, a)
    gam = np.exp(G)
    KS = mm(K, S0.T)
    R = V - gam[:, None] * KS
    Delta = mm(Tb, R)
    P = np.tril(E * mm(Q, K.T))
    Y = gam[:, None] * mm(Q, S0.T) + mm(P, Delta)
    D = np.exp(G[-1] - G)
    S1 = gam[-1] * S0 + mm((Delta * D[:, None]).T, K)
    return Y, S1


def chunk_bwd(K, Q, V, beta, a, S0, dY, dS1):
    """Returns dQ, dK, dV, dbeta, da, dS0 for one chunk."""
    G, E, KK, A, T, Tb = prep(K, beta, a)
    gam = np.exp(G)
    D = np.exp(G[-1] - G)
    M = np.tril(E)
    QK = mm(Q, K.T)
    P = M * QK
    KS = mm(K, S0.T)
    QS = mm(Q, S0.T)
    R = V - gam[:, None] * KS
    Delta = mm(Tb, R)
    # state pass
    KdS = mm(K, dS1.T)
    dDelta = mm(P.T, dY) + D[:, None] * KdS
    dR = mm(Tb.T, dDelta)
    dV = dR
    dS0 = gam[-1] * dS1 + mm((gam[:, None] * dY).T, Q) - mm((gam[:, None] * dR).T, K)
    # gradients
    dP = np.tril(mm(dY, Delta.T))
    dQ = gam[:, None] * mm(dY, S0) + mm(dP * M, K)
    dK = -gam[:, None] * mm(dR, S0) + D[:, None] * mm(Delta, dS1) + mm((dP * M).T, Q)
    dTb = np.tril(mm(dDelta, R.T))
    dT = dTb * beta[None, :]
    dbeta = (dTb * T).sum(0)
    dA = np.tril(-mm(mm(T.T, dT), T.T), -1)
    Gm = E * KK  # A = diag(beta) Gm (strict lower)
    dbeta += (dA * Gm).sum(1)
    dGm = beta[:, None] * dA
    dKK = dGm * E
    dK += mm(dKK + dKK.T, K)
    dG = np.zeros_like(a)
    # exp(G_i - G_j) factors: A (via Gm), P (via M)
    for X in (dGm * Gm, dP * P):
        dG += X.sum(1) - X.sum(0)
    dG += gam * (dY * QS).sum(1)              # Y's diag(gam) Q S0^T
    dG -= gam * (dR * KS).sum(1)              # R = V - diag(gam) KS
    dD = (Delta * KdS).sum(1)                 # S1's D_i = exp(G_{C-1} - G_i)
    dG[-1] += (dD * D).sum() + gam[-1] * np.sum(dS1 * S0)
    dG -= dD * D
    da = np.cumsum(dG[::-1])[::-1]
    return dQ, dK, dV, dbeta, da, dS0


def gated_delta_chunked(q, k, v, a, beta, s0, dy, ds_out, C=64):
    """Whole-sequence forward and backward through the chunk form, shapes as the oracle's (B, T, H, D), log-decay a.
    Returns y, s_out, dq, dk, dv, da, dbeta, ds0."""
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    grp = Hv // Hk
    y = np.zeros((B, T, Hv, Dv))
    s_out = np.zeros((B, Hv, Dv, Dk))
    dq, dk = np.zeros(q.shape), np.zeros(k.shape)
    dv = np.zeros(v.shape)
    da, dbeta = np.zeros(a.shape), np.zeros(beta.shape)
    ds0 = np.zeros((B, Hv, Dv, Dk))
    nch = (T + C - 1) // C

    def chunk(x, b, h, c):
        t0, t1 = c * C, min(T, c * C + C)
        out = np.zeros((C,) + x.shape[3:], x.dtype) if x.ndim == 4 else np.zeros(C, x.dtype)
        out[: t1 - t0] = x[b, t0:t1, h]
        return out

    for b in range(B):
        for hv in range(Hv):
            hk = hv // grp
            S = np.zeros((Dv, Dk), q.dtype) if s0 is None else s0[b, hv].copy()
            starts = []
            for c in range(nch):
                starts.append(S)
                Y, S = chunk_fwd(chunk(k, b, hk, c), chunk(q, b, hk, c), chunk(v, b, hv, c), chunk(beta, b, hv, c),
                                 chunk(a, b, hv, c), S)
                t0, t1 = c * C, min(T, c * C + C)
                y[b, t0:t1, hv] = Y[: t1 - t0]
            s_out[b, hv] = S
            dS = np.zeros((Dv, Dk), q.dtype) if ds_out is None else ds_out[b, hv].copy()
            for c in reversed(range(nch)):
                out = chunk_bwd(chunk(k, b, hk, c), chunk(q, b, hk, c), chunk(v, b, hv, c), chunk(beta, b, hv, c),
                                chunk(a, b, hv, c), starts[c], chunk(dy, b, hv, c), dS)
                dQ, dK, dV, dB, dA, dS = out
                t0, t1 = c * C, min(T, c * C + C)
                n = t1 - t0
                dq[b, t0:t1, hk] += dQ[:n]
                dk[b, t0:t1, hk] += dK[:n]
                dv[b, t0:t1, hv] = dV[:n]
                dbeta[b, t0:t1, hv] = dB[:n]
                da[b, t0:t1, hv] = dA[:n]
            ds0[b, hv] = dS
    return y, s_out, dq, dk, dv, da, dbeta, ds0
