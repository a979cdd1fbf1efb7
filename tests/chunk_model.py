"""NumPy model of the chunked (WY/UT) decomposition the HIP chunk kernels implement, kernel by kernel.

Per chunk of C tokens with entry state h = S^T ([Dk, Dv]), cumulative log decay G_r = sum_{u<=r} g_u,
gamma = exp(G), Gam_rs = exp(G_r - G_s) (s <= r):

  A  = strict_lower(diag(beta) (K K^T) * Gam)      T = (I + A)^-1
  W  = T diag(beta gamma) K                        U = T diag(beta) V
  Delta = U - W h                                  P = lower(Q K^T * Gam)
  Y  = diag(gamma) Q h + P Delta                   h' = gamma_C h + K^T diag(gamma_C / gamma) Delta

and the reverse pass below.  Used by tests to check kernel intermediates; itself checked against the oracle
in tests/test_chunk_model.py.
"""

import numpy as np


def prep(k, v, q, g_log, beta):
    """Per chunk: (G, T, W, U, P) for one head; k, q [C,Dk], v [C,Dv], g_log, beta [C]."""
    C = k.shape[0]
    G = np.cumsum(g_log.astype(np.float64))
    gam = np.exp(G)
    Gam = np.exp(np.tril(G[:, None] - G[None, :]))
    Gam = np.tril(Gam)
    A = np.tril(beta[:, None] * (k @ k.T) * Gam, -1)
    T = np.linalg.inv(np.eye(C) + A)
    W = T @ ((beta * gam)[:, None] * k)
    U = T @ (beta[:, None] * v)
    P = np.tril((q @ k.T) * Gam)
    return G, T, W, U, P


def fwd_chunk(h, q, k, G, W, U, P):
    gam = np.exp(G)
    Delta = U - W @ h
    Y = gam[:, None] * (q @ h) + P @ Delta
    gC = gam[-1]
    h_next = gC * h + k.T @ (np.exp(G[-1] - G)[:, None] * Delta)
    return Delta, Y, h_next


def bwd_state_chunk(dh_next, q, k, G, W, P, dY):
    """dDelta and the adjoint of the chunk's entry state."""
    gam = np.exp(G)
    Kt = np.exp(G[-1] - G)[:, None] * k
    dDelta = Kt @ dh_next + P.T @ dY
    dh = gam[-1] * dh_next + (gam[:, None] * q).T @ dY - W.T @ dDelta
    return dDelta, dh


def bwd_local_chunk(q, k, v, beta, G, T, P, h, dh_next, Delta, dDelta, dY):
    """dq, dk, dv, dbeta, dg_log for one chunk of one head."""
    C = q.shape[0]
    gam = np.exp(G)
    gC = gam[-1]
    r_C = np.exp(G[-1] - G)
    Gam = np.tril(np.exp(np.tril(G[:, None] - G[None, :])))
    dG = np.zeros(C)
    # terms with the entry state h and the exit-state adjoint dh_next
    X1 = dY @ h.T
    dq = gam[:, None] * X1
    dG += (q * dq).sum(1)
    X2 = Delta @ dh_next.T
    dk = r_C[:, None] * X2
    t2 = (k * dk).sum(1)
    dG -= t2
    dG[-1] += t2.sum() + gC * (dh_next * h).sum()
    dW = -(dDelta @ h.T)
    # output's intra-chunk term P = lower(Q K^T * Gam)
    dP = np.tril(dY @ Delta.T)
    dPG = dP * Gam
    dq += dPG @ k
    dk += dPG.T @ q
    e = dP * P
    dG += e.sum(1) - e.sum(0)
    # through T: W = T diag(beta gamma) K, U = T diag(beta) V
    TdW = T.T @ dW
    dk += (beta * gam)[:, None] * TdW
    s4 = (TdW * k).sum(1)
    dbeta = gam * s4
    dG += gam * beta * s4
    TdD = T.T @ dDelta
    dv = beta[:, None] * TdD
    dbeta += (v * TdD).sum(1)
    dT = dDelta @ (beta[:, None] * v).T + dW @ ((beta * gam)[:, None] * k).T
    dA = -np.tril(T.T @ dT @ T.T, -1)
    KK = k @ k.T
    dbeta += (dA * KK * Gam).sum(1)
    Amat = np.tril(beta[:, None] * KK * Gam, -1)
    e = dA * Amat
    dG += e.sum(1) - e.sum(0)
    M = beta[:, None] * dA * Gam
    dk += (M + M.T) @ k
    dg_log = np.cumsum(dG[::-1])[::-1]
    return dq, dk, dv, dbeta, dg_log


def bwd_local_chunk_z(q, k, v, beta, G, P, h, dh_next, Delta, TdD, dY):
    """bwd_local_chunk through Z = diag(beta) V - diag(beta gamma) K h (Delta = T Z), from TdD = T^T dDelta.

    Everything T contributes then follows from TdD alone: dV = diag(beta) TdD, dK -= diag(beta gamma) TdD h^T, the
    beta and gate terms of Z, and dA = -strict_lower(T^T dT T^T) = -strict_lower(TdD Delta^T) (dT = dDelta Z^T).
    T and dDelta themselves are not needed."""
    C = q.shape[0]
    gam = np.exp(G)
    gC = gam[-1]
    r_C = np.exp(G[-1] - G)
    Gam = np.tril(np.exp(np.tril(G[:, None] - G[None, :])))
    dG = np.zeros(C)
    X1 = dY @ h.T
    dq = gam[:, None] * X1
    dG += (q * dq).sum(1)
    X2 = Delta @ dh_next.T
    dk = r_C[:, None] * X2
    t2 = (k * dk).sum(1)
    dG -= t2
    dG[-1] += t2.sum() + gC * (dh_next * h).sum()
    dP = np.tril(dY @ Delta.T)
    dPG = dP * Gam
    dq += dPG @ k
    dk += dPG.T @ q
    e = dP * P
    dG += e.sum(1) - e.sum(0)
    # through Z
    Y2 = TdD @ h.T
    s4 = (Y2 * k).sum(1)
    dk -= (beta * gam)[:, None] * Y2
    dv = beta[:, None] * TdD
    dbeta = (v * TdD).sum(1) - gam * s4
    dG -= beta * gam * s4
    # through A
    dA = -np.tril(TdD @ Delta.T, -1)
    KK = k @ k.T
    dbeta += (dA * KK * Gam).sum(1)
    Amat = np.tril(beta[:, None] * KK * Gam, -1)
    e = dA * Amat
    dG += e.sum(1) - e.sum(0)
    M = beta[:, None] * dA * Gam
    dk += (M + M.T) @ k
    dg_log = np.cumsum(dG[::-1])[::-1]
    return dq, dk, dv, dbeta, dg_log


def run(q, k, v, g_log, beta, S0, dY, dS_T, C=64, z_form=False):
    """Whole-sequence forward + VJP for one batch element and one value head.

    q, k [T,Dk]; v, dY [T,Dv]; g_log, beta [T]; S0, dS_T [Dv,Dk] in the reference's state layout.
    Returns (y, S_T, dq, dk, dv, dg_log, dbeta, dS0) with the states in [Dv,Dk] layout.  z_form runs the local
    backward through TdD = T^T dDelta (bwd_local_chunk_z), as the bf16 kernel set does.
    """
    T_len, Dk = q.shape
    Dv = v.shape[1]
    nc = -(-T_len // C)
    pad = nc * C - T_len
    padf = lambda x: np.concatenate([x, np.zeros((pad,) + x.shape[1:], x.dtype)]) if pad else x
    q, k, v, g_log, beta, dY = (padf(np.asarray(x, np.float64)) for x in (q, k, v, g_log, beta, dY))
    h = np.asarray(S0, np.float64).T.copy()
    preps, hs, Ds = [], [], []
    y = np.zeros((nc * C, Dv))
    for c in range(nc):
        sl = slice(c * C, (c + 1) * C)
        pr = prep(k[sl], v[sl], q[sl], g_log[sl], beta[sl])
        preps.append(pr)
        hs.append(h)
        G, T, W, U, P = pr
        Delta, Y, h = fwd_chunk(h, q[sl], k[sl], G, W, U, P)
        Ds.append(Delta)
        y[sl] = Y
    S_T = h.T
    dh = np.asarray(dS_T, np.float64).T.copy()
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    dg, db = np.zeros(nc * C), np.zeros(nc * C)
    for c in range(nc - 1, -1, -1):
        sl = slice(c * C, (c + 1) * C)
        G, T, W, U, P = preps[c]
        dDelta, dh_prev = bwd_state_chunk(dh, q[sl], k[sl], G, W, P, dY[sl])
        if z_form:
            out = bwd_local_chunk_z(q[sl], k[sl], v[sl], beta[sl], G, P, hs[c], dh, Ds[c], T.T @ dDelta, dY[sl])
        else:
            out = bwd_local_chunk(q[sl], k[sl], v[sl], beta[sl], G, T, P, hs[c], dh, Ds[c], dDelta, dY[sl])
        dq[sl], dk[sl], dv[sl], db[sl], dg[sl] = out
        dh = dh_prev
    n = T_len
    return y[:n], S_T, dq[:n], dk[:n], dv[:n], dg[:n], db[:n], dh.T
