"""The decomposition the chunked form uses for masked steps, checked on the CPU against the oracle's masked
recurrence (tools/gdn_vjp.py:3-6, _step_parts :238-256): two unmasked passes over the effective gates
(decay 1 and beta 0 where the mask is 0), the second with k as the query, an elementwise fix-up of y at masked
tokens, and the fix-up's VJP feeding the two passes' backwards (gdn_mask.hip states the formulas).  Float64,
every output of forward and VJP, scalar decay and log-decay gates, GQA 2:1, with and without an initial state.
"""

import numpy as np
import pytest

from oracle import gdn_oracle as O


def _masked_by_two_passes(q, k, v, decay, beta, S0, mask, dy, dS_T, chunk):
    m = mask.astype(np.float64)
    B, T, Hk, D = q.shape
    Hv = v.shape[2]
    rep = Hv // Hk
    d2 = np.where(m[:, :, None] > 0, decay, 1.0)
    b2 = beta * m[:, :, None]
    # forward: y' (pass 1) and z (pass 2, k as query) over the effective gates
    (y1, S_T), _ = O.gated_delta_chunked_vjp(q, k, v, d2, b2, S0, None, np.zeros_like(v), None, chunk,
                                             np.float64)
    (z, _), _ = O.gated_delta_chunked_vjp(k, k, v, d2, b2, S0, None, np.zeros_like(v), None, chunk, np.float64)
    c = np.einsum("btkd,btkd->btk", q, k)                      # k . q per key head
    cv = np.repeat(c, rep, axis=2)[..., None]                  # per value head
    dd = decay[..., None]
    bb = beta[..., None]
    u = v - dd * z
    masked = (m < 0.5)[:, :, None, None]
    y = np.where(masked, dd * y1 + bb * cv * u, y1)
    # backward: cotangents of the passes, then the fix-up's own terms
    dy1 = np.where(masked, dd * dy, dy)
    dz = np.where(masked, -bb * cv * dd * dy, 0.0)
    _, g1 = O.gated_delta_chunked_vjp(q, k, v, d2, b2, S0, None, dy1, dS_T, chunk, np.float64)
    _, g2 = O.gated_delta_chunked_vjp(k, k, v, d2, b2, S0, None, dz, None, chunk, np.float64)
    s_u = (u * dy).sum(-1)                                      # u . dy      [B,T,Hv]
    s_d = ((y1 - bb * cv * z) * dy).sum(-1)                    # d y / d decay . dy
    f = (beta * s_u).reshape(B, T, Hk, rep).sum(-1)[..., None]  # per key head
    mk = masked[..., 0]                                         # [B,T,1]
    dq = g1[0] + np.where(mk[..., None], f * k, 0.0)
    dk = g1[1] + g2[1] + g2[0] + np.where(mk[..., None], f * q, 0.0)
    dv = g1[2] + g2[2] + np.where(masked, bb * cv * dy, 0.0)
    ddec = np.where(mk, s_d, g1[3] + g2[3])
    dbeta = np.where(mk, cv[..., 0] * s_u, g1[4] + g2[4])
    return y, S_T, (dq, dk, dv, ddec, dbeta, g1[5] + g2[5])


@pytest.mark.parametrize("s0_std", [0.0, 0.3])
@pytest.mark.parametrize("chunk", [4, 64])
def test_two_pass_decomposition_matches_masked_oracle(s0_std, chunk):
    B, T, Hk, Hv, D = 2, 23, 2, 4, 8
    d = O.make_inputs(B, T, Hk, Hv, D, seed=5 + chunk, s0_std=s0_std, dtype=np.float64)
    rng = np.random.default_rng(3)
    mask = rng.uniform(size=(B, T)) > 0.35
    mask[0, :3] = False     # a masked prefix (left padding)
    mask[1, -5:] = False    # a masked suffix (right padding)
    dS_T = rng.standard_normal(d["state"].shape)
    (wy, wS), wg = O.gated_delta_chunked_vjp(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], mask,
                                             d["dy"], dS_T, chunk, np.float64)
    y, S_T, g = _masked_by_two_passes(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], mask, d["dy"],
                                      dS_T, chunk)
    for name, a, b in [("y", y, wy), ("S_T", S_T, wS)] + list(zip(("dq", "dk", "dv", "dg", "dbeta", "dS0"), g, wg)):
        err = np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)
        assert err < 1e-11, (name, err)


def test_two_pass_decomposition_log_gate():
    """The log-decay gate: dg_log = decay * dg_decay at every token, the fix-up's included."""
    B, T, Hk, Hv, D = 1, 17, 1, 2, 8
    d = O.make_inputs(B, T, Hk, Hv, D, seed=9, s0_std=0.2, dtype=np.float64)
    mask = np.ones((B, T), bool)
    mask[0, 5:9] = False
    (_, _), wg = O.gated_delta_chunked_vjp(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], mask, d["dy"],
                                           None, 64, np.float64)
    _, _, g = _masked_by_two_passes(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], mask, d["dy"],
                                    np.zeros_like(d["state"]), 64)
    np.testing.assert_allclose(g[3] * d["decay"], wg[3] * d["decay"], rtol=1e-10, atol=1e-12)
