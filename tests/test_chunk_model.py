"""The chunked-form model (tests/chunk_model.py) agrees with the oracle: forward outputs and the full VJP."""

import numpy as np
import pytest

from oracle import gdn_oracle as O
import chunk_model


@pytest.mark.parametrize("z_form", [False, True])
@pytest.mark.parametrize("T,C,s0", [(64, 64, 0.0), (130, 64, 0.5), (37, 16, 1.0), (200, 32, 0.02)])
def test_chunk_model_matches_oracle(T, C, s0, z_form):
    d = O.make_inputs(1, T, 1, 2, 16, seed=T, s0_std=s0, dtype=np.float64)
    dS_T = np.random.default_rng(T).standard_normal(d["state"].shape) * 0.3
    (y, S), (dq, dk, dv, dg, db, dS0) = O.gated_delta_chunked_vjp(
        d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], None, d["dy"], dS_T, chunk=C,
        dtype=np.float64)
    dg_log = dg * d["decay"]
    for h in range(2):
        out = chunk_model.run(d["q"][0, :, 0], d["k"][0, :, 0], d["v"][0, :, h], d["g_log"][0, :, h],
                              d["beta"][0, :, h], d["state"][0, h], d["dy"][0, :, h], dS_T[0, h], C=C,
                              z_form=z_form)
        want = (y[0, :, h], S[0, h], None, None, dv[0, :, h], dg_log[0, :, h], db[0, :, h], dS0[0, h])
        for name, a, b in zip(("y", "S", "dq", "dk", "dv", "dg", "db", "dS0"), out, want):
            if b is not None:
                np.testing.assert_allclose(a, b, atol=1e-9, rtol=1e-7, err_msg=name)
    # dq / dk summed over the two value heads sharing the key head
    outs = [chunk_model.run(d["q"][0, :, 0], d["k"][0, :, 0], d["v"][0, :, h], d["g_log"][0, :, h],
                            d["beta"][0, :, h], d["state"][0, h], d["dy"][0, :, h], dS_T[0, h], C=C,
                            z_form=z_form)
            for h in range(2)]
    np.testing.assert_allclose(outs[0][2] + outs[1][2], dq[0, :, 0], atol=1e-9, rtol=1e-7)
    np.testing.assert_allclose(outs[0][3] + outs[1][3], dk[0, :, 0], atol=1e-9, rtol=1e-7)


def test_pair_blocked_equals_direct():
    rng = np.random.default_rng(3)
    X, Y = rng.standard_normal((64, 8)), rng.standard_normal((64, 8))
    G = np.cumsum(-rng.uniform(0.0, 3.0, (64, 8)), axis=0)   # down to exp(-190): exp(-G) alone would overflow fp32
    for incl in (False, True):
        np.testing.assert_allclose(chunk_model.pair_blocked(X, Y, G, incl), chunk_model.pair_direct(X, Y, G, incl),
                                   atol=1e-12, rtol=1e-10)


def test_pair_vjp_matches_finite_differences():
    rng = np.random.default_rng(4)
    X, Y = rng.standard_normal((64, 4)), rng.standard_normal((64, 4))
    G = np.cumsum(-rng.uniform(0.0, 1.0, (64, 4)), axis=0)
    dM = np.tril(rng.standard_normal((64, 64)))
    dX, dY, dG = chunk_model.pair_vjp(X, Y, G, dM)
    f = lambda X_, Y_, G_: (chunk_model.pair_direct(X_, Y_, G_, True) * dM).sum()
    eps = 1e-6
    for arr, grad, which in ((X, dX, 0), (Y, dY, 1), (G, dG, 2)):
        for (r, j) in ((0, 0), (17, 2), (40, 1), (63, 3)):
            args = [X.copy(), Y.copy(), G.copy()]
            args[which][r, j] += eps
            up = f(*args)
            args[which][r, j] -= 2 * eps
            dn = f(*args)
            assert abs((up - dn) / (2 * eps) - grad[r, j]) < 1e-6 * max(1.0, abs(grad[r, j])), (which, r, j)


@pytest.mark.parametrize("T,s0", [(64, 0.0), (130, 0.5), (40, 1.0)])
def test_vector_gate_chunk_model_matches_oracle(T, s0):
    """The per-channel-gate chunk model (16-token block factors, dg through the reverse sum of dG) agrees with the
    oracle's per-channel recurrence: every output and the full VJP, in float64."""
    d = O.make_inputs(1, T, 1, 2, 16, seed=T + 1, s0_std=s0, dtype=np.float64)
    rng = np.random.default_rng(T)
    decay = np.exp(-rng.uniform(0.0, 1.5, (1, T, 2, 16)))
    dS_T = rng.standard_normal(d["state"].shape) * 0.3
    (y, S), (dq, dk, dv, dg, db, dS0) = O.gated_delta_chunked_vjp(
        d["q"], d["k"], d["v"], decay, d["beta"], d["state"], None, d["dy"], dS_T, chunk=64, dtype=np.float64)
    outs = []
    for h in range(2):
        out = chunk_model.vg_run(d["q"][0, :, 0], d["k"][0, :, 0], d["v"][0, :, h], np.log(decay[0, :, h]),
                                 d["beta"][0, :, h], d["state"][0, h], d["dy"][0, :, h], dS_T[0, h])
        outs.append(out)
        want = (y[0, :, h], S[0, h], None, None, dv[0, :, h], dg[0, :, h] * decay[0, :, h], db[0, :, h], dS0[0, h])
        for name, a, b in zip(("y", "S", "dq", "dk", "dv", "dg", "db", "dS0"), out, want):
            if b is not None:
                np.testing.assert_allclose(a, b, atol=1e-9, rtol=1e-7, err_msg=name)
    np.testing.assert_allclose(outs[0][2] + outs[1][2], dq[0, :, 0], atol=1e-9, rtol=1e-7)
    np.testing.assert_allclose(outs[0][3] + outs[1][3], dk[0, :, 0], atol=1e-9, rtol=1e-7)


@pytest.mark.parametrize("T,zeros,top", [(64, 0.0, 1.5), (100, 0.0, 1.5), (100, 0.05, 1.5), (130, 0.02, 0.05)])
def test_vector_gate_decay_gradient_without_division(T, zeros, top):
    """vg_dg_decay forms d/d(decay) from factors <= 1: it equals d/d(log decay) / decay where both are defined, and
    at zero decays (a log decay of -1e4, whose exponential is exactly 0) it equals the oracle's per-channel
    recurrence, which differentiates the decay directly (S * decay, tools/gdn_vjp.py:174-179).  float64, two
    value heads, decays exp(-U(0, top)) with a fraction set to zero; top = 0.05 keeps the terms that span whole
    blocks (M_U, T0, the exit pair) large enough that leaving any one out fails the check.  The blocked
    restatement (the order of the GPU kernel) is held to the same bar."""
    d = O.make_inputs(1, T, 1, 2, 16, seed=T + 7, s0_std=0.5, dtype=np.float64)
    rng = np.random.default_rng(T + 3)
    decay = np.exp(-rng.uniform(0.0, top, (1, T, 2, 16)))
    decay[rng.random(decay.shape) < zeros] = 0.0
    g_log = np.where(decay > 0, np.log(np.where(decay > 0, decay, 1.0)), -1e4)
    dS_T = rng.standard_normal(d["state"].shape) * 0.3
    (_, _), (_, _, _, dg, _, _) = O.gated_delta_chunked_vjp(
        d["q"], d["k"], d["v"], decay, d["beta"], d["state"], None, d["dy"], dS_T, chunk=64, dtype=np.float64)
    for h in range(2):
        args = (d["q"][0, :, 0], d["k"][0, :, 0], d["v"][0, :, h], g_log[0, :, h], d["beta"][0, :, h],
                d["state"][0, h], d["dy"][0, :, h], dS_T[0, h])
        x = chunk_model.vg_run(*args, decay_grad=True)[5]
        np.testing.assert_allclose(x, dg[0, :, h], atol=1e-9, rtol=1e-7)
        xb = chunk_model.vg_run(*args, decay_grad="blocked")[5]
        np.testing.assert_allclose(xb, dg[0, :, h], atol=1e-9, rtol=1e-7)
        if not zeros:
            dgl = chunk_model.vg_run(*args)[5]
            np.testing.assert_allclose(x * decay[0, :, h], dgl, atol=1e-9, rtol=1e-7)
