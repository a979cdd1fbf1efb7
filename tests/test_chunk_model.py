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
