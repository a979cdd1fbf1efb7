"""Writes tests/golden/gdn_vjp_cases.npz: inputs and float64 forward + VJP results of the delta-rule
recurrence computed by torch autograd of the independent statement in tests/naive_torch.py.

The reference stores no backward vectors (its VJP tests recompute MLX autodiff at run time,
tools/test_gdn_vjp.py:96-138), so these vectors are produced by a library autodiff here.  Input
distributions follow tools/test_gdn_vjp.py:21-55 (q,k L2-normalised, q scaled by Dk^-1/2, decay ~ U(0.7,1),
beta ~ U(0.05,0.95), S0 ~ N(0,1), mask = uniform > 0.2), plus two cases with the measured workloads'
gates (log decay -exp(A_log) softplus(a)).

Run:  python tests/golden/make_golden.py
"""

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import naive_torch  # noqa: E402

CASES = [
    # name,           B, T,  Hk, Hv, Dk, Dv, gate_ndim, masked, gates
    ("tiny_scalar",   2, 7,  2,  4,  3,  5,  3, False, "uniform"),
    ("tiny_masked",   2, 9,  2,  4,  3,  5,  3, True,  "uniform"),
    ("tiny_vector",   2, 6,  2,  4,  3,  5,  4, True,  "uniform"),
    ("gqa_d16",       1, 33, 2,  4,  16, 16, 3, False, "uniform"),
    ("d32_loggate",   1, 40, 1,  2,  32, 32, 3, False, "loggate"),
    ("d32_masked",    2, 21, 2,  2,  32, 8,  3, True,  "loggate"),
    ("d128_short",    1, 5,  1,  2,  128, 128, 3, False, "loggate"),
]


def l2n(x, scale):
    return scale * x / np.sqrt((x.astype(np.float64) ** 2).sum(-1, keepdims=True) + 1e-6)


def make_case(seed, B, T, Hk, Hv, Dk, Dv, gate_ndim, masked, gates):
    rng = np.random.default_rng(seed)
    q = l2n(rng.standard_normal((B, T, Hk, Dk)), Dk ** -0.5)
    k = l2n(rng.standard_normal((B, T, Hk, Dk)), 1.0)
    v = rng.standard_normal((B, T, Hv, Dv))
    gshape = (B, T, Hv) + ((Dk,) if gate_ndim == 4 else ())
    if gates == "uniform":
        g = rng.uniform(0.7, 1.0, gshape)
        beta = rng.uniform(0.05, 0.95, (B, T, Hv))
    else:
        A_log = rng.uniform(0.0, math.log(16.0), (Hv,))
        a = rng.standard_normal((B, T, Hv))
        sp = np.log1p(np.exp(a))
        g = np.exp(-np.exp(A_log) * sp)
        beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, Hv))))
    state = rng.standard_normal((B, Hv, Dv, Dk))
    mask = (rng.random((B, T)) > 0.2) if masked else None
    dy = rng.standard_normal((B, T, Hv, Dv))
    dstate = rng.standard_normal((B, Hv, Dv, Dk))
    f32 = lambda x: np.asarray(x, np.float32)
    inputs = dict(q=f32(q), k=f32(k), v=f32(v), g=f32(g), beta=f32(beta), state=f32(state),
                  dy=f32(dy), dstate=f32(dstate))
    out = naive_torch.vjp(inputs["q"], inputs["k"], inputs["v"], inputs["g"], inputs["beta"],
                          inputs["state"], mask, inputs["dy"], inputs["dstate"])
    names = ("y", "S_T", "dq", "dk", "dv", "dg", "dbeta", "dS0")
    expected = {f"exp_{n}": x for n, x in zip(names, out)}
    if mask is not None:
        inputs["mask"] = mask
    return inputs, expected


def main():
    arrays = {}
    for i, (name, *cfg) in enumerate(CASES):
        inputs, expected = make_case(1000 + i, *cfg)
        for key, val in {**inputs, **expected}.items():
            arrays[f"{name}/{key}"] = val
    np.savez_compressed(HERE / "gdn_vjp_cases.npz", **arrays)
    print("wrote", HERE / "gdn_vjp_cases.npz", len(arrays), "arrays")


if __name__ == "__main__":
    main()
