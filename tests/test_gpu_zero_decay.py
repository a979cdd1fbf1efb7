"""Zero decays (and log decays of -inf) against the fp64 oracle.

A zero decay erases the state at its token (tools/gdn_vjp.py:174-179: S * decay), and d/d(decay) there is
sum dA * S_prev, which is not zero.  The chunked form works with cumulative log decays, so it takes a decay below 2^-64
as 2^-64: the forward changes by 2^-64 of a state, and with scalar gates d/d(decay) = d/d(log decay) / 2^-64 is the
derivative at the zero up to terms of that size (every pair term that straddles the token carries the factor).
Per-channel decays form d/d(decay) in ck_vg_dg from factors <= 1, with no division.  Cases: scalar decays with zeros
scattered over the sequence (fp32 and bf16, with and without a masked tail) on the chunked form, per-channel decays
with zeros (bf16, automatic choice: the chunked form), log decays with -inf entries, and a checkpointed call.  The
oracle runs the token recurrence itself.  Bars (normalised error max|gpu - oracle| / max|oracle| per output): 1e-4 at
fp32 and 1e-2 on the chunked form with bf16 inputs.
"""

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

NAMES = ("y", "S_T", "dq", "dk", "dv", "dg", "dbeta", "dS0")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import gdn_lib
    gdn_lib.load()
    return torch.device("cuda:0")


def _inputs(B, T, Hk, Hv, seed, bf16, vector=False, mask=False, frac=0.05):
    d = O.make_inputs(B, T, Hk, Hv, 128, seed=seed, s0_std=0.05)
    rng = np.random.default_rng(seed + 1)
    if vector:
        d["decay"] = np.exp(-rng.uniform(0.0, 1.5, (B, T, Hv, 128))).astype(np.float32)
    zero = rng.random(d["decay"].shape) < frac
    d["decay"] = np.where(zero, 0.0, d["decay"]).astype(np.float32)
    with np.errstate(divide="ignore"):
        d["g_log"] = np.log(d["decay"]).astype(np.float32)
    d["dS_T"] = (rng.standard_normal(d["state"].shape) * 0.1).astype(np.float32)
    if mask:
        d["mask"] = np.ones((B, T), bool)
        d["mask"][:, T - max(1, T // 8):] = False
    else:
        d["mask"] = None
    if bf16:
        bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
        d = dict(d, q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), dy=bf(d["dy"]))
    assert zero.any()
    return d


def _run(d, dev, bf16, chunk=64, log_gate=False, form="chunk"):
    import gdn_engine
    dt = torch.bfloat16 if bf16 else torch.float32
    t = lambda x, ty=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=ty)
    q, k, v = (t(d[n], dt).requires_grad_(True) for n in ("q", "k", "v"))
    g = t(d["g_log"] if log_gate else d["decay"]).requires_grad_(True)
    beta, S0 = (t(d[n]).requires_grad_(True) for n in ("beta", "state"))
    mask = None if d["mask"] is None else torch.tensor(d["mask"], device=dev)
    y, S = gdn_engine.recurrence(q, k, v, g, beta, S0, mask, chunk, log_gate=log_gate, form=form)
    grads = torch.autograd.grad([y, S], [q, k, v, g, beta, S0], [t(d["dy"], y.dtype), t(d["dS_T"])])
    torch.cuda.synchronize()
    return [x.detach().float().cpu().numpy() for x in (y, S, *grads)]


def _check(d, got, bf16, label, chunk=64, log_gate=False):
    (y, S), g = O.gated_delta_chunked_vjp(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], d["mask"],
                                          d["dy"], d["dS_T"], chunk=chunk, dtype=np.float64)
    want = [y, S, *g]
    if log_gate:
        want[5] = want[5] * d["decay"]  # d/d(log decay) = d/d(decay) * decay: 0 where the decay is 0
    errs = {}
    for n, a, w in zip(NAMES, got, want):
        assert np.isfinite(a).all(), (label, n)
        errs[n] = float(np.abs(a - w).max()) / max(float(np.abs(w).max()), 1e-30)
    print(label, {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= (1e-2 if bf16 else 1e-4), (label, n, e)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("mask", [False, True])
def test_zero_scalar_decays(dev, bf16, mask):
    d = _inputs(2, 300, 2, 4, seed=500 + 2 * bf16 + mask, bf16=bf16, mask=mask)
    print(f"zero decays bf16={bf16} mask={mask}", flush=True)
    _check(d, _run(d, dev, bf16), bf16, f"zero decays bf16={bf16} mask={mask}")


def test_zero_per_channel_decays(dev):
    import gdn_lib as L
    assert L.load().gdn_select_form(4, 128, 128, 0, L.GATE_DECAY_VEC, L.FORM_AUTO, L.BF16) == L.FORM_CHUNK
    d = _inputs(2, 300, 2, 4, seed=510, bf16=True, vector=True, frac=0.01)
    print("zero per-channel decays, automatic form", flush=True)
    _check(d, _run(d, dev, True, form=None), True, "zero per-channel decays")


@pytest.mark.parametrize("bf16", [False, True])
def test_minus_inf_log_decays(dev, bf16):
    d = _inputs(1, 200, 2, 4, seed=520 + bf16, bf16=bf16)
    print(f"-inf log decays bf16={bf16}", flush=True)
    _check(d, _run(d, dev, bf16, log_gate=True), bf16, f"-inf log decays bf16={bf16}", log_gate=True)


def test_zero_decays_checkpointed(dev):
    d = _inputs(1, 700, 2, 4, seed=530, bf16=False)
    print("zero decays chunk=256", flush=True)
    _check(d, _run(d, dev, False, chunk=256), False, "zero decays ckpt", chunk=256)
