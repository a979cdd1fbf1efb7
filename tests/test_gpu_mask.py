"""GPU parity of masked calls on the chunked form (two chunked passes over the effective gates plus the masked
tokens' fix-up, gdn_mask.hip), against the fp64 oracle's masked recurrence (tools/gdn_vjp.py:3-6, :247-256):
the reference's sequence lengths T in {1, 63, 64, 65, 200} at Dk = Dv = 128, fp32 (1e-4) and bf16 q/k/v/dO (1e-2),
checkpointed (chunk 256) and forward-only calls, and the measured head layout at T = 4096 against the recurrent
form.
"""

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

D = 128
NAMES = ("y", "S_T", "dq", "dk", "dv", "dg", "dbeta", "dS0")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import gdn_lib
    gdn_lib.load()
    return torch.device("cuda:0")


def nerr(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max()) / max(float(np.abs(b).max()), 1e-30)


def _inputs(B, T, Hk, Hv, seed, bf16=False):
    d = O.make_inputs(B, T, Hk, Hv, D, seed=seed, s0_std=0.05)
    rng = np.random.default_rng(seed + 1)
    mask = rng.uniform(size=(B, T)) > 0.3
    if T > 4:
        mask[0, :3] = False           # left padding
        mask[-1, T - 4:] = False      # right padding
    d["mask"] = mask
    d["dS_T"] = (rng.standard_normal(d["state"].shape) * 0.1).astype(np.float32)
    if bf16:
        bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
        d = dict(d, q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), dy=bf(d["dy"]))
    return d


def _gpu(d, dev, chunk=64, dtype=torch.float32, log_gate=True, form="auto", state_grad=True):
    import gdn_engine
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    q, k, v = (t(d[n], dtype).requires_grad_(True) for n in ("q", "k", "v"))
    g = t(d["g_log"] if log_gate else d["decay"]).requires_grad_(True)
    beta, S0 = t(d["beta"]).requires_grad_(True), t(d["state"]).requires_grad_(True)
    mask = torch.tensor(d["mask"], device=dev)
    y, S = gdn_engine.recurrence(q, k, v, g, beta, S0, mask, chunk, log_gate=log_gate, output_dtype=dtype,
                                 form=form)
    outs, cots = [y], [t(d["dy"], dtype)]
    if state_grad:
        outs.append(S)
        cots.append(t(d["dS_T"]))
    grads = torch.autograd.grad(outs, [q, k, v, g, beta, S0], cots)
    torch.cuda.synchronize()
    return [x.detach().float().cpu().numpy() for x in (y, S, *grads)]


def _oracle(d, hk, rep, b, log_gate=True, dS_T=True):
    sl = slice(hk * rep, hk * rep + rep)
    (y, S), g = O.gated_delta_chunked_vjp(
        d["q"][b:b + 1, :, hk:hk + 1], d["k"][b:b + 1, :, hk:hk + 1], d["v"][b:b + 1, :, sl],
        d["decay"][b:b + 1, :, sl], d["beta"][b:b + 1, :, sl], d["state"][b:b + 1, sl], d["mask"][b:b + 1],
        d["dy"][b:b + 1, :, sl], d["dS_T"][b:b + 1, sl] if dS_T else None, chunk=64, dtype=np.float64)
    dg = g[3] * d["decay"][b:b + 1, :, sl] if log_gate else g[3]
    return [y, S, g[0], g[1], g[2], dg, g[4], g[5]]


def _slice(got, hk, rep, b):
    sl = slice(hk * rep, hk * rep + rep)
    return [got[0][b:b + 1, :, sl], got[1][b:b + 1, sl], got[2][b:b + 1, :, hk:hk + 1],
            got[3][b:b + 1, :, hk:hk + 1], got[4][b:b + 1, :, sl], got[5][b:b + 1, :, sl],
            got[6][b:b + 1, :, sl], got[7][b:b + 1, sl]]


def _check(got, d, groups, rep, tol, label, **kw):
    for b, hk in groups:
        want = _oracle(d, hk, rep, b, **kw)
        errs = {n: nerr(a, w) for n, a, w in zip(NAMES, _slice(got, hk, rep, b), want)}
        print(label, f"b={b} hk={hk}", {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
        for n, e in errs.items():
            assert e <= tol, (label, b, hk, n, e)


def test_masked_calls_select_the_chunked_form(dev):
    import gdn_lib as L
    lib = L.load()
    assert lib.gdn_select_form(32, 128, 128, 1, L.GATE_LOG, L.FORM_AUTO, L.F32) == L.FORM_CHUNK
    assert lib.gdn_select_form(32, 128, 128, 1, L.GATE_DECAY_VEC, L.FORM_AUTO, L.F32) == L.FORM_RECURRENT


def test_masked_call_above_256_value_heads_runs_recurrent(dev):
    """Hv = 260 with a mask: AUTO resolves to the recurrent form (the fix-up kernels of the chunked form hold at most
    256 heads of a token), and the result matches the oracle on two key-head groups."""
    import gdn_lib as L
    lib = L.load()
    assert lib.gdn_select_form(260, 128, 128, 1, L.GATE_LOG, L.FORM_AUTO, L.F32) == L.FORM_RECURRENT
    d = _inputs(1, 40, 130, 260, seed=260)
    print("masked Hv=260 T=40 fp32, auto form", flush=True)
    got = _gpu(d, dev)
    _check(got, d, ((0, 0), (0, 129)), 2, 1e-4, "masked Hv=260")


@pytest.mark.parametrize("T", [1, 63, 64, 65, 200])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_chunked_against_oracle(dev, T, dtype):
    bf = dtype == torch.bfloat16
    d = _inputs(2, T, 2, 4, seed=100 + T, bf16=bf)
    print(f"masked chunked {dtype} T={T}", flush=True)
    got = _gpu(d, dev, dtype=dtype)
    _check(got, d, ((0, 0), (1, 1)), 2, 1e-2 if bf else 1e-4, f"masked {dtype} T={T}")


@pytest.mark.parametrize("log_gate", [True, False])
def test_masked_chunked_decay_gate_and_null_cotangent(dev, log_gate):
    d = _inputs(2, 130, 1, 3, seed=7)
    got = _gpu(d, dev, log_gate=log_gate, state_grad=False)
    _check(got, d, ((0, 0), (1, 0)), 3, 1e-4, f"masked log_gate={log_gate} no dS_T", log_gate=log_gate,
           dS_T=False)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_checkpointed_against_oracle(dev, dtype):
    """chunk = 256: the forward keeps pass 1's window states only; the backward rebuilds both passes from them."""
    bf = dtype == torch.bfloat16
    d = _inputs(2, 600, 2, 4, seed=55, bf16=bf)
    got = _gpu(d, dev, chunk=256, dtype=dtype)
    _check(got, d, ((0, 1), (1, 0)), 2, 1e-2 if bf else 1e-4, f"masked ckpt {dtype}")
    full = _gpu(d, dev, chunk=64, dtype=dtype)
    for n, a, b in zip(NAMES, got, full):
        assert nerr(a, b) <= (2e-3 if bf else 1e-5), (n, nerr(a, b))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_forward_only_against_oracle(dev, dtype):
    import gdn_engine
    bf = dtype == torch.bfloat16
    d = _inputs(2, 150, 2, 4, seed=31, bf16=bf)
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    with torch.no_grad():
        y, S = gdn_engine.recurrence(t(d["q"], dtype), t(d["k"], dtype), t(d["v"], dtype), t(d["g_log"]),
                                     t(d["beta"]), t(d["state"]), torch.tensor(d["mask"], device=dev), 64,
                                     log_gate=True, output_dtype=dtype)
    wy, wS = O.gated_delta_chunked(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], d["mask"], 64,
                                   dtype=np.float64)
    tol = 1e-2 if bf else 1e-4
    assert nerr(y.float().cpu().numpy(), wy) <= tol
    assert nerr(S.cpu().numpy(), wS) <= tol


def test_masked_measured_layout_chunked_vs_recurrent(dev):
    """B=4, T=4096, Hk=16, Hv=32, bf16, the last 10% of each sequence masked (the masked bench workload): every
    output of the chunked form against the recurrent form (both pinned against the oracle above)."""
    d = O.make_inputs(4, 4096, 16, 32, D, seed=8, s0_std=0.02)
    mask = np.ones((4, 4096), bool)
    mask[:, 4096 - 409:] = False
    d["mask"] = mask
    d["dS_T"] = np.zeros_like(d["state"])
    print("masked B=4 T=4096 bf16 chunked vs recurrent", flush=True)
    a = _gpu(d, dev, dtype=torch.bfloat16, state_grad=False)
    b = _gpu(d, dev, dtype=torch.bfloat16, form="recurrent", state_grad=False)
    errs = {n: nerr(x, y) for n, x, y in zip(NAMES, a, b)}
    print({n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= 1e-2, (n, e)
