"""GPU parity with fp16 q / k / v (fp32 state and gates) against the fp64 oracle on the same fp16-rounded inputs.

fp16 inputs run the fp32 kernel sets, which read the element dtype from their arguments: the chunked form's fp32 set
at Dk = Dv = 128 (scalar gates, with or without a mask), the token-recurrent form otherwise (other head sizes,
per-channel gates).  The arithmetic is fp32, so the fp32 outputs (y, which promotes to fp32 as in the reference,
S_T, dg, dbeta, dS0) are held to the fp32 bar of 1e-4, and dq, dk, dv, returned in fp16, to 2e-3 (fp16 rounding is
2^-11 of an element).  Error: max|gpu - oracle| / max|oracle| per output.
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


def _inputs(B, T, Hk, Hv, D, seed, vector=False, mask=None):
    d = O.make_inputs(B, T, Hk, Hv, D, seed=seed, s0_std=0.05)
    rng = np.random.default_rng(seed + 1)
    if vector:
        d["decay"] = np.exp(-rng.uniform(0.0, 1.5, (B, T, Hv, D))).astype(np.float32)
    d["dS_T"] = (rng.standard_normal(d["state"].shape) * 0.1).astype(np.float32)
    if mask == "random":
        d["mask"] = rng.random((B, T)) > 0.25
    elif mask == "tail":
        d["mask"] = np.ones((B, T), bool)
        d["mask"][:, T - max(1, T // 8):] = False
    else:
        d["mask"] = None
    h = lambda x: torch.tensor(x).half().float().numpy()
    return dict(d, q=h(d["q"]), k=h(d["k"]), v=h(d["v"]))


def _run(d, dev, chunk, form=None):
    import gdn_engine
    t = lambda x, ty=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=ty)
    q, k, v = (t(d[n], torch.float16).requires_grad_(True) for n in ("q", "k", "v"))
    g, beta, S0 = (t(d[n]).requires_grad_(True) for n in ("decay", "beta", "state"))
    mask = None if d["mask"] is None else torch.tensor(d["mask"], device=dev)
    y, S = gdn_engine.recurrence(q, k, v, g, beta, S0, mask, chunk, form=form)
    assert y.dtype == torch.float32
    grads = torch.autograd.grad([y, S], [q, k, v, g, beta, S0], [t(d["dy"], y.dtype), t(d["dS_T"])])
    assert grads[0].dtype == torch.float16 and grads[2].dtype == torch.float16
    torch.cuda.synchronize()
    return [x.detach().float().cpu().numpy() for x in (y, S, *grads)]


def _check(d, got, chunk, label):
    (y, S), g = O.gated_delta_chunked_vjp(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], d["mask"],
                                          d["dy"], d["dS_T"], chunk=chunk, dtype=np.float64)
    errs = {}
    for n, a, w in zip(NAMES, got, [y, S, *g]):
        errs[n] = float(np.abs(a - w).max()) / max(float(np.abs(w).max()), 1e-30)
    print(label, {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= (2e-3 if n in ("dq", "dk", "dv") else 1e-4), (label, n, e)


@pytest.mark.parametrize("T", [1, 65, 200])
@pytest.mark.parametrize("mask", [None, "tail"])
def test_fp16_inputs_on_the_chunked_form(dev, T, mask):
    import gdn_lib as L
    assert L.load().gdn_select_form(4, 128, 128, int(mask is not None), L.GATE_DECAY, L.FORM_AUTO,
                                    L.F16) == L.FORM_CHUNK
    d = _inputs(2, T, 2, 4, 128, seed=400 + T, mask=mask)
    print(f"fp16 chunked T={T} mask={mask}", flush=True)
    _check(d, _run(d, dev, 64, form="chunk"), 64, f"fp16 chunked T={T} mask={mask}")


def test_fp16_inputs_checkpointed_on_the_chunked_form(dev):
    d = _inputs(1, 700, 2, 4, 128, seed=410)
    print("fp16 chunked T=700 chunk=256", flush=True)
    _check(d, _run(d, dev, 256, form="chunk"), 256, "fp16 chunked ckpt")


@pytest.mark.parametrize("D, vector, mask", [(64, False, "random"), (128, True, None), (32, True, "tail")])
def test_fp16_inputs_on_the_recurrent_form(dev, D, vector, mask):
    d = _inputs(2, 150, 2, 4, D, seed=420 + D, vector=vector, mask=mask)
    print(f"fp16 recurrent D={D} vector={vector} mask={mask}", flush=True)
    _check(d, _run(d, dev, 64), 64, f"fp16 recurrent D={D} vector={vector} mask={mask}")
