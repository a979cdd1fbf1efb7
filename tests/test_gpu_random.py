"""GPU parity over seeded random combinations of the call's options, each against the fp64 oracle.

Every case draws: the form (chunked, token-recurrent, or the default choice), the head size (128 on the chunked
form; 32, 64 or 128 on the recurrent one), the input dtype (fp32, or bf16 with an fp32 state), B (1..3), T (1..300),
the GQA layout (Hk 1-2, Hv/Hk 1, 2 or 4), the gate (log or decay space per head, or one decay per key channel: on the
chunked form with bf16 inputs and no mask, else on the recurrent form), the mask (none, random, or a masked tail), the snapshot interval `chunk` (16, 64, 100, 256),
a zero or random initial state and a zero or random exit-state cotangent.  Eight more draws run at B = 1,
T = 1000..3000 (several checkpoint windows and groups), and twelve put per-channel gates on the chunked form (bf16,
no mask) with the layout, B, T up to 1500, chunk and states drawn.  Bars, as normalised error max|gpu - oracle| / max|oracle|
per output, are set by each output's arithmetic (``bar``): 1e-4 for fp32 inputs and for the fp32 outputs of the
token-recurrent form with bf16 inputs, 4e-3 for that form's bf16 dq / dk / dv, 1e-2 on the chunked form with bf16
inputs.
"""

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

NAMES = ("y", "S_T", "dq", "dk", "dv", "dg", "dbeta", "dS0")
N_CASES = 32
N_LONG = 8  # B = 1, T in 1000..3000: several checkpoint windows and groups
N_VEC = 12  # per-channel gates on the chunked form


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import gdn_lib
    gdn_lib.load()
    return torch.device("cuda:0")


def draw(i, long=False):
    rng = np.random.default_rng((9000 if long else 5000) + i)
    form = ("chunk", "recurrent", "auto")[rng.integers(3)]
    vector = bool(rng.random() < 0.3)
    D = 128 if form != "recurrent" else int(rng.choice([32, 64, 128]))
    bf16 = bool(rng.random() < 0.5)
    B, T = (1, int(rng.integers(1000, 3001))) if long else (int(rng.integers(1, 4)), int(rng.integers(1, 301)))
    Hk = int(rng.integers(1, 3))
    Hv = Hk * int(rng.choice([1, 2, 4]))
    mask_kind = ("none", "random", "tail")[rng.integers(3)]
    if vector and form == "chunk" and not (bf16 and mask_kind == "none"):
        form = "auto"  # the chunked form takes per-channel gates with bf16 inputs and no mask only
    chunk = int(rng.choice([16, 64, 100, 256]))
    log_gate = (not vector) and bool(rng.random() < 0.5)
    s0 = bool(rng.random() < 0.5)
    dS = bool(rng.random() < 0.5)
    return dict(form=form, vector=vector, D=D, bf16=bf16, B=B, T=T, Hk=Hk, Hv=Hv, mask=mask_kind, chunk=chunk,
                log_gate=log_gate, s0=s0, dS=dS, seed=(8000 if long else 7000) + i)


def draw_vector_chunked(i):
    """One decay per key channel on the chunked form (bf16, no mask, D = 128): GQA layout, B, T (up to 1500, so
    several checkpoint windows and groups), chunk, S0 and the exit cotangent drawn."""
    rng = np.random.default_rng(6000 + i)
    form = ("chunk", "auto")[rng.integers(2)]
    B, T = int(rng.integers(1, 4)), int(rng.integers(1, 1501))
    Hk = int(rng.integers(1, 3))
    Hv = Hk * int(rng.choice([1, 2, 4]))
    chunk = int(rng.choice([16, 64, 100, 256]))
    s0 = bool(rng.random() < 0.5)
    dS = bool(rng.random() < 0.5)
    return dict(form=form, vector=True, D=128, bf16=True, B=B, T=T, Hk=Hk, Hv=Hv, mask="none", chunk=chunk,
                log_gate=False, s0=s0, dS=dS, seed=7500 + i)


def chunked(c):
    """Whether the case runs on the chunked form (what gdn_select_form picks for it)."""
    if c["form"] == "recurrent" or c["D"] != 128:
        return False
    if c["vector"]:
        return c["bf16"] and c["mask"] == "none"
    return True


def inputs(c):
    d = O.make_inputs(c["B"], c["T"], c["Hk"], c["Hv"], c["D"], seed=c["seed"], s0_std=0.05 if c["s0"] else 0.0)
    rng = np.random.default_rng(c["seed"] + 1)
    if c["vector"]:
        d["decay"] = np.exp(-rng.uniform(0.0, 1.5, (c["B"], c["T"], c["Hv"], c["D"]))).astype(np.float32)
    d["dS_T"] = ((rng.standard_normal(d["state"].shape) * 0.1).astype(np.float32) if c["dS"]
                 else np.zeros_like(d["state"]))
    if c["mask"] == "random":
        d["mask"] = rng.random((c["B"], c["T"])) > 0.25
    elif c["mask"] == "tail":
        d["mask"] = np.ones((c["B"], c["T"]), bool)
        d["mask"][:, c["T"] - max(1, c["T"] // 8):] = False
    else:
        d["mask"] = None
    if c["bf16"]:
        bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
        d = dict(d, q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), dy=bf(d["dy"]))
    return d


def run_engine(c, d, dev):
    import gdn_engine
    dt = torch.bfloat16 if c["bf16"] else torch.float32
    t = lambda x, ty=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=ty)
    q, k, v = (t(d[n], dt).requires_grad_(True) for n in ("q", "k", "v"))
    g = t(d["g_log"] if c["log_gate"] else d["decay"]).requires_grad_(True)
    beta, S0 = (t(d[n]).requires_grad_(True) for n in ("beta", "state"))
    mask = None if d["mask"] is None else torch.tensor(d["mask"], device=dev)
    form = None if c["form"] == "auto" else c["form"]
    y, S = gdn_engine.recurrence(q, k, v, g, beta, S0, mask, c["chunk"], log_gate=c["log_gate"], form=form)
    grads = torch.autograd.grad([y, S], [q, k, v, g, beta, S0], [t(d["dy"], y.dtype), t(d["dS_T"])])
    torch.cuda.synchronize()
    return [x.detach().float().cpu().numpy() for x in (y, S, *grads)]


def nerr(a, b):
    if not b.size:
        return 0.0
    return float(np.abs(a - b).max()) / max(float(np.abs(b).max()), 1e-30)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_combination_against_oracle(dev, i):
    check(draw(i), dev, i)


@pytest.mark.parametrize("i", range(N_LONG))
def test_random_long_combination_against_oracle(dev, i):
    check(draw(i, long=True), dev, i)


@pytest.mark.parametrize("i", range(N_VEC))
def test_random_vector_gate_chunked_against_oracle(dev, i):
    c = draw_vector_chunked(i)
    assert chunked(c)
    check(c, dev, i)


def check(c, dev, i):
    print("case", i, c, flush=True)
    d = inputs(c)
    got = run_engine(c, d, dev)
    (y, S), g = O.gated_delta_chunked_vjp(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], d["mask"],
                                          d["dy"], d["dS_T"], chunk=c["chunk"], dtype=np.float64)
    want = [y, S, *g]
    if c["log_gate"]:
        want[5] = want[5] * d["decay"]  # the oracle's d/d(decay) -> d/d(log decay), what the engine returns
    errs = {}
    for n, a, w in zip(NAMES, got, want):
        assert a.shape == w.shape, (n, a.shape, w.shape)
        errs[n] = nerr(a, w)
    print("  errors", {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= bar(c, n), (i, n, e, bar(c, n), c)


def bar(c, name):
    """The bar each output's arithmetic sets.  fp32 inputs: 1e-4.  bf16 inputs on the token-recurrent form (the
    oracle sees the same bf16-rounded inputs and the recurrence runs in fp32): 1e-4 for the fp32 outputs y, S_T, dg,
    dbeta and dS0, and 4e-3 for dq, dk and dv, which come back rounded to bf16 (2^-9 of an element, plus the fp32
    sums).  bf16 inputs on the chunked form, whose products take bf16 MFMA operands: 1e-2."""
    if not c["bf16"]:
        return 1e-4
    if chunked(c):
        return 1e-2
    return 4e-3 if name in ("dq", "dk", "dv") else 1e-4
