"""GPU parity of the decode path: the one-token step (gdn_decode_step, the counterpart of gdn_recurrent_step,
engine/include/gdn.h:27-38, engine/src/gdn.c:63-108), the conv and recurrent state caches of
qwen3_5.GatedDeltaNet, and token-by-token decoding of the tiny model.

* token-by-token decode matches the fp64 oracle (1e-4 with fp32 or bf16 inputs: its arithmetic and y are fp32) and
  equals the full-sequence forward (1e-2 where that runs the chunked form on bf16 inputs, else 1e-4);
* a prefill of part of a sequence followed by one call per token, through the block's caches, equals the block's
  full-sequence forward, which the float64 block oracle pins (frozen / eval path at Dk = Dv = 128, chunked form);
* the tiny model's logits decoded one token at a time equal its full forward.
"""

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O
from oracle import gdn_block_oracle as BO

pytestmark = pytest.mark.gpu


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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("Hk,Hv,D,gate", [(2, 4, 128, "log"), (2, 4, 128, "decay"), (1, 3, 32, "vector"),
                                          (2, 2, 8, "decay"), (2, 4, 100, "log"), (1, 2, 96, "vector"),
                                          (1, 2, 128, "logvec"), (1, 3, 32, "logvec")])
def test_decode_steps_match_sequence_and_oracle(dev, dtype, Hk, Hv, D, gate):
    """gate: log or decay per head, a decay per key channel, or a log decay per key channel (exp(-U(0, 8)), about 2%
    of them -inf, a zero decay)."""
    import gdn_engine
    B, T = 2, 20
    d = O.make_inputs(B, T, Hk, Hv, D, seed=D + Hv, s0_std=0.05)
    if gate == "vector":
        rng = np.random.default_rng(3)
        d["decay"] = rng.uniform(0.5, 1.0, (B, T, Hv, D)).astype(np.float32)
    elif gate == "logvec":
        rng = np.random.default_rng(4)
        gl = -rng.uniform(0.0, 8.0, (B, T, Hv, D))
        gl[rng.random(gl.shape) < 0.02] = -np.inf
        d["g_log"] = gl.astype(np.float32)
        d["decay"] = np.exp(gl).astype(np.float32)
    if dtype == torch.bfloat16:
        bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
        d = dict(d, q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]))
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    q, k, v = (t(d[n], dtype) for n in ("q", "k", "v"))
    log_gate = gate in ("log", "logvec")
    g = t(d["g_log"]) if log_gate else t(d["decay"])
    beta, S0 = t(d["beta"]), t(d["state"])
    print(f"decode {dtype} Hk={Hk} Hv={Hv} D={D} gate={gate}", flush=True)
    state = S0.clone()
    ys = []
    for i in range(T):
        ys.append(gdn_engine.decode_step(q[:, i], k[:, i], v[:, i], g[:, i], beta[:, i], state, state, log_gate,
                                         torch.float32))
    y_dec = torch.stack(ys, 1)
    with torch.no_grad():
        y_seq, S_seq = gdn_engine.recurrence(q, k, v, g, beta, S0, None, 64, log_gate=log_gate,
                                             output_dtype=torch.float32)
    torch.cuda.synchronize()
    wy, wS = O.gated_delta_chunked(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], None, 64,
                                   dtype=np.float64)
    # the decode step computes in fp32 from the same bf16-rounded inputs the oracle sees, and returns y in fp32: 1e-4
    # with either input dtype.  The sequence forward runs the chunked form at D = 128, whose bf16 inputs enter bf16
    # MFMA products: 1e-2 there.
    seq_tol = 1e-2 if dtype == torch.bfloat16 and D == 128 else 1e-4
    errs = dict(y=nerr(y_dec.cpu().numpy(), wy), S=nerr(state.cpu().numpy(), wS),
                y_seq=nerr(y_dec.cpu().numpy(), y_seq.cpu().numpy()),
                S_seq=nerr(state.cpu().numpy(), S_seq.cpu().numpy()))
    print("  errors", {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    assert errs["y"] <= 1e-4 and errs["S"] <= 1e-4, errs
    assert errs["y_seq"] <= seq_tol and errs["S_seq"] <= seq_tol, errs


def test_decode_step_out_of_place_and_zero_state(dev):
    """state_out distinct from state_in leaves state_in untouched; state_in = None starts from zeros."""
    import gdn_engine
    d = O.make_inputs(3, 1, 2, 4, 64, seed=5, s0_std=0.1)
    t = lambda x: torch.tensor(np.asarray(x), device=dev)
    S0 = t(d["state"])
    keep = S0.clone()
    out = torch.empty_like(S0)
    y = gdn_engine.decode_step(t(d["q"])[:, 0], t(d["k"])[:, 0], t(d["v"])[:, 0], t(d["decay"])[:, 0],
                               t(d["beta"])[:, 0], S0, out)
    out0 = torch.empty_like(S0)
    y0 = gdn_engine.decode_step(t(d["q"])[:, 0], t(d["k"])[:, 0], t(d["v"])[:, 0], t(d["decay"])[:, 0],
                                t(d["beta"])[:, 0], None, out0)
    torch.cuda.synchronize()
    assert torch.equal(S0, keep)
    wy, wS = O.gated_delta_chunked(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], None, 64,
                                   dtype=np.float64)
    assert nerr(y.cpu().numpy(), wy[:, 0]) <= 1e-5 and nerr(out.cpu().numpy(), wS) <= 1e-5
    wy0, wS0 = O.gated_delta_chunked(d["q"], d["k"], d["v"], d["decay"], d["beta"], None, None, 64,
                                     dtype=np.float64)
    assert nerr(y0.cpu().numpy(), wy0[:, 0]) <= 1e-5 and nerr(out0.cpu().numpy(), wS0) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_prefill_then_decode(dev, dtype):
    """GatedDeltaNet at Dk = Dv = 128 (chunked prefill, decode steps): a 24-token prefill through the caches, then
    one call per token, equals the full-sequence forward; the full forward matches the float64 block oracle."""
    import qwen3_5 as Q
    from test_gpu_block import build_block
    h, Hk, Hv, D = 256, 2, 4, 128
    B, T, T0 = 2, 40, 24
    P = BO.make_block_params(h, Hk, Hv, D, D, seed=11)
    x = np.random.default_rng(12).standard_normal((B, T, h)).astype(np.float32)
    blk = build_block(P, h, Hk, Hv, D, D, dev, dtype, 0, 1.0).eval()
    tx = torch.tensor(x, device=dev, dtype=dtype)
    with torch.no_grad():
        full = blk(tx)
        cache = Q.GDNCache()
        parts = [blk(tx[:, :T0], cache=cache)]
        for i in range(T0, T):
            parts.append(blk(tx[:, i:i + 1], cache=cache))
    torch.cuda.synchronize()
    dec = torch.cat(parts, 1).float().cpu().numpy()
    assert cache[0].shape == (B, 3, 2 * Hk * D + Hv * D) and cache[1].shape == (B, Hv, D, D)
    tol = 3e-2 if dtype == torch.bfloat16 else 1e-4
    want, _ = BO.block_forward(x, P, Hk, Hv, D, D)
    print(f"block decode {dtype}: full vs oracle {nerr(full.float().cpu().numpy(), want):.1e}, "
          f"decode vs full {nerr(dec, full.float().cpu().numpy()):.1e}", flush=True)
    assert nerr(full.float().cpu().numpy(), want) <= tol
    assert nerr(dec, full.float().cpu().numpy()) <= (1e-2 if dtype == torch.bfloat16 else 1e-5)


def test_tiny_model_decodes_token_by_token(dev):
    """The tiny Qwen3.5 stack (GDN layers with Dk = Dv = 8, attention layers with a KV cache): logits of a prefill
    plus one call per token equal the logits of the full forward."""
    import qwen3_5 as Q
    torch.manual_seed(0)
    model = Q.Model(Q.ModelArgs()).to(dev).eval()
    tokens = torch.randint(0, 1000, (2, 12), device=dev)
    with torch.no_grad():
        full = model(tokens)
        cache = model.make_cache()
        parts = [model(tokens[:, :5], cache=cache)]
        for i in range(5, 12):
            parts.append(model(tokens[:, i:i + 1], cache=cache))
    torch.cuda.synchronize()
    assert nerr(torch.cat(parts, 1).cpu().numpy(), full.cpu().numpy()) <= 1e-5
