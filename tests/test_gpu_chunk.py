"""GPU parity of the chunked (WY/UT, MFMA) form.

* every intermediate the forward keeps (cumulative log decay G, T = (I+A)^-1, P, W, U, entry states, Delta)
  against the NumPy chunk model (tests/chunk_model.py, itself checked against the oracle on the CPU);
* forward + full VJP against the fp64 oracle: normalised error <= 1e-4 for fp32 inputs, <= 1e-2 for bf16
  q/k/v/dO with fp32 state;
* the chunked form against the recurrent form at the measured head layout.
"""

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O
import chunk_model

pytestmark = pytest.mark.gpu

C, D = 64, 128
NAMES = ("y", "S_T", "dq", "dk", "dv", "dg", "dbeta", "dS0")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import gdn_lib
    gdn_lib.load()
    return torch.device("cuda:0")


def nerr(a, b):
    return float(np.abs(a - b).max()) / max(float(np.abs(b).max()), 1e-30)


def _inputs(B, T, Hk, Hv, seed, s0_std, dtype=np.float32):
    d = O.make_inputs(B, T, Hk, Hv, D, seed=seed, s0_std=s0_std)
    d["dS_T"] = (np.random.default_rng(seed + 7).standard_normal(d["state"].shape) * 0.1).astype(np.float32)
    return d


def _gpu(d, dev, form, dtype=torch.float32, log_gate=True):
    import gdn_engine
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    q, k, v = (t(d[n], dtype).requires_grad_(True) for n in ("q", "k", "v"))
    g = t(d["g_log"] if log_gate else d["decay"]).requires_grad_(True)
    beta = t(d["beta"]).requires_grad_(True)
    S0 = t(d["state"]).requires_grad_(True)
    y, S = gdn_engine.recurrence(q, k, v, g, beta, S0, None, 64, log_gate=log_gate, output_dtype=dtype,
                                 form=form)
    grads = torch.autograd.grad([y, S], [q, k, v, g, beta, S0], [t(d["dy"], dtype), t(d["dS_T"])])
    torch.cuda.synchronize()
    return [x.detach().float().cpu().numpy() for x in (y, S, *grads)]


def _oracle_group(d, hk, rep, b=0, log_gate=True):
    sl = slice(hk * rep, hk * rep + rep)
    (y, S), g = O.gated_delta_chunked_vjp(
        d["q"][b:b + 1, :, hk:hk + 1], d["k"][b:b + 1, :, hk:hk + 1], d["v"][b:b + 1, :, sl],
        d["decay"][b:b + 1, :, sl], d["beta"][b:b + 1, :, sl], d["state"][b:b + 1, sl], None,
        d["dy"][b:b + 1, :, sl], d["dS_T"][b:b + 1, sl], chunk=64, dtype=np.float64)
    dg = g[3] * d["decay"][b:b + 1, :, sl] if log_gate else g[3]
    return [y, S, g[0], g[1], g[2], dg, g[4], g[5]]


def _slice(got, hk, rep, b=0):
    sl = slice(hk * rep, hk * rep + rep)
    return [got[0][b:b + 1, :, sl], got[1][b:b + 1, sl], got[2][b:b + 1, :, hk:hk + 1],
            got[3][b:b + 1, :, hk:hk + 1], got[4][b:b + 1, :, sl], got[5][b:b + 1, :, sl],
            got[6][b:b + 1, :, sl], got[7][b:b + 1, sl]]


def test_saved_intermediates_match_chunk_model(dev):
    """Run the forward through the C ABI and decode the saved buffer."""
    import gdn_lib as L
    B, T, Hk, Hv = 1, 150, 1, 2
    d = _inputs(B, T, Hk, Hv, seed=11, s0_std=0.3)
    lib = L.load()
    t = lambda x: torch.tensor(np.asarray(x), device=dev, dtype=torch.float32).contiguous()
    q, k, v, g, beta, S0 = (t(d[n]) for n in ("q", "k", "v", "g_log", "beta", "state"))
    y = torch.empty((B, T, Hv, D), device=dev)
    ST = torch.empty((B, Hv, D, D), device=dev)
    nbytes = lib.gdn_saved_bytes(B, T, Hk, Hv, D, D, 64, L.GATE_LOG, 0, L.FORM_CHUNK, L.F32)
    saved = torch.zeros(nbytes, device=dev, dtype=torch.uint8)
    assert lib.gdn_fwd_workspace_bytes(B, T, Hk, Hv, D, D, 64, L.GATE_LOG, 0, L.FORM_CHUNK, L.F32, 1) == 0
    L.check(lib.gdn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), S0.data_ptr(),
                        None, y.data_ptr(), ST.data_ptr(), saved.data_ptr(), nbytes, None, 0, B, T, Hk, Hv, D, D, 64,
                        L.F32, L.F32, L.GATE_LOG, L.FORM_CHUNK, None))
    torch.cuda.synchronize()
    raw = saved.cpu().numpy()
    NC = -(-T // C)
    al = lambda x: (x + 255) // 256 * 256
    # the fp32 set's buffers in their order (the bf16 operand tiles have no storage in this set)
    sizes = [("G", B * Hv * NC * C * 8, np.float64), ("U", B * Hv * NC * C * D * 4, np.float32),
             ("H", B * Hv * NC * D * D * 4, np.float32), ("Dl", B * Hv * NC * C * D * 4, np.float32),
             ("T", B * Hv * NC * C * C * 4, np.float32), ("P", B * Hv * NC * C * C * 4, np.float32),
             ("W", B * Hv * NC * C * D * 4, np.float32)]
    buf, off = {}, 0
    for name, n, dt in sizes:
        buf[name] = raw[off:off + n].view(dt)
        off += al(n)
    assert off == nbytes
    H = buf["H"].reshape(B, Hv, NC, D, D)
    G = buf["G"].reshape(B, Hv, NC, C)
    Tm = buf["T"].reshape(B, Hv, NC, C, C)
    P = buf["P"].reshape(B, Hv, NC, C, C)
    W = buf["W"].reshape(B, Hv, NC, C, D)
    U = buf["U"].reshape(B, Hv, NC, C, D)
    Dl = buf["Dl"].reshape(B, Hv, NC, C, D)
    pad = NC * C - T
    for hv in range(Hv):
        padf = lambda x: np.concatenate([x, np.zeros((pad,) + x.shape[1:])]) if pad else x
        qh, kh = padf(d["q"][0, :, 0].astype(np.float64)), padf(d["k"][0, :, 0].astype(np.float64))
        vh = padf(d["v"][0, :, hv].astype(np.float64))
        gl, bt = padf(d["g_log"][0, :, hv].astype(np.float64)), padf(d["beta"][0, :, hv].astype(np.float64))
        h = d["state"][0, hv].astype(np.float64).T
        for c in range(NC):
            sl = slice(c * C, (c + 1) * C)
            Gm, Tmod, Wm, Um, Pm = chunk_model.prep(kh[sl], vh[sl], qh[sl], gl[sl], bt[sl])
            msg = f"head {hv} chunk {c}"
            np.testing.assert_allclose(G[0, hv, c], Gm, rtol=1e-6, atol=1e-6, err_msg="G " + msg)
            assert nerr(Tm[0, hv, c], Tmod) < 1e-5, "T " + msg
            assert nerr(P[0, hv, c], Pm) < 1e-5, "P " + msg
            assert nerr(W[0, hv, c], Wm) < 1e-5, "W " + msg
            assert nerr(U[0, hv, c], Um) < 1e-5, "U " + msg
            assert nerr(H[0, hv, c], h) < 1e-5, "H " + msg   # saved as h = S^T ([Dk][Dv])
            Delta, _, h = chunk_model.fwd_chunk(h, qh[sl], kh[sl], Gm, Wm, Um, Pm)
            assert nerr(Dl[0, hv, c], Delta) < 1e-5, "Delta " + msg
        assert nerr(ST[0, hv].cpu().numpy(), h.T) < 1e-5


@pytest.mark.parametrize("T", [64, 100, 257])
@pytest.mark.parametrize("log_gate", [True, False])
def test_chunk_fp32_matches_oracle(dev, T, log_gate):
    d = _inputs(2, T, 2, 4, seed=T, s0_std=0.05)
    print(f"chunk fp32 T={T} log_gate={log_gate}", flush=True)
    got = _gpu(d, dev, "chunk", log_gate=log_gate)
    for b in (0, 1):
        for hk in (0, 1):
            want = _oracle_group(d, hk, 2, b, log_gate)
            for n, a, w in zip(NAMES, _slice(got, hk, 2, b), want):
                assert nerr(a, w) <= 1e-4, (b, hk, n, nerr(a, w))


@pytest.mark.parametrize("T", [64, 200])
def test_chunk_bf16_matches_oracle(dev, T):
    d = _inputs(1, T, 2, 4, seed=T + 1, s0_std=0.05)
    bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
    d = dict(d, q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), dy=bf(d["dy"]))
    got = _gpu(d, dev, "chunk", dtype=torch.bfloat16)
    for hk in (0, 1):
        want = _oracle_group(d, hk, 2)
        for n, a, w in zip(NAMES, _slice(got, hk, 2), want):
            assert nerr(a, w) <= 1e-2, (hk, n, nerr(a, w))


def test_chunk_bf16_measured_layout_against_oracle(dev):
    """B=4, Hk=16, Hv=32 (value slices of 64 in the sequential kernels), T=600 (ten chunks, the last one ragged),
    bf16 q/k/v/dO, fp32 state and gates: two key-head groups against the fp64 oracle."""
    d = _inputs(4, 600, 16, 32, seed=21, s0_std=0.02)
    bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
    d = dict(d, q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), dy=bf(d["dy"]))
    got = _gpu(d, dev, "chunk", dtype=torch.bfloat16)
    for b, hk in ((0, 0), (3, 13)):
        want = _oracle_group(d, hk, 2, b)
        errs = {n: nerr(a, w) for n, a, w in zip(NAMES, _slice(got, hk, 2, b), want)}
        print(f"bf16 B=4 T=600 b={b} hk={hk}", {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
        for n, e in errs.items():
            assert e <= 1e-2, (b, hk, n, e)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("Hk,Hv", [(3, 3), (1, 4)])
def test_chunk_value_head_groups(dev, Hk, Hv, dtype):
    """dq, dk summed over groups of one and of four value heads per key head (one backward workgroup per chunk and
    key head walks the group's value heads and keeps a running sum) against the fp64 oracle."""
    rep = Hv // Hk
    d = _inputs(2, 150, Hk, Hv, seed=40 + Hv, s0_std=0.05)
    tol = 1e-4
    if dtype == torch.bfloat16:
        bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
        d = dict(d, q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), dy=bf(d["dy"]))
        tol = 1e-2
    print(f"chunk {dtype} value-head groups Hk={Hk} Hv={Hv}", flush=True)
    got = _gpu(d, dev, "chunk", dtype=dtype)
    for b in (0, 1):
        for hk in range(Hk):
            want = _oracle_group(d, hk, rep, b)
            for n, a, w in zip(NAMES, _slice(got, hk, rep, b), want):
                assert nerr(a, w) <= tol, (b, hk, n, nerr(a, w))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_chunk_matches_recurrent_full_heads(dev, dtype):
    """B=1, T=1000, Hk=16, Hv=32: the two forms agree (recurrent form itself checked against the oracle)."""
    d = _inputs(1, 1000, 16, 32, seed=3, s0_std=0.02)
    a = _gpu(d, dev, "chunk", dtype=dtype)
    b = _gpu(d, dev, "recurrent", dtype=dtype)
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    for n, x, y in zip(NAMES, a, b):
        assert nerr(x, y) <= tol, (n, nerr(x, y))


def test_headline_config_chunk_matches_recurrent(dev):
    """The measured workload itself, B=4, T=4096, Hk=16, Hv=32, bf16 q/k/v/dO, fp32 state: every output of the
    chunked form against the recurrent form (each form checked against the fp64 oracle at smaller sizes),
    normalised error <= 1e-2."""
    d = _inputs(4, 4096, 16, 32, seed=5, s0_std=0.02)
    print("headline config B=4 T=4096 chunk vs recurrent (bf16)", flush=True)
    a = _gpu(d, dev, "chunk", dtype=torch.bfloat16)
    b = _gpu(d, dev, "recurrent", dtype=torch.bfloat16)
    errs = {n: nerr(x, y) for n, x, y in zip(NAMES, a, b)}
    print({n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= 1e-2, (n, e)


@pytest.mark.parametrize("B", [2, 4])
def test_chunk_matches_recurrent_wide_slices(dev, B):
    """B*Hv = 64 / 128 heads select value slices of 32 / 64 in the sequential kernels."""
    d = _inputs(B, 130, 16, 32, seed=B, s0_std=0.02)
    a = _gpu(d, dev, "chunk", dtype=torch.bfloat16)
    b = _gpu(d, dev, "recurrent", dtype=torch.bfloat16)
    for n, x, y in zip(NAMES, a, b):
        assert nerr(x, y) <= 1e-2, (n, nerr(x, y))
    a = _gpu(d, dev, "chunk")
    b = _gpu(d, dev, "recurrent")
    for n, x, y in zip(NAMES, a, b):
        assert nerr(x, y) <= 1e-4, (n, nerr(x, y))


def test_auto_form_selection(dev):
    import gdn_lib as L
    lib = L.load()
    assert lib.gdn_select_form(32, 128, 128, 0, L.GATE_LOG, L.FORM_AUTO, L.F32) == L.FORM_CHUNK
    assert lib.gdn_select_form(32, 128, 128, 1, L.GATE_LOG, L.FORM_AUTO, L.F32) == L.FORM_CHUNK   # masks: two chunked passes
    assert lib.gdn_select_form(32, 64, 128, 0, L.GATE_DECAY, L.FORM_AUTO, L.F32) == L.FORM_RECURRENT
    assert lib.gdn_select_form(32, 128, 128, 0, L.GATE_DECAY_VEC, L.FORM_AUTO, L.F32) == L.FORM_RECURRENT
    assert lib.gdn_select_form(32, 128, 128, 1, L.GATE_DECAY_VEC, L.FORM_CHUNK, L.F32) == L.GDN_ERR_UNSUPPORTED
