"""GPU parity of the HIP engine against the oracle (and the float64 autograd golden vectors).

Tolerances: the reference's absolute ones (tools/test_gdn_vjp.py:17-18: recurrence 1e-5, gradients 1e-4)
on its own input distributions, and a normalised error max|gpu - oracle| / max|oracle| <= 1e-4 for fp32
inputs and <= 1e-2 for bf16 inputs with fp32 state, per output tensor.
"""

import math

import numpy as np
import pytest
import torch

from golden import binfix
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

GOLD = np.load(binfix.GOLDEN / "gdn_vjp_cases.npz")
CASES = sorted({k.split("/")[0] for k in GOLD.files})
OUT_NAMES = ("y", "S_T", "dq", "dk", "dv", "dg", "dbeta", "dS0")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import gdn_lib
    gdn_lib.load()
    return torch.device("cuda:0")


def run_gpu(c, dev, chunk=64, dtype=torch.float32, impl="staged", log_gate=False):
    import gdn_vjp
    import gdn_engine
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    q, k, v = (t(c[n], dtype).requires_grad_(True) for n in ("q", "k", "v"))
    g = t(c["g"]).requires_grad_(True)
    beta = t(c["beta"]).requires_grad_(True)
    state = t(c["state"]).requires_grad_(True)
    mask = None if c.get("mask") is None else torch.tensor(np.asarray(c["mask"]), device=dev)
    if log_gate:
        y, S = gdn_engine.recurrence(q, k, v, g, beta, state, mask, chunk, log_gate=True)
    else:
        y, S = gdn_vjp.gated_delta_chunked(q, k, v, g, beta, state, mask, chunk, impl=impl)
    dy = t(c["dy"], y.dtype)
    dS = t(c["dstate"])
    grads = torch.autograd.grad([y, S], [q, k, v, g, beta, state], [dy, dS])
    torch.cuda.synchronize()
    return [x.detach().float().cpu().numpy() for x in (y, S, *grads)]


def oracle_vjp(c, chunk=64, dtype=np.float64):
    (y, S), grads = O.gated_delta_chunked_vjp(c["q"], c["k"], c["v"], c["g"], c["beta"], c["state"],
                                              c.get("mask"), c["dy"], c["dstate"], chunk=chunk, dtype=dtype)
    return [y, S, *grads]


def nerr(a, b):
    scale = float(np.abs(b).max()) if b.size else 0.0
    return float(np.abs(a - b).max()) / max(scale, 1e-30) if a.size else 0.0


def assert_close(got, want, atol_fwd=1e-5, atol_grad=1e-4, rel=1e-4, names=OUT_NAMES):
    for n, a, b in zip(names, got, want):
        assert a.shape == b.shape, (n, a.shape, b.shape)
        e = nerr(a, b)
        scale = max(1.0, float(np.abs(b).max()) if b.size else 1.0)
        atol = (atol_fwd if n in ("y", "S_T") else atol_grad) * scale
        if b.size:
            assert float(np.abs(a - b).max()) <= atol or e <= rel, f"{n}: abs {np.abs(a - b).max():.3e} rel {e:.3e}"


# ------------------------------------------------------------------------------ golden vectors

@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("chunk", [4, 64])
def test_golden_vectors(dev, name, chunk):
    c = {k.split("/")[1]: GOLD[k] for k in GOLD.files if k.startswith(name + "/")}
    print(f"case {name} chunk {chunk}", flush=True)
    got = run_gpu(c, dev, chunk)
    want = [c["exp_" + n] for n in OUT_NAMES]
    assert_close(got, want)
    assert_close(got, oracle_vjp(c, chunk, np.float32))


# ------------------------------------------------------------------------------ the reference's VJP matrix

def _ref_matrix_inputs(timesteps, masked, gate_ndim):
    """Input distributions of tools/test_gdn_vjp.py:21-55 (B=2, Hk=2, Hv=4, Dk=3, Dv=5)."""
    rng = np.random.default_rng(1000 + timesteps + 10 * gate_ndim)
    B, Hk, Hv, Dk, Dv = 2, 2, 4, 3, 5
    q = O.l2norm(rng.standard_normal((B, timesteps, Hk, Dk)), 1e-6, Dk ** -0.5)
    k = O.l2norm(rng.standard_normal((B, timesteps, Hk, Dk)), 1e-6, 1.0)
    v = rng.standard_normal((B, timesteps, Hv, Dv))
    gshape = (B, timesteps, Hv) + ((Dk,) if gate_ndim == 4 else ())
    c = dict(q=q, k=k, v=v, g=rng.uniform(0.7, 1.0, gshape), beta=rng.uniform(0.05, 0.95, (B, timesteps, Hv)),
             state=rng.standard_normal((B, Hv, Dv, Dk)), dy=rng.standard_normal((B, timesteps, Hv, Dv)),
             dstate=rng.standard_normal((B, Hv, Dv, Dk)))
    c = {n: x.astype(np.float32) for n, x in c.items()}
    c["mask"] = (np.random.default_rng(timesteps + gate_ndim).random((B, timesteps)) > 0.2) if masked else None
    return c


@pytest.mark.parametrize("timesteps", [1, 63, 64, 65, 200])
@pytest.mark.parametrize("chunk", [16, 64])
@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("gate_ndim", [3, 4])
def test_forward_and_six_cotangents_match_oracle(dev, timesteps, chunk, masked, gate_ndim):
    c = _ref_matrix_inputs(timesteps, masked, gate_ndim)
    got = run_gpu(c, dev, chunk)
    assert_close(got, oracle_vjp(c, chunk))


@pytest.mark.parametrize("gate_ndim", [3, 4])
def test_kernel_impl_parity_case(dev, gate_ndim):
    """Counterpart of tools/test_gdn_vjp.py:79-107: Dk=32, Dv=3, T=2, chunk=T, mask [[True, False]],
    impl="kernel", against the float64 oracle at the reference's gradient atol 1e-4."""
    rng = np.random.default_rng(777 + gate_ndim)
    B, T, Hk, Hv, Dk, Dv = 1, 2, 1, 2, 32, 3
    q = O.l2norm(rng.standard_normal((B, T, Hk, Dk)), 1e-6, Dk ** -0.5)
    k = O.l2norm(rng.standard_normal((B, T, Hk, Dk)), 1e-6, 1.0)
    gshape = (B, T, Hv) + ((Dk,) if gate_ndim == 4 else ())
    c = dict(q=q, k=k, v=rng.standard_normal((B, T, Hv, Dv)), g=rng.uniform(0.7, 1.0, gshape),
             beta=rng.uniform(0.05, 0.95, (B, T, Hv)), state=rng.standard_normal((B, Hv, Dv, Dk)),
             dy=rng.standard_normal((B, T, Hv, Dv)), dstate=rng.standard_normal((B, Hv, Dv, Dk)))
    c = {n: x.astype(np.float32) for n, x in c.items()}
    c["mask"] = np.array([[True, False]])
    got = run_gpu(c, dev, T, impl="kernel")
    want = oracle_vjp(c, T)
    for n, a, b in zip(OUT_NAMES, got, want):
        assert a.shape == b.shape, n
        assert float(np.abs(a - b).max()) <= 1e-4, (n, float(np.abs(a - b).max()))


# ------------------------------------------------------------------------------ checkpoint matrix, real heads

@pytest.mark.parametrize("timesteps", [1, 63, 64, 65, 200])
@pytest.mark.parametrize("chunk", [16, 64])
@pytest.mark.parametrize("masked", [False, True])
def test_checkpointed_real_head_sizes(dev, timesteps, chunk, masked):
    """tools/test_gdn_checkpoint.py:27-58 inputs (Hk=16, Hv=32, D=128, g ~ U(0.9,1)); loss = sum(y)+sum(S_T)
    as :_scalar_recurrence; compared on one key-head group against the oracle, all heads vs each other."""
    import gdn_checkpoint
    rng = np.random.default_rng(1000 + timesteps)
    B, Hk, Hv, D = 1, 16, 32, 128
    q = O.l2norm(rng.standard_normal((B, timesteps, Hk, D)), 1e-6, D ** -0.5).astype(np.float32)
    k = O.l2norm(rng.standard_normal((B, timesteps, Hk, D)), 1e-6, 1.0).astype(np.float32)
    v = rng.standard_normal((B, timesteps, Hv, D)).astype(np.float32)
    g = rng.uniform(0.9, 1.0, (B, timesteps, Hv)).astype(np.float32)
    beta = rng.uniform(0.05, 0.95, (B, timesteps, Hv)).astype(np.float32)
    state = rng.standard_normal((B, Hv, D, D)).astype(np.float32)
    mask = (np.random.default_rng(1000 + timesteps).random((B, timesteps)) > 0.15) if masked else None
    t = lambda x: torch.tensor(x, device=dev).requires_grad_(True)
    xs = [t(x) for x in (q, k, v, g, beta, state)]
    m = None if mask is None else torch.tensor(mask, device=dev)
    y, S = gdn_checkpoint.gated_delta_ops_checkpointed(*xs, m, chunk)
    (y.sum() + S.sum()).backward()
    got = [x.detach().cpu().numpy() for x in (y, S)] + [x.grad.cpu().numpy() for x in xs]
    # oracle on key head 3 (value heads 6, 7)
    sl = slice(6, 8)
    c = dict(q=q[:, :, 3:4], k=k[:, :, 3:4], v=v[:, :, sl], g=g[:, :, sl], beta=beta[:, :, sl],
             state=state[:, sl], mask=mask, dy=np.ones_like(v[:, :, sl]), dstate=np.ones_like(state[:, sl]))
    want = oracle_vjp(c, chunk)
    got_slice = [got[0][:, :, sl], got[1][:, sl], got[2][:, :, 3:4], got[3][:, :, 3:4], got[4][:, :, sl],
                 got[5][:, :, sl], got[6][:, :, sl], got[7][:, sl]]
    assert_close(got_slice, want)


# ------------------------------------------------------------------------------ measured workloads

def _workload(T, B=1, s0_std=0.0, seed=0, heads=(16, 32), D=128):
    d = O.make_inputs(B, T, heads[0], heads[1], D, seed=seed, s0_std=s0_std)
    return dict(q=d["q"], k=d["k"], v=d["v"], g=d["decay"], g_log=d["g_log"], beta=d["beta"],
                state=d["state"], dy=d["dy"], dstate=np.zeros_like(d["state"]), mask=None)


def _slice_group(c, hk, rep=2):
    sl = slice(hk * rep, hk * rep + rep)
    return dict(q=c["q"][:, :, hk:hk + 1], k=c["k"][:, :, hk:hk + 1], v=c["v"][:, :, sl], g=c["g"][:, :, sl],
                beta=c["beta"][:, :, sl], state=c["state"][:, sl], dy=c["dy"][:, :, sl],
                dstate=c["dstate"][:, sl], mask=None)


def _slice_out(got, hk, rep=2):
    sl = slice(hk * rep, hk * rep + rep)
    return [got[0][:, :, sl], got[1][:, sl], got[2][:, :, hk:hk + 1], got[3][:, :, hk:hk + 1],
            got[4][:, :, sl], got[5][:, :, sl], got[6][:, :, sl], got[7][:, sl]]


def test_config0_full_against_oracle(dev):
    """B=1, T=64, Hk=16, Hv=32, D=128, fp32, S0=0: every head against the fp64 oracle."""
    c = _workload(64)
    got = run_gpu(c, dev, 64)
    want = oracle_vjp(c, 64)
    for n, a, b in zip(OUT_NAMES, got, want):
        assert nerr(a, b) <= 1e-4, (n, nerr(a, b))


def test_config0_log_gate_matches_decay_gate(dev):
    """Log-space gates give dg w.r.t. log decay = dg_decay * decay."""
    c = _workload(64, seed=3)
    got = run_gpu(c, dev, 64)
    c_log = dict(c, g=c["g_log"])
    got_log = run_gpu(c_log, dev, 64, log_gate=True)
    for n, a, b in zip(OUT_NAMES, got_log, got):
        if n == "dg":
            b = b * c["g"]
        assert nerr(a, b) <= 1e-5, (n, nerr(a, b))


def test_config1_T2048_group_slices(dev):
    """B=1, T=2048, S0 ~ N(0, 0.02), full dS0: two key-head groups against the fp64 oracle."""
    c = _workload(2048, s0_std=0.02, seed=1)
    got = run_gpu(c, dev, 64)
    for hk in (0, 11):
        want = oracle_vjp(_slice_group(c, hk), 64)
        for n, a, b in zip(OUT_NAMES, _slice_out(got, hk), want):
            assert nerr(a, b) <= 1e-4, (hk, n, nerr(a, b))


def test_bf16_inputs_fp32_state(dev):
    """bf16 q/k/v/dO with fp32 state and gates: against the oracle fed the same bf16-rounded inputs."""
    c = _workload(256, B=2, seed=2)
    bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
    c = dict(c, q=bf(c["q"]), k=bf(c["k"]), v=bf(c["v"]), dy=bf(c["dy"]))
    got = run_gpu(c, dev, 64, dtype=torch.bfloat16)
    for hk in (0, 15):
        cb = {n: (x[1:2] if isinstance(x, np.ndarray) else x) for n, x in c.items()}
        want = oracle_vjp(_slice_group(cb, hk), 64)
        gs = [x[1:2] for x in _slice_out(got, hk)]
        for n, a, b in zip(OUT_NAMES, gs, want):
            assert nerr(a, b) <= 1e-2, (hk, n, nerr(a, b))


@pytest.mark.parametrize("gate_ndim", [3, 4])
def test_recurrent_wide_grid_against_oracle(dev, monkeypatch, gate_ndim):
    """The recurrent form at B=4, Hk=16, Hv=32, D=128, T=80 (a partial second chunk and partial sub-chunks), a mask,
    random dS_T, scalar or per-channel decay gates: with per-channel gates this grid takes the backward's 8-wave,
    32-row workgroups (per-channel gates and B * Hv * Dv / 32 >= 512), with scalar gates the 16-row ones.  Two
    key-head groups in two sequences against the fp64 oracle."""
    monkeypatch.setenv("GDN_FORM", "recurrent")
    rng = np.random.default_rng(77 + gate_ndim)
    B, T, Hk, Hv, D = 4, 80, 16, 32, 128
    q = O.l2norm(rng.standard_normal((B, T, Hk, D)), 1e-6, D ** -0.5).astype(np.float32)
    k = O.l2norm(rng.standard_normal((B, T, Hk, D)), 1e-6, 1.0).astype(np.float32)
    gshape = (B, T, Hv) + ((D,) if gate_ndim == 4 else ())
    c = dict(q=q, k=k, v=rng.standard_normal((B, T, Hv, D)).astype(np.float32),
             g=rng.uniform(0.9, 1.0, gshape).astype(np.float32),
             beta=rng.uniform(0.05, 0.95, (B, T, Hv)).astype(np.float32),
             state=(0.1 * rng.standard_normal((B, Hv, D, D))).astype(np.float32),
             dy=rng.standard_normal((B, T, Hv, D)).astype(np.float32),
             dstate=(0.1 * rng.standard_normal((B, Hv, D, D))).astype(np.float32),
             mask=rng.random((B, T)) > 0.2)
    got = run_gpu(c, dev, 64)
    for bi, hk in ((0, 0), (3, 13)):
        cb = {n: (x[bi:bi + 1] if isinstance(x, np.ndarray) else x) for n, x in c.items()}
        want = oracle_vjp(dict(_slice_group(cb, hk), mask=cb["mask"]), 64)
        gs = [x[bi:bi + 1] for x in _slice_out(got, hk)]
        for n, a, b in zip(OUT_NAMES, gs, want):
            assert nerr(a, b) <= 1e-4, (bi, hk, n, nerr(a, b))


@pytest.mark.parametrize("form", ["recurrent", "chunk"])
def test_fp16_inputs_fp32_state(dev, monkeypatch, form):
    """fp16 q/k/v with fp32 state, gates and cotangent: the kernels that read the input dtype from their arguments
    (the recurrent form's and the fp32 chunked set's run-time dtype variants), against the oracle fed the same
    fp16-rounded inputs.  The arithmetic is fp32, so y, S_T, dg, dbeta and dS0 (fp32) meet the fp32 bar; dq, dk and
    dv come out in the input dtype, within fp16's rounding (2^-11 of the largest value) of the oracle."""
    monkeypatch.setenv("GDN_FORM", form)
    c = _workload(200, B=1, seed=6, heads=(2, 4))
    hf = lambda x: torch.tensor(x).half().float().numpy()
    c = dict(c, q=hf(c["q"]), k=hf(c["k"]), v=hf(c["v"]), dstate=np.full_like(c["state"], 0.01))
    got = run_gpu(c, dev, 64, dtype=torch.float16)
    want = oracle_vjp(c, 64)
    for n, a, b in zip(OUT_NAMES, got, want):
        bar = 1e-3 if n in ("dq", "dk", "dv") else 1e-4
        assert nerr(a, b) <= bar, (form, n, nerr(a, b))


def test_chunk_invariance_long(dev, monkeypatch):
    """The recurrent form's snapshot interval is an implementation detail: chunk 64 vs 256 vs 1000 agree."""
    monkeypatch.setenv("GDN_FORM", "recurrent")
    c = _workload(1500, s0_std=0.02, seed=4)
    base = run_gpu(c, dev, 64)
    for chunk in (256, 1000):
        other = run_gpu(c, dev, chunk)
        for n, a, b in zip(OUT_NAMES, other, base):
            assert nerr(a, b) <= 1e-5, (chunk, n, nerr(a, b))


def test_forward_only_path_matches(dev):
    import gated_delta
    c = _workload(300, seed=5)
    t = lambda x: torch.tensor(x, device=dev)
    y0, S0 = gated_delta.gated_delta_kernel(t(c["q"]), t(c["k"]), t(c["v"]), t(c["g"]), t(c["beta"]),
                                            t(c["state"]))
    got = run_gpu(c, dev, 64)
    assert np.array_equal(y0.cpu().numpy(), got[0]) and np.array_equal(S0.cpu().numpy(), got[1])


def test_empty_and_edge_inputs(dev):
    import gdn_vjp
    # T = 0: y empty, S_T = S0, dS0 = dS_T
    S0 = torch.randn(1, 2, 4, 3, device=dev, requires_grad=True)
    q = torch.zeros(1, 0, 1, 3, device=dev, requires_grad=True)
    v = torch.zeros(1, 0, 2, 4, device=dev)
    y, S = gdn_vjp.gated_delta_chunked(q, q, v, torch.zeros(1, 0, 2, device=dev),
                                       torch.zeros(1, 0, 2, device=dev), S0)
    assert y.shape == (1, 0, 2, 4) and torch.equal(S, S0)
    dS = torch.randn_like(S)
    (gS0,) = torch.autograd.grad(S, [S0], dS)
    assert torch.equal(gS0, dS)
    # Dk = 256 (largest supported) and Dv not a multiple of 16
    c = _ref_matrix_inputs(20, True, 3)
    rng = np.random.default_rng(0)
    c["q"] = O.l2norm(rng.standard_normal((2, 20, 2, 256)), 1e-6, 1 / 16).astype(np.float32)
    c["k"] = O.l2norm(rng.standard_normal((2, 20, 2, 256)), 1e-6, 1.0).astype(np.float32)
    c["v"] = rng.standard_normal((2, 20, 4, 21)).astype(np.float32)
    c["state"] = rng.standard_normal((2, 4, 21, 256)).astype(np.float32)
    c["dstate"] = rng.standard_normal((2, 4, 21, 256)).astype(np.float32)
    c["dy"] = rng.standard_normal((2, 20, 4, 21)).astype(np.float32)
    assert_close(run_gpu(c, dev, 8), oracle_vjp(c, 8))


def test_errors_match_reference(dev):
    import gdn_vjp
    q = torch.zeros(1, 4, 2, 8, device=dev)
    v = torch.zeros(1, 4, 3, 8, device=dev)
    g = torch.ones(1, 4, 3, device=dev)
    with pytest.raises(ValueError, match="chunk must be a positive integer"):
        gdn_vjp.gated_delta_chunked(q, q, v, g, g, chunk=0)
    with pytest.raises(ValueError, match="impl must be"):
        gdn_vjp.gated_delta_chunked(q, q, v, g, g, impl="fast")
    with pytest.raises(ValueError, match="head count must divide"):
        gdn_vjp.gated_delta_chunked(q, q, v, g, g)
    # impl="kernel" checks key_dim and the shared dtype when the backward runs (tools/gdn_vjp.py:391-394):
    # the forward succeeds, with and without a graph, and the backward raises
    v2, g2 = torch.zeros(1, 4, 2, 8, device=dev), g[:, :, :2]
    with torch.no_grad():
        y, S = gdn_vjp.gated_delta_chunked(q, q, v2, g2, g2, impl="kernel")
    assert y.shape == (1, 4, 2, 8) and S.shape == (1, 2, 8, 8)
    qg = q.clone().requires_grad_(True)
    y, S = gdn_vjp.gated_delta_chunked(qg, q, v2, g2, g2, impl="kernel")
    with pytest.raises(ValueError, match="key_dim divisible by 32"):
        y.sum().backward()
    q32 = torch.randn(1, 4, 2, 32, device=dev)
    k32 = q32.to(torch.bfloat16)
    v32 = torch.zeros(1, 4, 2, 32, device=dev)
    with torch.no_grad():
        gdn_vjp.gated_delta_chunked(q32, k32, v32, g2, g2, impl="kernel")
    qg = q32.clone().requires_grad_(True)
    y, S = gdn_vjp.gated_delta_chunked(qg, k32, v32, g2, g2, impl="kernel")
    with pytest.raises(ValueError, match="share a dtype"):
        y.sum().backward()
    # the other impls take the same inputs through the backward
    qg = q32.clone().requires_grad_(True)
    y, S = gdn_vjp.gated_delta_chunked(qg, k32, v32, g2, g2, impl="staged")
    y.sum().backward()
    assert qg.grad is not None and bool(torch.isfinite(qg.grad).all())
    with pytest.raises(ValueError, match="Unsupported gating shape"):
        gdn_vjp.gated_delta_chunked(q, q, torch.zeros(1, 4, 2, 8, device=dev), g[:, :, 0], g[:, :, :2])
