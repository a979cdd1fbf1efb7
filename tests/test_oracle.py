"""Pins the CPU oracle (oracle/gdn_oracle.py) against the reference's golden vectors, the reference's own C
compiled from source, torch autograd of an independent naive recurrence, finite differences and closed
forms.  CPU only."""

import math

import numpy as np
import pytest
import torch

from golden import binfix
from oracle import gdn_oracle as O
from oracle import ref_c
import naive_torch

GOLD = np.load(binfix.GOLDEN / "gdn_vjp_cases.npz")
CASE_NAMES = sorted({k.split("/")[0] for k in GOLD.files})
NAMES = ("y", "S_T", "dq", "dk", "dv", "dg", "dbeta", "dS0")


def _case(name):
    d = {k.split("/")[1]: GOLD[k] for k in GOLD.files if k.startswith(name + "/")}
    return d


def _oracle_vjp(c, dtype, chunk=64, oracle=O):
    (y, S), grads = oracle.gated_delta_chunked_vjp(
        c["q"], c["k"], c["v"], c["g"], c["beta"], c["state"], c.get("mask"), c["dy"], c["dstate"],
        chunk=chunk, dtype=dtype)
    return (y, S, *grads)


# ---------------------------------------------------------------- forward vs reference golden vectors / C

def test_forward_matches_reference_mlx_fixture():
    """gdn_recurrence.bin: MLX ground truth (tools/gen_gdn_fixture.py:59-77), tol of engine/tests/test_gdn.c."""
    a = binfix.load("gdn_recurrence.bin")
    Hk, Hv, Dk, Dv, T = (int(x) for x in a[0])
    steps = [a[1 + 6 * t: 7 + 6 * t] for t in range(T)]
    q = np.stack([s[0].reshape(Hk, Dk) for s in steps])[None]
    k = np.stack([s[1].reshape(Hk, Dk) for s in steps])[None]
    v = np.stack([s[2].reshape(Hv, Dv) for s in steps])[None]
    g = np.stack([s[3] for s in steps])[None]
    beta = np.stack([s[4] for s in steps])[None]
    want_y = np.stack([s[5].reshape(Hv, Dv) for s in steps])[None]
    want_S = a[1 + 6 * T].reshape(1, Hv, Dv, Dk)
    for chunk in (1, 2, 64):
        y, S = O.gated_delta_chunked(q, k, v, g, beta, chunk=chunk)
        np.testing.assert_allclose(y, want_y, atol=2e-5, rtol=2e-5)
        np.testing.assert_allclose(S, want_S, atol=2e-5, rtol=2e-5)


@pytest.mark.skipif(not ref_c.available(), reason="oracle/_ref not built (make -C oracle)")
@pytest.mark.parametrize("Hk,Hv,Dk,Dv,T", [(2, 4, 32, 16, 50), (1, 2, 128, 128, 6), (16, 32, 8, 8, 9)])
def test_forward_matches_reference_c(Hk, Hv, Dk, Dv, T):
    rng = np.random.default_rng(Hk * 100 + T)
    q = (rng.standard_normal((T, Hk, Dk)) * 0.3).astype(np.float32)
    k = (rng.standard_normal((T, Hk, Dk)) * 0.3).astype(np.float32)
    v = rng.standard_normal((T, Hv, Dv)).astype(np.float32)
    g = rng.uniform(0.5, 1.0, (T, Hv)).astype(np.float32)
    beta = rng.uniform(0, 1, (T, Hv)).astype(np.float32)
    S0 = rng.standard_normal((Hv, Dv, Dk)).astype(np.float32)
    y_c, S_c = ref_c.recurrence(q, k, v, g, beta, S0)
    y, S = O.gated_delta_chunked(q[None], k[None], v[None], g[None], beta[None], S0[None], chunk=16)
    np.testing.assert_allclose(y[0], y_c, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(S[0], S_c, atol=2e-5, rtol=2e-5)


# ---------------------------------------------------------------- backward vs torch autograd golden vectors

@pytest.mark.parametrize("name", CASE_NAMES)
def test_oracle_fp64_matches_autograd_golden(name):
    c = _case(name)
    got = _oracle_vjp(c, np.float64, chunk=16)
    for n, x in zip(NAMES, got):
        np.testing.assert_allclose(x, c["exp_" + n], atol=1e-10, rtol=1e-9, err_msg=n)


@pytest.mark.parametrize("name", CASE_NAMES)
def test_oracle_fp32_within_reference_tolerance(name):
    """fp32 oracle vs float64 truth at the reference tolerances (tools/test_gdn_vjp.py:17-18)."""
    c = _case(name)
    got = _oracle_vjp(c, np.float32, chunk=64)
    for n, x in zip(NAMES, got):
        atol = 1e-5 if n in ("y", "S_T") else 1e-4
        scale = max(1.0, float(np.abs(c["exp_" + n]).max()))
        np.testing.assert_allclose(x, c["exp_" + n], atol=atol * scale, rtol=0, err_msg=n)


def test_golden_has_teeth_against_planted_mistakes(monkeypatch):
    """A dropped (1-m)*dS term or a transposed gate reduction in the oracle must fail the golden check."""
    c = _case("tiny_masked")
    good = _oracle_vjp(c, np.float64, chunk=4)
    np.testing.assert_allclose(good[-1], c["exp_dS0"], atol=1e-10)
    real = O.chunk_vjp

    def dropped_keep_term(q, k, v, g, beta, s0, mask, dy, dstate):
        return real(q, k, v, g, beta, s0, None if mask is None else np.ones_like(mask), dy, dstate)

    monkeypatch.setattr(O, "chunk_vjp", dropped_keep_term)
    bad = _oracle_vjp(c, np.float64, chunk=4)
    assert not np.allclose(bad[-1], c["exp_dS0"], atol=1e-4)
    monkeypatch.setattr(O, "chunk_vjp", real)
    real_decay = O.decay_view
    monkeypatch.setattr(O, "decay_view", lambda g: real_decay(g) ** 1.01)
    bad = _oracle_vjp(c, np.float64, chunk=4)
    assert not np.allclose(bad[5], c["exp_dg"], atol=1e-4)


def test_oracle_backward_matches_finite_differences():
    rng = np.random.default_rng(5)
    B, T, Hk, Hv, Dk, Dv = 1, 5, 1, 2, 3, 2
    x = dict(q=rng.standard_normal((B, T, Hk, Dk)) * 0.5, k=rng.standard_normal((B, T, Hk, Dk)) * 0.5,
             v=rng.standard_normal((B, T, Hv, Dv)), g=rng.uniform(0.6, 1.0, (B, T, Hv)),
             beta=rng.uniform(0.1, 0.9, (B, T, Hv)), state=rng.standard_normal((B, Hv, Dv, Dk)))
    mask = np.array([[True, False, True, True, False]])
    dy = rng.standard_normal((B, T, Hv, Dv))
    dS = rng.standard_normal((B, Hv, Dv, Dk))

    def loss(d):
        y, S = O.gated_delta_chunked(d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"], mask,
                                     chunk=2, dtype=np.float64)
        return float((y * dy).sum() + (S * dS).sum())

    _, grads = O.gated_delta_chunked_vjp(x["q"], x["k"], x["v"], x["g"], x["beta"], x["state"], mask,
                                         dy, dS, chunk=2, dtype=np.float64)
    eps = 1e-6
    for name, grad in zip(("q", "k", "v", "g", "beta", "state"), grads):
        fd = np.zeros_like(x[name])
        for idx in np.ndindex(x[name].shape):
            d_plus = {n: a.copy() for n, a in x.items()}
            d_minus = {n: a.copy() for n, a in x.items()}
            d_plus[name][idx] += eps
            d_minus[name][idx] -= eps
            fd[idx] = (loss(d_plus) - loss(d_minus)) / (2 * eps)
        np.testing.assert_allclose(grad, fd, atol=1e-6, rtol=1e-5, err_msg=name)


# ---------------------------------------------------------------- closed forms and invariants

def _rand(seed, B=1, T=6, Hk=1, Hv=2, Dk=4, Dv=3):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((B, T, Hk, Dk)), rng.standard_normal((B, T, Hk, Dk)),
            rng.standard_normal((B, T, Hv, Dv)), rng.uniform(0.5, 1, (B, T, Hv)),
            rng.uniform(0.1, 0.9, (B, T, Hv)), rng.standard_normal((B, Hv, Dv, Dk)))


def test_single_step_closed_form():
    q, k, v, g, beta, S0 = _rand(1, T=1)
    y, S = O.gated_delta_chunked(q, k, v, g, beta, S0, dtype=np.float64)
    for h in range(2):
        A = g[0, 0, h] * S0[0, h]
        d = beta[0, 0, h] * (v[0, 0, h] - A @ k[0, 0, 0])
        S1 = A + np.outer(d, k[0, 0, 0])
        np.testing.assert_allclose(S[0, h], S1, atol=1e-12)
        np.testing.assert_allclose(y[0, 0, h], S1 @ q[0, 0, 0], atol=1e-12)


def test_beta_zero_is_pure_decay_and_decay_zero_kills_ds0():
    q, k, v, g, beta, S0 = _rand(2)
    y, S = O.gated_delta_chunked(q, k, v, g, np.zeros_like(beta), S0, dtype=np.float64)
    np.testing.assert_allclose(S[0], S0[0] * np.prod(g[0], axis=0)[:, None, None], atol=1e-12)
    g0 = g.copy()
    g0[:, 0] = 0.0   # the first step discards S0 entirely
    dy = np.ones_like(v)
    _, grads = O.gated_delta_chunked_vjp(q, k, v, g0, beta, S0, None, dy, np.ones_like(S0),
                                         chunk=4, dtype=np.float64)
    assert np.abs(grads[-1]).max() == 0.0


def test_decay_one_beta_zero_reads_initial_state():
    q, k, v, g, beta, S0 = _rand(3)
    y, _ = O.gated_delta_chunked(q, k, v, np.ones_like(g), np.zeros_like(beta), S0, dtype=np.float64)
    want = np.einsum("bhij,btj->bthi", S0, q[:, :, 0])
    np.testing.assert_allclose(y, want, atol=1e-12)


@pytest.mark.parametrize("T", [1, 63, 64, 65, 200])
def test_chunk_invariance(T):
    q, k, v, g, beta, S0 = _rand(T, T=T, Dk=5, Dv=3)
    rng = np.random.default_rng(T)
    mask = rng.random((1, T)) > 0.2
    dy = rng.standard_normal(v.shape)
    dS = rng.standard_normal(S0.shape)
    outs = [_oracle_vjp(dict(q=q, k=k, v=v, g=g, beta=beta, state=S0, mask=mask, dy=dy, dstate=dS),
                        np.float64, chunk=c) for c in (16, 64)]
    for a, b in zip(*outs):
        np.testing.assert_allclose(a, b, atol=1e-10)


# ---------------------------------------------------------------- gates, l2norm, conv, rmsnorm

def test_gates_match_reference_fixture_and_c():
    a, b, A_log, dt, want_g, want_b = binfix.load("gdn_gates.bin")[1:]
    g, beta = O.gates(a.astype(np.float64), b.astype(np.float64), A_log.astype(np.float64),
                      dt.astype(np.float64))
    np.testing.assert_allclose(g, want_g, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(beta, want_b, atol=2e-5, rtol=2e-5)
    if ref_c.available():
        gc, bc = ref_c.gates(a, b, A_log, dt)
        np.testing.assert_allclose(g, gc, atol=2e-6, rtol=2e-6)


def test_l2norm_matches_reference_fixture():
    hdr, q, qn, k, kn = binfix.load("gdn_l2norm.bin")
    H, Dk = int(hdr[0]), int(hdr[1])
    np.testing.assert_allclose(O.l2norm(q.reshape(H, Dk), 1e-6, Dk ** -0.5), qn.reshape(H, Dk),
                               atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(O.l2norm(k.reshape(H, Dk), 1e-6, 1.0), kn.reshape(H, Dk),
                               atol=2e-5, rtol=2e-5)


def test_conv_matches_reference_fixture_and_c():
    hdr, w, xs, want = binfix.load("gdn_conv.bin")
    C, K, T = (int(x) for x in hdr)
    w = w.reshape(C, K)
    xs = xs.reshape(T, C)
    out, _ = O.conv_silu(xs[None].astype(np.float64), w.astype(np.float64))
    np.testing.assert_allclose(out[0], want.reshape(T, C), atol=2e-5, rtol=2e-5)
    if ref_c.available():
        np.testing.assert_allclose(out[0], ref_c.conv_silu(xs, w), atol=2e-5, rtol=2e-5)


def test_rmsnorm_and_silu_mul_match_reference_fixtures():
    x, w, want = binfix.load("ops_rmsnorm.bin")
    np.testing.assert_allclose(O.rmsnorm(x, w, 1e-6), want, atol=2e-5, rtol=2e-5)
    g, u, want = binfix.load("ops_silu_mul.bin")
    np.testing.assert_allclose(O.silu_mul(g.astype(np.float64), u), want, atol=2e-5, rtol=2e-5)


def _autograd(fn, *xs):
    ts = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in xs]
    out = fn(*ts)
    return out, ts


def test_elementwise_backwards_match_autograd():
    rng = np.random.default_rng(9)
    # gates (a in both softplus branches)
    a = rng.standard_normal((3, 5, 4)) * 3
    a[0, 0, 0] = 25.0
    b = rng.standard_normal((3, 5, 4))
    A_log = rng.uniform(0, 2.7, 4)
    dt = rng.standard_normal(4) * 0.1
    dd, db_ = rng.standard_normal((2, 3, 5, 4))
    ta, tb, tA, tdt = [torch.tensor(x, requires_grad=True) for x in (a, b, A_log, dt)]
    x = ta + tdt
    sp = torch.where(x > 20, x, torch.log1p(torch.exp(torch.clamp(x, max=20))))
    dec = torch.exp(-torch.exp(tA) * sp)
    bet = 2 * torch.sigmoid(tb)
    ((dec * torch.tensor(dd)).sum() + (bet * torch.tensor(db_)).sum()).backward()
    got = O.gates_bwd(a, b, A_log, dt, dd, db_, allow_neg_eigval=True)
    for g_, t in zip(got, (ta, tb, tA, tdt)):
        np.testing.assert_allclose(g_, t.grad.numpy(), atol=1e-10, rtol=1e-9)
    # l2norm
    xq = rng.standard_normal((4, 16))
    dy = rng.standard_normal((4, 16))
    t = torch.tensor(xq, requires_grad=True)
    (0.25 * t / torch.sqrt((t * t).sum(-1, keepdim=True) + 1e-6) * torch.tensor(dy)).sum().backward()
    np.testing.assert_allclose(O.l2norm_bwd(xq, dy, 1e-6, 0.25), t.grad.numpy(), atol=1e-10)
    # conv + silu
    xc = rng.standard_normal((2, 7, 5))
    wc = rng.standard_normal((5, 4))
    dout = rng.standard_normal((2, 7, 5))
    tx, tw = [torch.tensor(z, requires_grad=True) for z in (xc, wc)]
    pre = torch.nn.functional.conv1d(tx.transpose(1, 2), tw[:, None, :], padding=3, groups=5)[..., :7]
    (torch.nn.functional.silu(pre).transpose(1, 2) * torch.tensor(dout)).sum().backward()
    dx, dw = O.conv_silu_bwd(xc, wc, dout)
    np.testing.assert_allclose(dx, tx.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(dw, tw.grad.numpy(), atol=1e-10)
    # gated rmsnorm
    y = rng.standard_normal((3, 8))
    z = rng.standard_normal((3, 8))
    w = rng.standard_normal(8)
    do = rng.standard_normal((3, 8))
    ty, tz, tw = [torch.tensor(u, requires_grad=True) for u in (y, z, w)]
    n = ty * torch.rsqrt((ty * ty).mean(-1, keepdim=True) + 1e-6) * tw
    (n * torch.nn.functional.silu(tz) * torch.tensor(do)).sum().backward()
    got = O.gated_rmsnorm_bwd(y, z, w, do)
    for g_, t in zip(got, (ty, tz, tw)):
        np.testing.assert_allclose(g_, t.grad.numpy(), atol=1e-10)


def test_make_inputs_distributions():
    d = O.make_inputs(1, 64, 16, 32, 128, seed=0, s0_std=0.02)
    assert d["q"].shape == (1, 64, 16, 128) and d["state"].shape == (1, 32, 128, 128)
    np.testing.assert_allclose(np.linalg.norm(d["k"], axis=-1), 1.0, atol=1e-5)
    np.testing.assert_allclose(np.linalg.norm(d["q"], axis=-1), 128 ** -0.5, atol=1e-5)
    assert (d["g_log"] < 0).all() and (d["g_log"] > -16 * 25).all()
    assert abs(float(d["state"].std()) - 0.02) < 1e-3


# ---------------------------------------------------------------- whole block (forward + VJP with LoRA)

def test_block_vjp_matches_torch_autograd():
    """The composed block VJP against torch float64 autograd of tests/naive_torch.py::gdn_block, with LoRA
    adapters on all five projections (B random so that every adapter gradient is non-zero)."""
    from oracle import gdn_block_oracle as BO
    Bsz, T, h, Hk, Hv, Dk, Dv = 2, 37, 12, 2, 4, 8, 6
    P = BO.make_block_params(h, Hk, Hv, Dk, Dv, K=4, rank=3, b_std=0.05, seed=1, w_std=0.3)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((Bsz, T, h))
    dout = rng.standard_normal((Bsz, T, h))
    out, g = BO.block_vjp(x, P, dout, Hk, Hv, Dk, Dv, chunk=16)
    tP = {k: (torch.tensor(np.asarray(v, np.float64), requires_grad=True) if isinstance(v, np.ndarray) else v)
          for k, v in P.items()}
    tx = torch.tensor(x, requires_grad=True)
    tout = naive_torch.gdn_block(tx, tP, Hk, Hv, Dk, Dv)
    np.testing.assert_allclose(out, tout.detach().numpy(), rtol=1e-9, atol=1e-12)
    names = ["x", "conv_w", "A_log", "dt_bias", "norm_w"] + [f"{p}_{n}" for n in BO.PROJ for p in ("A", "B")]
    leaves = [tx] + [tP[n] for n in names[1:]]
    tg = torch.autograd.grad(tout, leaves, torch.tensor(dout))
    for n, want in zip(names, tg):
        np.testing.assert_allclose(g[n], want.numpy(), rtol=1e-8, atol=1e-10, err_msg=n)


def test_block_lora_b_zero_gives_zero_a_gradient():
    """With B = 0 (the LoRA initialisation) grad(A) = s B^T dW is exactly zero and grad(B) is not."""
    from oracle import gdn_block_oracle as BO
    P = BO.make_block_params(12, 2, 4, 8, 6, rank=3, b_std=0.0, seed=3, w_std=0.3)
    rng = np.random.default_rng(4)
    x, dout = rng.standard_normal((1, 20, 12)), rng.standard_normal((1, 20, 12))
    _, g = BO.block_vjp(x, P, dout, 2, 4, 8, 6, chunk=8)
    for n in BO.PROJ:
        assert not np.any(g["A_" + n])
        assert np.abs(g["B_" + n]).max() > 0
