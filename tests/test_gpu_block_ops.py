"""GPU parity of the block ops around the recurrence (gates, q/k L2 norm, causal conv1d + SiLU, gated RMSNorm),
forward and backward, through the C ABI via the torch wrappers in gdn_block.

Forwards are checked against the reference's own fixtures (gdn_gates.bin, gdn_l2norm.bin, gdn_conv.bin,
ops_rmsnorm.bin + ops_silu_mul.bin) and against the float64 oracle; backwards against the oracle, whose
backward functions are themselves checked against torch float64 autograd on the CPU.  Tolerances: normalised
max error <= 1e-5 for fp32 forwards, <= 1e-4 for fp32 backwards (parameter gradients sum over all tokens),
<= 1e-2 for bf16 activations.
"""

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O
from golden import binfix

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


def T_(x, dev, dtype=torch.float32, grad=False):
    t = torch.tensor(np.asarray(x), device=dev, dtype=dtype)
    return t.requires_grad_(True) if grad else t


def np_(t):
    return t.detach().float().cpu().numpy()


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------------------------------------ gates


def test_gates_fixture(dev):
    import gdn_block
    a, b, A_log, dt, want_g, want_b = binfix.load("gdn_gates.bin")[1:]
    print("gates fixture", a.shape, flush=True)
    g, beta = gdn_block.gates(T_(a[None], dev), T_(b[None], dev), T_(A_log, dev), T_(dt, dev))
    torch.cuda.synchronize()
    assert nerr(np_(g)[0], want_g) <= 1e-5
    assert nerr(np_(beta)[0], want_b) <= 1e-5


@pytest.mark.parametrize("log_space", [False, True])
@pytest.mark.parametrize("neg", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gates_fwd_bwd(dev, log_space, neg, dtype):
    import gdn_block
    B, T, Hv = 2, 300, 32
    r = rng(1)
    a = r.standard_normal((B, T, Hv)) * 3
    a[0, 0, :4] = [25.0, 30.0, -25.0, 21.0]  # both softplus branches
    b = r.standard_normal((B, T, Hv))
    A_log = np.log(r.uniform(1, 16, Hv))
    dt = r.standard_normal(Hv) * 0.5
    if dtype == torch.bfloat16:
        a = torch.tensor(a).bfloat16().double().numpy()
        b = torch.tensor(b).bfloat16().double().numpy()
    dd, db_ = r.standard_normal((B, T, Hv)), r.standard_normal((B, T, Hv))
    print(f"gates log_space={log_space} neg={neg} {dtype}", flush=True)
    ta, tb = T_(a, dev, dtype, True), T_(b, dev, dtype, True)
    tA, tdt = T_(A_log, dev, grad=True), T_(dt, dev, grad=True)
    g, beta = gdn_block.gates(ta, tb, tA, tdt, log_space=log_space, allow_neg_eigval=neg)
    dec, bw = O.gates(a, b, A_log, dt)
    bw = bw * (2.0 if neg else 1.0)
    want_g = -np.exp(A_log) * O.softplus(a + dt) if log_space else dec
    assert nerr(np_(g), want_g) <= 1e-5
    assert nerr(np_(beta), bw) <= 1e-5
    grads = torch.autograd.grad([g, beta], [ta, tb, tA, tdt], [T_(dd, dev), T_(db_, dev)])
    torch.cuda.synchronize()
    d_decay = dd / dec if log_space else dd  # cotangent w.r.t. the decay
    want = O.gates_bwd(a, b, A_log, dt, d_decay, db_, allow_neg_eigval=neg)
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    for name, got, w in zip(("da", "db", "dA_log", "ddt_bias"), grads, want):
        assert nerr(np_(got), w) <= tol, (name, nerr(np_(got), w))


def test_gates_many_tokens_reduction(dev):
    """dA_log / ddt_bias over 2*8192 tokens: the block-per-column reduction path (> 128 partial rows)."""
    import gdn_block
    B, T, Hv = 2, 32768, 32
    r = rng(2)
    a, b = r.standard_normal((B, T, Hv)), r.standard_normal((B, T, Hv))
    A_log, dt = np.log(r.uniform(1, 16, Hv)), np.zeros(Hv)
    dd = r.standard_normal((B, T, Hv))
    ta = T_(a, dev, grad=True)
    tA, tdt = T_(A_log, dev, grad=True), T_(dt, dev, grad=True)
    g, _ = gdn_block.gates(ta, T_(b, dev), tA, tdt, log_space=True)
    got = torch.autograd.grad(g, [tA, tdt], T_(dd, dev))
    dec = O.compute_g(A_log, a, dt)
    want = O.gates_bwd(a, b, A_log, dt, dd / dec, np.zeros_like(dd))
    assert nerr(np_(got[0]), want[2]) <= 1e-4
    assert nerr(np_(got[1]), want[3]) <= 1e-4


# ------------------------------------------------------------------------------------------------ l2 norm


def test_l2norm_fixture(dev):
    import gdn_block
    hdr, q, qn, k, kn = binfix.load("gdn_l2norm.bin")
    H, Dk = int(hdr[0]), int(hdr[1])
    gq = gdn_block.l2norm(T_(q.reshape(H, Dk), dev), Dk ** -0.5)
    gk = gdn_block.l2norm(T_(k.reshape(H, Dk), dev), 1.0)
    torch.cuda.synchronize()
    assert nerr(np_(gq), qn.reshape(H, Dk)) <= 1e-5
    assert nerr(np_(gk), kn.reshape(H, Dk)) <= 1e-5


@pytest.mark.parametrize("D", [128, 64, 512, 32, 100, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_l2norm_fwd_bwd(dev, D, dtype):
    import gdn_block
    r = rng(D)
    x = r.standard_normal((3, 37, 5, D))
    if dtype == torch.bfloat16:
        x = torch.tensor(x).bfloat16().double().numpy()
    dy = r.standard_normal(x.shape)
    scale = D ** -0.5
    print(f"l2norm D={D} {dtype}", flush=True)
    tx = T_(x, dev, dtype, True)
    y = gdn_block.l2norm(tx, scale)
    (dx,) = torch.autograd.grad(y, tx, T_(dy, dev, dtype))
    torch.cuda.synchronize()
    tol_f, tol_b = (1e-5, 1e-4) if dtype == torch.float32 else (1e-2, 1e-2)
    dyq = np_(T_(dy, dev, dtype)).astype(np.float64)
    assert nerr(np_(y), O.l2norm(x, 1e-6, scale)) <= tol_f
    assert nerr(np_(dx), O.l2norm_bwd(x, dyq, 1e-6, scale)) <= tol_b


def test_l2norm_unaligned_view_and_zero_rows(dev):
    import gdn_block
    r = rng(5)
    base = torch.tensor(r.standard_normal(1 + 4 * 128), device=dev, dtype=torch.float32)
    x = base[1:].reshape(4, 128)  # 4-byte offset: element-load path after .contiguous() keeps it
    y = gdn_block.l2norm(x, 0.5)
    assert nerr(np_(y), O.l2norm(np_(x).astype(np.float64), 1e-6, 0.5)) <= 1e-5
    z = gdn_block.l2norm(torch.zeros((0, 128), device=dev))
    assert z.shape == (0, 128)


# ------------------------------------------------------------------------------------------------ conv + SiLU


def test_conv_fixture(dev):
    import gdn_block
    hdr, w, xs, want = binfix.load("gdn_conv.bin")
    C, K, T = int(hdr[0]), int(hdr[1]), int(hdr[2])
    out = gdn_block.conv_silu(T_(xs.reshape(1, T, C), dev), T_(w.reshape(C, K), dev))
    torch.cuda.synchronize()
    assert nerr(np_(out)[0], want.reshape(T, C)) <= 1e-5


# fp16 runs the kernels that read the element dtype from their arguments (bf16 and fp32 have it fixed at compile
# time)
@pytest.mark.parametrize("C,K,T", [(8192, 4, 300), (64, 4, 6), (100, 4, 70), (256, 2, 513), (96, 3, 129),
                                   (64, 8, 200)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_conv_fwd_bwd(dev, C, K, T, dtype):
    import gdn_block
    B = 2
    r = rng(C + K + T)
    x = r.standard_normal((B, T, C))
    if dtype != torch.float32:
        x = torch.tensor(x).to(dtype).double().numpy()
    w = r.standard_normal((C, K)) * 0.5
    dout = r.standard_normal((B, T, C))
    print(f"conv C={C} K={K} T={T} {dtype}", flush=True)
    tx, tw = T_(x, dev, dtype, True), T_(w, dev, grad=True)
    out = gdn_block.conv_silu(tx, tw)
    dx, dw = torch.autograd.grad(out, [tx, tw], T_(dout, dev, dtype))
    torch.cuda.synchronize()
    doq = np_(T_(dout, dev, dtype)).astype(np.float64)
    want_out, _ = O.conv_silu(x, w)
    want_dx, want_dw = O.conv_silu_bwd(x, w, doq)
    tol_f, tol_b = (1e-5, 1e-4) if dtype == torch.float32 else (1e-2, 1e-2)
    assert nerr(np_(out), want_out) <= tol_f
    assert nerr(np_(dx), want_dx) <= tol_b
    assert nerr(np_(dw), want_dw) <= tol_b


def test_conv_torch_weight_layout_and_state_continuation(dev):
    """[C,1,K] torch Conv1d weights; running [0,T1) then [T1,T) with the carried state equals one pass."""
    import gdn_block
    B, T, C, K, T1 = 2, 150, 192, 4, 61
    r = rng(9)
    x = T_(r.standard_normal((B, T, C)), dev)
    w = T_(r.standard_normal((C, 1, K)) * 0.5, dev)
    full = gdn_block.conv_silu(x, w)
    a, s = gdn_block.conv_silu(x[:, :T1], w, return_state=True)
    b, s2 = gdn_block.conv_silu(x[:, T1:], w, s, return_state=True)
    torch.cuda.synchronize()
    assert nerr(np_(torch.cat([a, b], 1)), np_(full)) <= 1e-6
    assert np.array_equal(np_(s), np_(x[:, T1 - K + 1:T1]))
    assert np.array_equal(np_(s2), np_(x[:, T - K + 1:]))
    # a decode step of one token from a state matches the full pass at that token
    c, _ = gdn_block.conv_silu(x[:, T1:T1 + 1], w, s, return_state=True)
    assert nerr(np_(c)[:, 0], np_(full)[:, T1]) <= 1e-6
    # state shorter than K-1 tokens of history: T=2 then state carries one old token
    d, s3 = gdn_block.conv_silu(x[:, :2], w, return_state=True)
    assert np.array_equal(np_(s3)[:, 0], np.zeros((B, C), np.float32))
    assert np.array_equal(np_(s3)[:, 1:], np_(x[:, :2]))


def test_conv_backward_with_state(dev):
    import gdn_block
    B, T, C, K = 1, 40, 64, 4
    r = rng(10)
    x = r.standard_normal((B, T, C))
    w = r.standard_normal((C, K)) * 0.5
    st = r.standard_normal((B, K - 1, C))
    dout = r.standard_normal((B, T, C))
    tx, tw = T_(x, dev, grad=True), T_(w, dev, grad=True)
    out = gdn_block.conv_silu(tx, tw, T_(st, dev))
    dx, dw = torch.autograd.grad(out, [tx, tw], T_(dout, dev))
    xx = np.concatenate([st, x], 1)  # the state is the K-1 inputs before x
    want_out, _ = O.conv_silu(xx, w)
    dxx, want_dw = O.conv_silu_bwd(xx, w, np.concatenate([np.zeros((B, K - 1, C)), dout], 1))
    assert nerr(np_(out), want_out[:, K - 1:]) <= 1e-5
    assert nerr(np_(dx), dxx[:, K - 1:]) <= 1e-4
    assert nerr(np_(dw), want_dw) <= 1e-4


# ------------------------------------------------------------------------------------------------ gated RMSNorm


def test_gated_rmsnorm_fixtures(dev):
    """The reference's rmsnorm (n = 2048) and silu_mul (n = 512) fixtures through the fused kernel: with z random,
    out = rmsnorm(x) * silu(z); with w = 1, out * rms(u) = silu(g) * u."""
    import gdn_block
    x, w, want_rms = binfix.load("ops_rmsnorm.bin")
    z = rng(3).standard_normal(x.shape).astype(np.float32)
    out = gdn_block.gated_rmsnorm(T_(x[None], dev), T_(z[None], dev), T_(w, dev))
    torch.cuda.synchronize()
    assert nerr(np_(out)[0], want_rms * O.silu(z.astype(np.float64))) <= 1e-5
    g, u, want_sm = binfix.load("ops_silu_mul.bin")
    rms = np.sqrt((u.astype(np.float64) ** 2).mean() + 1e-6)
    out = gdn_block.gated_rmsnorm(T_(u[None], dev), T_(g[None], dev), torch.ones(u.size, device=dev))
    torch.cuda.synchronize()
    assert nerr(np_(out)[0] * rms, want_sm) <= 1e-5


@pytest.mark.parametrize("D", [128, 64, 256, 100, 1024, 2000])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_rmsnorm_fwd_bwd(dev, D, dtype):
    import gdn_block
    r = rng(D + 1)
    y = r.standard_normal((2, 300, 4, D))
    z = r.standard_normal(y.shape) * 2
    if dtype == torch.bfloat16:
        y = torch.tensor(y).bfloat16().double().numpy()
        z = torch.tensor(z).bfloat16().double().numpy()
    w = 1 + 0.1 * r.standard_normal(D)
    dout = r.standard_normal(y.shape)
    print(f"gated rmsnorm D={D} {dtype}", flush=True)
    ty, tz, tw = T_(y, dev, dtype, True), T_(z, dev, dtype, True), T_(w, dev, grad=True)
    out = gdn_block.gated_rmsnorm(ty, tz, tw)
    dy, dz, dw = torch.autograd.grad(out, [ty, tz, tw], T_(dout, dev, dtype))
    torch.cuda.synchronize()
    doq = np_(T_(dout, dev, dtype)).astype(np.float64)
    tol_f, tol_b = (1e-5, 1e-4) if dtype == torch.float32 else (1e-2, 1e-2)
    assert nerr(np_(out), O.gated_rmsnorm(y, z, w, 1e-6)) <= tol_f
    want = O.gated_rmsnorm_bwd(y, z, w, doq, 1e-6)
    for name, got, wv in zip(("dy", "dz", "dw"), (dy, dz, dw), want):
        assert nerr(np_(got), wv) <= tol_b, (name, nerr(np_(got), wv))


# ------------------------------------------------------------------------------------------------ errors


def test_block_op_errors(dev):
    import gdn_block
    import gdn_lib as L
    x = torch.zeros((1, 4, 8), device=dev)
    with pytest.raises(ValueError, match="conv weight"):
        gdn_block.conv_silu(x, torch.zeros((7, 4), device=dev))
    with pytest.raises(L.GDNError, match="K > 8"):
        gdn_block.conv_silu(x, torch.zeros((8, 9), device=dev))
    with pytest.raises(ValueError, match="K must be >= 2"):
        gdn_block.conv_silu(x, torch.zeros((8, 1), device=dev))
    y = torch.zeros((2, 4097), device=dev, requires_grad=True)
    out = gdn_block.gated_rmsnorm(y, torch.zeros((2, 4097), device=dev), torch.zeros(4097, device=dev))
    with pytest.raises(L.GDNError, match="longer than 4096"):
        out.sum().backward()
    with pytest.raises(L.GDNError, match="Hv > 256"):
        gdn_block.gates(torch.zeros((2, 257), device=dev), torch.zeros((2, 257), device=dev),
                        torch.zeros(257, device=dev), torch.zeros(257, device=dev))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        gdn_block.l2norm(torch.zeros(4, 8))


# ------------------------------------------------------------------------------------------------ fused conv + split + L2 norm


def _conv_qkv_oracle(x, w, Hk, Dk, Hv, Dv, scale, dq, dk, dv, state=None):
    """Composition of the oracle's conv, split and L2 norm (forward) and their backwards."""
    B, T, C = x.shape
    K = w.shape[1]
    xx = x if state is None else np.concatenate([state, x], 1)
    c, _ = O.conv_silu(xx, w)
    c = c[:, -T:]
    kd = Hk * Dk
    q, k, v = c[..., :kd].reshape(B, T, Hk, Dk), c[..., kd:2 * kd].reshape(B, T, Hk, Dk), c[..., 2 * kd:]
    outs = (O.l2norm(q, 1e-6, scale), O.l2norm(k, 1e-6, 1.0), v.reshape(B, T, Hv, Dv))
    dc = np.concatenate([O.l2norm_bwd(q, dq, 1e-6, scale).reshape(B, T, -1),
                         O.l2norm_bwd(k, dk, 1e-6, 1.0).reshape(B, T, -1), dv.reshape(B, T, -1)], -1)
    if state is not None:
        dc = np.concatenate([np.zeros((B, K - 1, C)), dc], 1)
    dxx, dw = O.conv_silu_bwd(xx, w, dc)
    return outs, dxx[:, -T:], dw


@pytest.mark.parametrize("Hk,Dk,Hv,Dv,T", [(2, 128, 4, 128, 150), (16, 128, 32, 128, 70), (3, 64, 6, 32, 65),
                                           (2, 256, 4, 64, 40), (2, 32, 2, 48, 33)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_conv_qkv_fused(dev, Hk, Dk, Hv, Dv, T, dtype):
    import gdn_block
    B, K = 2, 4
    C = 2 * Hk * Dk + Hv * Dv
    r = rng(Hk * Dk + T)
    x = r.standard_normal((B, T, C))
    if dtype != torch.float32:
        x = torch.tensor(x).to(dtype).double().numpy()
    w = r.standard_normal((C, K)) * 0.5
    dq, dk = r.standard_normal((B, T, Hk, Dk)), r.standard_normal((B, T, Hk, Dk))
    dv = r.standard_normal((B, T, Hv, Dv))
    scale = Dk ** -0.5
    print(f"conv_qkv Hk={Hk} Dk={Dk} Hv={Hv} Dv={Dv} T={T} {dtype}", flush=True)
    tx, tw = T_(x, dev, dtype, True), T_(w, dev, grad=True)
    q, k, v = gdn_block.conv_qkv(tx, tw, Hk, Dk, Hv, Dv, scale)
    gq, gk, gv = (T_(a, dev, dtype) for a in (dq, dk, dv))
    dx, dw = torch.autograd.grad([q, k, v], [tx, tw], [gq, gk, gv])
    torch.cuda.synchronize()
    rq = lambda t: np_(t).astype(np.float64)
    outs, want_dx, want_dw = _conv_qkv_oracle(x, w, Hk, Dk, Hv, Dv, scale, rq(gq), rq(gk), rq(gv))
    tol_f, tol_b = (1e-5, 1e-4) if dtype == torch.float32 else (1e-2, 1e-2)
    for name, got, want in zip("qkv", (q, k, v), outs):
        assert got.is_contiguous()
        assert nerr(np_(got), want) <= tol_f, (name, nerr(np_(got), want))
    assert nerr(np_(dx), want_dx) <= tol_b, nerr(np_(dx), want_dx)
    assert nerr(np_(dw), want_dw) <= tol_b, nerr(np_(dw), want_dw)


def test_conv_qkv_state_and_fallback(dev):
    """Carried conv state through the fused kernels, and the composed path (K = 3, unaligned input) giving the
    same results as the oracle."""
    import gdn_block
    B, T, Hk, Dk, Hv, Dv, K = 1, 90, 2, 128, 4, 128, 4
    C = 2 * Hk * Dk + Hv * Dv
    r = rng(77)
    x, w = r.standard_normal((B, T, C)), r.standard_normal((C, K)) * 0.5
    st = r.standard_normal((B, K - 1, C))
    dq, dk = r.standard_normal((B, T, Hk, Dk)), r.standard_normal((B, T, Hk, Dk))
    dv = r.standard_normal((B, T, Hv, Dv))
    tx, tw = T_(x, dev, grad=True), T_(w, dev, grad=True)
    q, k, v, s_out = gdn_block.conv_qkv(tx, tw, Hk, Dk, Hv, Dv, 0.1, state=T_(st, dev), return_state=True)
    dx, dw = torch.autograd.grad([q, k, v], [tx, tw], [T_(a, dev) for a in (dq, dk, dv)])
    outs, want_dx, want_dw = _conv_qkv_oracle(x, w, Hk, Dk, Hv, Dv, 0.1, dq, dk, dv, state=st)
    for got, want in zip((q, k, v), outs):
        assert nerr(np_(got), want) <= 1e-5
    assert nerr(np_(dx), want_dx) <= 1e-4 and nerr(np_(dw), want_dw) <= 1e-4
    assert np.array_equal(np_(s_out), x[:, T - K + 1:].astype(np.float32))
    # K = 3 is not fused: the composed kernels run instead
    w3 = r.standard_normal((C, 3)) * 0.5
    tw3 = T_(w3, dev, grad=True)
    q, k, v = gdn_block.conv_qkv(tx, tw3, Hk, Dk, Hv, Dv, 0.1)
    dx, dw = torch.autograd.grad([q, k, v], [tx, tw3], [T_(a, dev) for a in (dq, dk, dv)])
    outs, want_dx, want_dw = _conv_qkv_oracle(x, w3, Hk, Dk, Hv, Dv, 0.1, dq, dk, dv)
    for got, want in zip((q, k, v), outs):
        assert nerr(np_(got), want) <= 1e-5
    assert nerr(np_(dx), want_dx) <= 1e-4 and nerr(np_(dw), want_dw) <= 1e-4
    # an input at a 4-byte offset is copied to an aligned buffer and still takes the fused path
    base = T_(np.concatenate([[0.0], x.ravel()]), dev)
    xo = base[1:].view(B, T, C)
    q2, k2, v2 = gdn_block.conv_qkv(xo, tw, Hk, Dk, Hv, Dv, 0.1)
    outs, _, _ = _conv_qkv_oracle(x, w, Hk, Dk, Hv, Dv, 0.1, dq, dk, dv)
    for got, want in zip((q2, k2, v2), outs):
        assert nerr(np_(got), want) <= 1e-5
