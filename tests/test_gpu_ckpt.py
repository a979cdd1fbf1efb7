"""GPU parity of the chunked form's group-wise paths: checkpointing (chunk > 64), forward-only calls, a NULL exit-state
cotangent and the measured workload at its full length.

* checkpointing (tools/gdn_checkpoint.py:39-50,81-95): the forward keeps ceil(T/W) - 1 fp32 window states and the
  backward rebuilds each group of windows from them; checked against the fp64 oracle (1e-4 fp32, 1e-2 bf16), against
  the chunk = 64 run of the same engine, with groups of one or two windows forced through a small workspace, and at
  T = 16384 against the oracle on one key-head group and through full-size properties (agreement with chunk = 64,
  finite gradients, peak memory);
* forward-only calls (saved = NULL, frozen layers) against the oracle's forward, group by group;
* the headline workload (B=4, T=4096, Hk=16, Hv=32, bf16 q/k/v/dO, fp32 state) against the fp64 oracle on two
  key-head groups, with the errors printed at T = 600, 2048 and 4096;
* fp32 at B=1, T=4096, Hk=16, Hv=32 on both forms against the fp64 oracle at 1e-4 (two key-head groups).
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
    return float(np.abs(a - b).max()) / max(float(np.abs(b).max()), 1e-30)


def _inputs(B, T, Hk, Hv, seed, s0_std=0.02, bf16=False, dS_T=True):
    d = O.make_inputs(B, T, Hk, Hv, D, seed=seed, s0_std=s0_std)
    d["dS_T"] = ((np.random.default_rng(seed + 7).standard_normal(d["state"].shape) * 0.1).astype(np.float32)
                 if dS_T else np.zeros_like(d["state"]))
    if bf16:
        bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
        d = dict(d, q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), dy=bf(d["dy"]))
    return d


def _engine(d, dev, chunk, dtype=torch.float32, state_grad=True, form="chunk"):
    """gdn_engine forward + VJP (log gates), grads of y (and of S_T when state_grad)."""
    import gdn_engine
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    q, k, v = (t(d[n], dtype).requires_grad_(True) for n in ("q", "k", "v"))
    g, beta, S0 = (t(d[n]).requires_grad_(True) for n in ("g_log", "beta", "state"))
    leaves = [q, k, v, g, beta, S0]
    y, S = gdn_engine.recurrence(q, k, v, g, beta, S0, None, chunk, log_gate=True, output_dtype=dtype, form=form)
    if state_grad:
        grads = torch.autograd.grad([y, S], leaves, [t(d["dy"], dtype), t(d["dS_T"])])
    else:
        grads = torch.autograd.grad([y], leaves, [t(d["dy"], dtype)])
    torch.cuda.synchronize()
    return [x.detach().float().cpu().numpy() for x in (y, S, *grads)]


def _abi(d, dev, chunk, dtype=torch.float32, fwd_ws_T=None, bwd_ws_T=None):
    """The same through the C ABI, with the forward / backward workspaces sized for fwd_ws_T / bwd_ws_T tokens
    (fewer tokens than T force smaller groups)."""
    import gdn_lib as L
    lib = L.load()
    B, T, Hk = d["q"].shape[:3]
    Hv = d["v"].shape[2]
    code = L.DTYPE_CODE[dtype]
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt).contiguous()
    q, k, v = (t(d[n], dtype) for n in ("q", "k", "v"))
    g, beta, S0, dS_T = (t(d[n]) for n in ("g_log", "beta", "state", "dS_T"))
    dy = t(d["dy"], dtype)
    y = torch.empty((B, T, Hv, D), device=dev, dtype=dtype)
    ST = torch.empty((B, Hv, D, D), device=dev)
    common = (D, D, chunk, L.GATE_LOG, 0, L.FORM_CHUNK, code)
    n_saved = lib.gdn_saved_bytes(B, T, Hk, Hv, *common)
    saved = torch.empty(max(n_saved, 1), device=dev, dtype=torch.uint8)
    n_fws = lib.gdn_fwd_workspace_bytes(B, fwd_ws_T or T, Hk, Hv, *common, 1)
    fws = torch.empty(max(n_fws, 1), device=dev, dtype=torch.uint8)
    L.check(lib.gdn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), S0.data_ptr(),
                        None, y.data_ptr(), ST.data_ptr(), saved.data_ptr(), n_saved, fws.data_ptr(), n_fws,
                        B, T, Hk, Hv, D, D, chunk, code, code, L.GATE_LOG, L.FORM_CHUNK, None))
    outs = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(g),
            torch.empty_like(beta), torch.empty_like(S0)]
    n_bws = lib.gdn_bwd_workspace_bytes(B, bwd_ws_T or T, Hk, Hv, *common)
    bws = torch.empty(max(n_bws, 1), device=dev, dtype=torch.uint8)
    L.check(lib.gdn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), S0.data_ptr(),
                        None, saved.data_ptr(), n_saved, dy.data_ptr(), dS_T.data_ptr(),
                        *(o.data_ptr() for o in outs), bws.data_ptr(), n_bws, B, T, Hk, Hv, D, D, chunk,
                        code, code, code, L.GATE_LOG, L.FORM_CHUNK, None))
    torch.cuda.synchronize()
    return [x.float().cpu().numpy() for x in (y, ST, *outs)]


def _oracle_group(d, hk, rep, b=0):
    sl = slice(hk * rep, hk * rep + rep)
    (y, S), g = O.gated_delta_chunked_vjp(
        d["q"][b:b + 1, :, hk:hk + 1], d["k"][b:b + 1, :, hk:hk + 1], d["v"][b:b + 1, :, sl],
        d["decay"][b:b + 1, :, sl], d["beta"][b:b + 1, :, sl], d["state"][b:b + 1, sl], None,
        d["dy"][b:b + 1, :, sl], d["dS_T"][b:b + 1, sl], chunk=64, dtype=np.float64)
    return [y, S, g[0], g[1], g[2], g[3] * d["decay"][b:b + 1, :, sl], g[4], g[5]]


def _slice(got, hk, rep, b=0):
    sl = slice(hk * rep, hk * rep + rep)
    return [got[0][b:b + 1, :, sl], got[1][b:b + 1, sl], got[2][b:b + 1, :, hk:hk + 1],
            got[3][b:b + 1, :, hk:hk + 1], got[4][b:b + 1, :, sl], got[5][b:b + 1, :, sl],
            got[6][b:b + 1, :, sl], got[7][b:b + 1, sl]]


def _check_groups(got, d, groups, rep, tol, label):
    for b, hk in groups:
        want = _oracle_group(d, hk, rep, b)
        errs = {n: nerr(a, w) for n, a, w in zip(NAMES, _slice(got, hk, rep, b), want)}
        print(label, f"b={b} hk={hk}", {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
        for n, e in errs.items():
            assert e <= tol, (label, b, hk, n, e)


# ---------------------------------------------------------------------------------------------- checkpointing

def test_checkpoint_fp32_measured_heads_against_oracle(dev):
    """fp32, B=1, T=2048, Hk=16, Hv=32, D=128, chunk=256 through gated_delta_ops_checkpointed: two key-head
    groups against the fp64 oracle at 1e-4, and the state snapshots are what the call keeps."""
    import gdn_checkpoint
    import gdn_lib as L
    d = _inputs(1, 2048, 16, 32, seed=31)
    print("checkpoint fp32 B=1 T=2048 Hv=32 chunk=256", flush=True)
    t = lambda x: torch.tensor(np.asarray(x), device=dev).requires_grad_(True)
    leaves = [t(d[n]) for n in ("q", "k", "v", "decay", "beta", "state")]
    y, S = gdn_checkpoint.gated_delta_ops_checkpointed(*leaves, None, 256)
    grads = torch.autograd.grad([y, S], leaves, [t(d["dy"]), t(d["dS_T"])])
    torch.cuda.synchronize()
    got = [x.detach().cpu().numpy() for x in (y, S, *grads)]
    got[5] = got[5] * d["decay"]   # d/d(decay) -> d/d(log decay), as the oracle group reports
    _check_groups(got, d, ((0, 0), (0, 11)), 2, 1e-4, "ckpt fp32")
    snaps = L.load().gdn_saved_bytes(1, 2048, 16, 32, D, D, 256, L.GATE_DECAY, 0, L.FORM_CHUNK, L.F32)
    assert snaps == 7 * 32 * D * D * 4


def test_checkpoint_t16384_against_oracle(dev):
    """The checkpoint configuration at its own length: fp32, B=1, T=16384, Hk=16, Hv=32, D=128, S0 ~ N(0, 0.02),
    snapshots every 256 tokens (63 windows, several backward groups) through gated_delta_ops_checkpointed, with one
    key-head group (two value heads) against the fp64 oracle at 1e-4."""
    import gdn_checkpoint
    d = _inputs(1, 16384, 16, 32, seed=41)
    print("checkpoint fp32 B=1 T=16384 Hv=32 chunk=256 against the oracle (key head 5)", flush=True)
    t = lambda x: torch.tensor(np.asarray(x), device=dev).requires_grad_(True)
    leaves = [t(d[n]) for n in ("q", "k", "v", "decay", "beta", "state")]
    y, S = gdn_checkpoint.gated_delta_ops_checkpointed(*leaves, None, 256)
    grads = torch.autograd.grad([y, S], leaves, [t(d["dy"]), t(d["dS_T"])])
    torch.cuda.synchronize()
    got = [x.detach().cpu().numpy() for x in (y, S, *grads)]
    del y, S, grads, leaves
    got[5] = got[5] * d["decay"]   # d/d(decay) -> d/d(log decay), as the oracle group reports
    _check_groups(got, d, ((0, 5),), 2, 1e-4, "ckpt fp32 T=16384")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_checkpoint_groups_of_windows(dev, dtype):
    """B=2, T=1000 (the last window and chunk ragged), Hk=2, Hv=4, chunk=100 (windows of 128 tokens): groups of one
    and two windows (forced by small workspaces) give the same results as one group and as chunk = 64, and match
    the fp64 oracle."""
    bf = dtype == torch.bfloat16
    d = _inputs(2, 1000, 2, 4, seed=17, bf16=bf)
    tol = 1e-2 if bf else 1e-4
    print(f"checkpoint groups {dtype}", flush=True)
    one = _abi(d, dev, 100, dtype)
    full = _abi(d, dev, 64, dtype)
    for fT, bT in ((128, 128), (256, 256), (128, 384)):
        print(f"  forward groups of {fT} tokens, backward groups of {bT}", flush=True)
        got = _abi(d, dev, 100, dtype, fwd_ws_T=fT, bwd_ws_T=bT)
        for n, a, w in zip(NAMES, got, one):
            assert nerr(a, w) <= 1e-6, (fT, bT, n, nerr(a, w))
    for n, a, w in zip(NAMES, one, full):
        assert nerr(a, w) <= (2e-3 if bf else 1e-5), (n, nerr(a, w))
    _check_groups(one, d, ((0, 0), (1, 1)), 2, tol, f"ckpt {dtype}")


def test_checkpoint_t16384_full_size(dev):
    """The checkpoint configuration itself, fp32, B=1, T=16384, Hk=16, Hv=32, snapshots every 256 tokens: every
    output agrees with the chunk = 64 run (whose parity the oracle pins at smaller T), the gradients are finite, and
    the call keeps 63 states instead of the 64-token tile set, with a lower peak."""
    B, T, Hk, Hv = 1, 16384, 16, 32
    d = _inputs(B, T, Hk, Hv, seed=9, s0_std=0.0)
    # inputs, dy, dS_T, y, S_T and the six gradients, all fp32
    io = 4 * (2 * (2 * B * T * Hk * D + B * T * Hv * D + 2 * B * T * Hv + B * Hv * D * D)
              + 2 * B * T * Hv * D + 2 * B * Hv * D * D)
    print("checkpoint fp32 B=1 T=16384 chunk=256 vs 64", flush=True)
    extra, res = {}, {}
    for chunk in (256, 64):
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        res[chunk] = _engine(d, dev, chunk)
        extra[chunk] = (torch.cuda.max_memory_allocated(dev) - base - io) / 2 ** 30
    print(f"peak GiB beyond inputs, outputs and gradients ({io / 2 ** 30:.2f} GiB)",
          {c: f"{p:.2f}" for c, p in extra.items()}, flush=True)
    for n, a, w in zip(NAMES, res[256], res[64]):
        assert np.isfinite(a).all(), n
        assert nerr(a, w) <= 1e-5, (n, nerr(a, w))
    assert extra[256] < 0.5 * extra[64]
    assert extra[256] < 1.2


# ---------------------------------------------------------------------------------------------- forward only

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_forward_only_against_oracle(dev, dtype):
    """saved = NULL (frozen layers, no_grad): y and S_T of the chunked form against the oracle's forward, in one
    group and in groups of one 64-token chunk."""
    import gdn_engine
    import gdn_lib as L
    bf = dtype == torch.bfloat16
    d = _inputs(2, 300, 2, 4, seed=23, bf16=bf)
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    with torch.no_grad():
        y, S = gdn_engine.recurrence(t(d["q"], dtype), t(d["k"], dtype), t(d["v"], dtype), t(d["g_log"]),
                                     t(d["beta"]), t(d["state"]), None, 64, log_gate=True, output_dtype=dtype,
                                     form="chunk")
    wy, wS = O.gated_delta_chunked(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], None, 64,
                                   dtype=np.float64)
    tol = 1e-2 if bf else 1e-4
    assert nerr(y.float().cpu().numpy(), wy) <= tol
    assert nerr(S.cpu().numpy(), wS) <= tol
    # groups of one chunk through the C ABI
    lib = L.load()
    code = L.DTYPE_CODE[dtype]
    B, T, Hk, Hv = 2, 300, 2, 4
    n_ws = lib.gdn_fwd_workspace_bytes(B, 64, Hk, Hv, D, D, 64, L.GATE_LOG, 0, L.FORM_CHUNK, code, 0)
    assert n_ws > 0
    ws = torch.empty(n_ws, device=dev, dtype=torch.uint8)
    q, k, v = (t(d[n], dtype).contiguous() for n in ("q", "k", "v"))
    g, beta, S0 = (t(d[n]).contiguous() for n in ("g_log", "beta", "state"))
    y2 = torch.empty_like(y)
    S2 = torch.empty_like(S)
    L.check(lib.gdn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), S0.data_ptr(),
                        None, y2.data_ptr(), S2.data_ptr(), None, 0, ws.data_ptr(), n_ws, B, T, Hk, Hv, D, D, 64,
                        code, code, L.GATE_LOG, L.FORM_CHUNK, None))
    torch.cuda.synchronize()
    assert nerr(y2.float().cpu().numpy(), y.float().cpu().numpy()) <= 1e-6
    assert nerr(S2.cpu().numpy(), S.cpu().numpy()) <= 1e-6


def test_forward_only_keeps_no_tiles(dev):
    """A no_grad forward of the measured workload (B=4, T=4096, Hv=32, bf16) allocates its output and a bounded group
    workspace, far below the 1.6 GB tile set a training forward keeps."""
    import gdn_engine
    import gdn_lib as L
    B, T, Hk, Hv = 4, 4096, 16, 32
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    q = torch.randn(B, T, Hk, D, device=dev, generator=g).bfloat16() * 0.05
    k = torch.randn(B, T, Hk, D, device=dev, generator=g).bfloat16() * 0.05
    v = torch.randn(B, T, Hv, D, device=dev, generator=g).bfloat16()
    gl = -torch.rand(B, T, Hv, device=dev, generator=g)
    beta = torch.rand(B, T, Hv, device=dev, generator=g)
    S0 = torch.zeros(B, Hv, D, D, device=dev)
    tiles = L.load().gdn_saved_bytes(B, T, Hk, Hv, D, D, 64, L.GATE_LOG, 0, L.FORM_CHUNK, L.BF16)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    with torch.no_grad():
        y, S = gdn_engine.recurrence(q, k, v, gl, beta, S0, None, 64, log_gate=True, output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated(dev) - base - y.numel() * 2 - S.numel() * 4
    print(f"forward-only extra {extra / 2 ** 20:.0f} MiB, tile set {tiles / 2 ** 20:.0f} MiB", flush=True)
    assert tiles > 1.5e9
    assert extra < 0.2 * tiles
    assert torch.isfinite(y.float()).all() and torch.isfinite(S).all()


# ---------------------------------------------------------------------------------------------- cotangents

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_null_state_cotangent_chunked(dev, dtype):
    """Grads of y only (the exit-state cotangent reaches the library as NULL, as in bench.py) at D=128 on the
    chunked form, against the oracle with dS_T = 0."""
    bf = dtype == torch.bfloat16
    d = _inputs(2, 200, 2, 4, seed=51, bf16=bf, dS_T=False)
    got = _engine(d, dev, 64, dtype, state_grad=False)
    _check_groups(got, d, ((0, 0), (1, 1)), 2, 1e-2 if bf else 1e-4, f"null dS_T {dtype}")


def test_bf16_inputs_fp16_output(dev):
    """bf16 q/k/v with an fp16 y: the fp16 cotangent is widened before the chunked backward (which reads bf16 or
    fp32 dy) and the gradients match the oracle."""
    import gdn_vjp
    d = _inputs(1, 150, 2, 4, seed=61, bf16=True)
    d["dy"] = torch.tensor(d["dy"]).half().float().numpy()
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt).requires_grad_(True)
    leaves = [t(d["q"], torch.bfloat16), t(d["k"], torch.bfloat16), t(d["v"], torch.bfloat16), t(d["decay"]),
              t(d["beta"]), t(d["state"])]
    y, S = gdn_vjp.gated_delta_chunked(*leaves, output_dtype=torch.float16)
    assert y.dtype == torch.float16
    grads = torch.autograd.grad([y, S], leaves, [t(d["dy"], torch.float16), t(d["dS_T"])])
    got = [x.detach().float().cpu().numpy() for x in (y, S, *grads)]
    got[5] = got[5] * d["decay"]
    _check_groups(got, d, ((0, 0), (0, 1)), 2, 1e-2, "bf16 in, fp16 out")


# ---------------------------------------------------------------------------------------------- headline workload

def test_headline_config_against_oracle_full_length(dev):
    """B=4, Hk=16, Hv=32, D=128, bf16 q/k/v/dO, fp32 state and gates, chunk 64: two key-head groups against the
    fp64 oracle at T = 600, 2048 and 4096 (the measured length), normalised error <= 1e-2, errors printed."""
    grow = {}
    for T in (600, 2048, 4096):
        d = _inputs(4, T, 16, 32, seed=77, bf16=True)
        print(f"headline bf16 B=4 T={T}", flush=True)
        got = _engine(d, dev, 64, torch.bfloat16, state_grad=False)
        d["dS_T"] = np.zeros_like(d["state"])
        worst = {}
        for b, hk in ((0, 3), (3, 14)):
            want = _oracle_group(d, hk, 2, b)
            for n, a, w in zip(NAMES, _slice(got, hk, 2, b), want):
                worst[n] = max(worst.get(n, 0.0), nerr(a, w))
        print(f"  T={T}", {n: f"{e:.1e}" for n, e in worst.items()}, flush=True)
        grow[T] = worst
        for n, e in worst.items():
            assert e <= 1e-2, (T, n, e)


@pytest.mark.parametrize("form", ["chunk", "recurrent"])
def test_fp32_b1_t4096_against_oracle(dev, form):
    """fp32 throughout, B=1, T=4096, Hk=16, Hv=32, D=128 (32 value heads), S0 ~ N(0, 0.02) and a full exit-state
    cotangent: two key-head groups of every output against the fp64 oracle, normalised error <= 1e-4, on the
    chunked form (chunk 64) and on the token-recurrent form (snapshots every 64 tokens)."""
    d = _inputs(1, 4096, 16, 32, seed=91)
    print(f"fp32 B=1 T=4096 form={form}", flush=True)
    got = _engine(d, dev, 64, torch.float32, state_grad=True, form=form)
    _check_groups(got, d, ((0, 0), (0, 11)), 2, 1e-4, f"fp32 B=1 T=4096 {form}")
