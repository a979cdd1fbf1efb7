"""GPU parity of per-channel (vector) gates, one decay per key channel [B,T,Hv,Dk] (tools/gdn_vjp.py:174-179,
311-314), against the fp64 oracle.

With bf16 inputs, Dk = Dv = 128 and no mask they run on the chunked form (gdn_chunk_vg.hip: the decay factors of
the pair sums formed per 16-token block pair through a boundary token, so that no factor exceeds 1); fp32 inputs and
masked calls run on the token-recurrent form.  Bars (normalised error max|gpu - oracle| / max|oracle| per output):
1e-2 on the chunked form with bf16 inputs; on the recurrent form 1e-4 for fp32 inputs and for the fp32 outputs with
bf16 inputs, 4e-3 for its bf16 dq / dk / dv.
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


def _inputs(B, T, Hk, Hv, seed, decay=(0.7, 1.0), log_decay=None, masked=False, bf16=True):
    """The reference's matrix distributions (tools/test_gdn_vjp.py:21-55) at Dk = Dv = 128: q, k L2-normalised (q
    times Dk^-1/2), decays U(0.7, 1) per channel (or exp(-U(log_decay))), beta U(0.05, 0.95), S0, dy, dS_T normal."""
    rng = np.random.default_rng(seed)
    q = O.l2norm(rng.standard_normal((B, T, Hk, D)), 1e-6, D ** -0.5)
    k = O.l2norm(rng.standard_normal((B, T, Hk, D)), 1e-6, 1.0)
    if log_decay is None:
        dec = rng.uniform(decay[0], decay[1], (B, T, Hv, D))
    else:
        dec = np.exp(-rng.uniform(log_decay[0], log_decay[1], (B, T, Hv, D)))
    d = dict(q=q, k=k, v=rng.standard_normal((B, T, Hv, D)), decay=dec, beta=rng.uniform(0.05, 0.95, (B, T, Hv)),
             state=rng.standard_normal((B, Hv, D, D)) * 0.1, dy=rng.standard_normal((B, T, Hv, D)),
             dS_T=rng.standard_normal((B, Hv, D, D)) * 0.1)
    d = {n: x.astype(np.float32) for n, x in d.items()}
    d["mask"] = (np.random.default_rng(seed + 1).random((B, T)) > 0.2) if masked else None
    if bf16:
        bf = lambda x: torch.tensor(x).bfloat16().float().numpy()
        d = dict(d, q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), dy=bf(d["dy"]))
    return d


def _gpu(d, dev, dtype, chunk=64, form=None):
    import gdn_engine
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    q, k, v = (t(d[n], dtype).requires_grad_(True) for n in ("q", "k", "v"))
    g, beta, S0 = (t(d[n]).requires_grad_(True) for n in ("decay", "beta", "state"))
    mask = None if d["mask"] is None else torch.tensor(d["mask"], device=dev)
    y, S = gdn_engine.recurrence(q, k, v, g, beta, S0, mask, chunk, form=form)
    grads = torch.autograd.grad([y, S], [q, k, v, g, beta, S0], [t(d["dy"], y.dtype), t(d["dS_T"])])
    torch.cuda.synchronize()
    return [x.detach().float().cpu().numpy() for x in (y, S, *grads)]


def _oracle(d, chunk=64):
    (y, S), g = O.gated_delta_chunked_vjp(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], d["mask"],
                                          d["dy"], d["dS_T"], chunk=chunk, dtype=np.float64)
    return [y, S, *g]


def _bar(name, chunked, bf16):
    if chunked:
        return 1e-2
    if bf16 and name in ("dq", "dk", "dv"):
        return 4e-3
    return 1e-4


def _check(got, want, chunked, bf16, label):
    errs = {n: nerr(a, w) for n, a, w in zip(NAMES, got, want)}
    print(label, {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= _bar(n, chunked, bf16), (label, n, e)


def test_vector_gates_select_the_chunked_form_for_bf16(dev):
    import gdn_lib as L
    lib = L.load()
    assert lib.gdn_select_form(4, D, D, 0, L.GATE_DECAY_VEC, L.FORM_AUTO, L.BF16) == L.FORM_CHUNK
    assert lib.gdn_select_form(4, D, D, 0, L.GATE_DECAY_VEC, L.FORM_AUTO, L.F32) == L.FORM_RECURRENT
    assert lib.gdn_select_form(4, D, D, 1, L.GATE_DECAY_VEC, L.FORM_AUTO, L.BF16) == L.FORM_RECURRENT


@pytest.mark.parametrize("T", [1, 63, 64, 65, 200])
@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_reference_vector_gate_matrix_at_d128(dev, T, masked, dtype):
    """The reference's lengths with and without a mask, bf16 (chunked form without a mask) and fp32 (recurrent)."""
    bf16 = dtype == torch.bfloat16
    d = _inputs(2, T, 2, 4, seed=300 + T + 7 * masked, masked=masked, bf16=bf16)
    print(f"vector gates {dtype} T={T} masked={masked}", flush=True)
    _check(_gpu(d, dev, dtype), _oracle(d), bf16 and not masked, bf16, f"T={T} masked={masked} {dtype}")


@pytest.mark.parametrize("log_decay", [(0.0, 1.5), (0.0, 6.0), (0.0, 9.0)])
def test_strong_decays_on_the_chunked_form(dev, log_decay):
    """Decays down to exp(-9) per token: over a chunk exp(-G) reaches exp(570), beyond fp32, while every factor the
    chunked form forms stays <= 1."""
    d = _inputs(2, 200, 2, 4, seed=11, log_decay=log_decay)
    print(f"vector gates bf16 T=200 log decays {log_decay}", flush=True)
    _check(_gpu(d, dev, torch.bfloat16), _oracle(d), True, True, f"log decay {log_decay}")


def test_checkpointed_and_forward_only(dev):
    """chunk = 256 (window snapshots, each group of windows rebuilt in backward) against the oracle; a forward-only
    call (no graph) equals the training forward."""
    import gdn_engine
    d = _inputs(1, 1000, 2, 4, seed=21, log_decay=(0.0, 1.5))
    print("vector gates bf16 T=1000 chunk=256", flush=True)
    got = _gpu(d, dev, torch.bfloat16, chunk=256)
    _check(got, _oracle(d), True, True, "ckpt 256")
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    with torch.no_grad():
        y, S = gdn_engine.recurrence(t(d["q"], torch.bfloat16), t(d["k"], torch.bfloat16), t(d["v"], torch.bfloat16),
                                     t(d["decay"]), t(d["beta"]), t(d["state"]), None, 64)
    torch.cuda.synchronize()
    assert nerr(y.float().cpu().numpy(), got[0]) <= 2e-3
    assert nerr(S.cpu().numpy(), got[1]) <= 2e-3


def test_measured_workload_chunked_against_recurrent(dev):
    """B=4, T=4096, Hk=16, Hv=32, D=128, bf16, decays exp(-U(0, 1.5)) per channel (the measured vector-gate
    workload): the chunked form against the recurrent form, every output."""
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    B, T, Hk, Hv = 4, 4096, 16, 32
    n = lambda *s: torch.randn(*s, device=dev, generator=g)
    q = (torch.nn.functional.normalize(n(B, T, Hk, D), dim=-1) * D ** -0.5).bfloat16()
    k = torch.nn.functional.normalize(n(B, T, Hk, D), dim=-1).bfloat16()
    v = n(B, T, Hv, D).bfloat16()
    dec = torch.exp(-1.5 * torch.rand(B, T, Hv, D, device=dev, generator=g))
    beta = torch.sigmoid(n(B, T, Hv))
    dy = n(B, T, Hv, D).bfloat16()
    print("vector gates bf16 B=4 T=4096 Hv=32: chunked against recurrent", flush=True)
    res = {}
    import gdn_engine
    for form in ("chunk", "recurrent"):
        xs = [x.detach().clone().requires_grad_(True) for x in (q, k, v, dec, beta)]
        S0 = torch.zeros(B, Hv, D, D, device=dev, requires_grad=True)
        y, S = gdn_engine.recurrence(*xs, S0, None, 64, form=form, output_dtype=torch.bfloat16)
        grads = torch.autograd.grad([y], [*xs, S0], [dy])
        torch.cuda.synchronize()
        res[form] = [x.detach().float() for x in (y, S, *grads)]
    for name, a, b in zip(NAMES, res["chunk"], res["recurrent"]):
        e = float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))
        print(f"  {name} {e:.1e}", flush=True)
        assert e <= 1e-2, (name, e)


@pytest.mark.parametrize("T", [1, 65, 200])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_log_vector_gates_at_any_decay_size(dev, T, dtype):
    """Per-channel log decays (log_gate=True, [B,T,Hv,Dk]): -U(0, 20) with about 2% of them -inf, so decays from 1
    down to 2e-9 and exact zeros.  bf16 runs the chunked form, whose gradient for the log decay is its suffix sums
    with no division by the decay; fp32 the recurrent one.  dg against the oracle's d/d(decay) times the decay."""
    import gdn_engine
    bf16 = dtype == torch.bfloat16
    d = _inputs(2, T, 2, 4, seed=700 + T, bf16=bf16)
    rng = np.random.default_rng(710 + T)
    gl = -rng.uniform(0.0, 20.0, (2, T, 4, D))
    gl[rng.random(gl.shape) < 0.02] = -np.inf
    d["decay"] = np.exp(gl).astype(np.float32)
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt)
    q, k, v = (t(d[n], dtype).requires_grad_(True) for n in ("q", "k", "v"))
    g = t(gl.astype(np.float32)).requires_grad_(True)
    beta, S0 = (t(d[n]).requires_grad_(True) for n in ("beta", "state"))
    print(f"log vector gates {dtype} T={T}", flush=True)
    y, S = gdn_engine.recurrence(q, k, v, g, beta, S0, None, 64, log_gate=True)
    grads = torch.autograd.grad([y, S], [q, k, v, g, beta, S0], [t(d["dy"], y.dtype), t(d["dS_T"])])
    torch.cuda.synchronize()
    got = [x.detach().float().cpu().numpy() for x in (y, S, *grads)]
    want = _oracle(d)
    want[5] = want[5] * d["decay"]
    assert all(np.isfinite(x).all() for x in got)
    _check(got, want, bf16, bf16, f"log gates T={T} {dtype}")


@pytest.mark.parametrize("T, chunk", [(1, 64), (65, 64), (200, 64), (700, 256)])
def test_decays_of_any_size_on_the_chunked_form(dev, T, chunk):
    """Per-channel decays exp(-U(0, 20)) with about 2% exact zeros, on the chunked form (pinned): d/d(decay) is formed
    by ck_vg_dg from factors <= 1 (no division by the decay), so it holds the chunked bar against the oracle's
    recurrence, which differentiates the decay itself, down to decays of 2e-9 and at the zeros (taken as 2^-64:
    the gradient there differs from the one at zero by terms of that size).  chunk = 256 rebuilds each group of
    windows in backward."""
    d = _inputs(2, T, 2, 4, seed=800 + T, log_decay=(0.0, 20.0))
    rng = np.random.default_rng(810 + T)
    d["decay"] = np.where(rng.random(d["decay"].shape) < 0.02, 0.0, d["decay"]).astype(np.float32)
    print(f"vector decays of any size bf16 T={T} chunk={chunk}, chunked form", flush=True)
    got = _gpu(d, dev, torch.bfloat16, chunk=chunk, form="chunk")
    assert all(np.isfinite(x).all() for x in got)
    _check(got, _oracle(d, chunk), True, True, f"decays of any size T={T} chunk={chunk}")


@pytest.mark.parametrize("Hk, Hv", [(4, 4), (1, 4)])
def test_decays_on_the_chunked_form_across_head_groupings(dev, Hk, Hv):
    """Per-channel decays with 2% zeros on the chunked form at one and four value heads per key head: ck_vg_dg reads
    q and k through the key head of each value head, and ck_bwd_local_vg sums dq and dk over a key head's value
    heads."""
    d = _inputs(2, 130, Hk, Hv, seed=830 + Hk, log_decay=(0.0, 6.0))
    rng = np.random.default_rng(840 + Hk)
    d["decay"] = np.where(rng.random(d["decay"].shape) < 0.02, 0.0, d["decay"]).astype(np.float32)
    print(f"vector decays bf16 T=130 Hk={Hk} Hv={Hv}, chunked form", flush=True)
    _check(_gpu(d, dev, torch.bfloat16, form="chunk"), _oracle(d), True, True, f"decays Hk={Hk} Hv={Hv}")


def _abi_vg(d, dev, chunk, fwd_ws_T=None, bwd_ws_T=None):
    """Forward + backward of per-channel decays (bf16) through the C ABI, with the forward / backward workspaces
    sized for fwd_ws_T / bwd_ws_T tokens (fewer tokens than T force smaller groups of windows)."""
    import gdn_lib as L
    lib = L.load()
    B, T, Hk = d["q"].shape[:3]
    Hv = d["v"].shape[2]
    t = lambda x, dt=torch.float32: torch.tensor(np.asarray(x), device=dev, dtype=dt).contiguous()
    q, k, v, dy = (t(d[n], torch.bfloat16) for n in ("q", "k", "v", "dy"))
    g, beta, S0, dS_T = (t(d[n]) for n in ("decay", "beta", "state", "dS_T"))
    y = torch.empty((B, T, Hv, D), device=dev, dtype=torch.bfloat16)
    ST = torch.empty((B, Hv, D, D), device=dev)
    common = (D, D, chunk, L.GATE_DECAY_VEC, 0, L.FORM_CHUNK, L.BF16)
    n_saved = lib.gdn_saved_bytes(B, T, Hk, Hv, *common)
    saved = torch.empty(max(n_saved, 1), device=dev, dtype=torch.uint8)
    n_fws = lib.gdn_fwd_workspace_bytes(B, fwd_ws_T or T, Hk, Hv, *common, 1)
    fws = torch.empty(max(n_fws, 1), device=dev, dtype=torch.uint8)
    L.check(lib.gdn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), S0.data_ptr(),
                        None, y.data_ptr(), ST.data_ptr(), saved.data_ptr(), n_saved, fws.data_ptr(), n_fws,
                        B, T, Hk, Hv, D, D, chunk, L.BF16, L.BF16, L.GATE_DECAY_VEC, L.FORM_CHUNK, None))
    outs = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(g),
            torch.empty_like(beta), torch.empty_like(S0)]
    n_bws = lib.gdn_bwd_workspace_bytes(B, bwd_ws_T or T, Hk, Hv, *common)
    bws = torch.empty(max(n_bws, 1), device=dev, dtype=torch.uint8)
    L.check(lib.gdn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), S0.data_ptr(),
                        None, saved.data_ptr(), n_saved, dy.data_ptr(), dS_T.data_ptr(),
                        *(o.data_ptr() for o in outs), bws.data_ptr(), n_bws, B, T, Hk, Hv, D, D, chunk,
                        L.BF16, L.BF16, L.BF16, L.GATE_DECAY_VEC, L.FORM_CHUNK, None))
    torch.cuda.synchronize()
    return [x.float().cpu().numpy() for x in (y, ST, *outs)]


def test_decays_checkpointed_in_groups_of_windows(dev):
    """Per-channel decays with 2% zeros, chunk = 100 (windows of 128 tokens) over T = 700, through the C ABI: the
    backward in groups of one and of three windows (forced by small workspaces, each group with its own d/d(decay)
    buffers) gives the same results as one group, and that matches the fp64 oracle."""
    d = _inputs(2, 700, 2, 4, seed=850, log_decay=(0.0, 6.0))
    rng = np.random.default_rng(851)
    d["decay"] = np.where(rng.random(d["decay"].shape) < 0.02, 0.0, d["decay"]).astype(np.float32)
    print("vector decays bf16 T=700 chunk=100, groups of windows", flush=True)
    one = _abi_vg(d, dev, 100)
    for fT, bT in ((128, 128), (256, 384)):
        print(f"  forward groups of {fT} tokens, backward groups of {bT}", flush=True)
        got = _abi_vg(d, dev, 100, fwd_ws_T=fT, bwd_ws_T=bT)
        for n, a, w in zip(NAMES, got, one):
            assert nerr(a, w) <= 1e-6, (fT, bT, n, nerr(a, w))
    _check(one, _oracle(d, 100), True, True, "decays ckpt groups")
