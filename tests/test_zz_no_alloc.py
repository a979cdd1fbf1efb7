"""gdn_fwd_noalloc (the forward-only call with no allocation and no workspace) against the existing entry point,
gdn_fwd with saved = NULL and a workspace, through the C ABI: two calls in a row, the second with a smaller input.

Both run the same kernels, group by group from carried fp32 states, so the outputs are equal bit for bit whatever
the group sizes (the fixed scratch holds fewer chunks per group than the workspace gdn_fwd_workspace_bytes sizes).
The recurrent form (a mask) needs no scratch and is checked the same way.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import gdn_lib
    gdn_lib.load()
    return torch.device("cuda:0")


def _inputs(B, T, Hk, Hv, D, dtype, dev, seed, vector=False):
    """q, k L2-normalised (q times D^-1/2), v and S0 normal; the gate a log decay -U(0, 1) per value head, or with
    vector=True a decay exp(-U(0, 1.5)) per key channel [B, T, Hv, D]."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    n = lambda *s: torch.randn(*s, device=dev, generator=g)
    q = torch.nn.functional.normalize(n(B, T, Hk, D), dim=-1) * D ** -0.5
    k = torch.nn.functional.normalize(n(B, T, Hk, D), dim=-1)
    v = n(B, T, Hv, D).to(dtype)
    gate = (torch.exp(-1.5 * torch.rand(B, T, Hv, D, device=dev, generator=g)) if vector
            else -torch.rand(B, T, Hv, device=dev, generator=g))
    return dict(q=q.to(dtype), k=k.to(dtype), v=v, g=gate, beta=torch.rand(B, T, Hv, device=dev, generator=g),
                S0=n(B, Hv, D, D) * 0.02)


def _run(x, dev, noalloc, mask=None, form=None):
    import gdn_lib as L
    lib = L.load()
    B, T, Hk, D = x["q"].shape
    Hv = x["v"].shape[2]
    code = L.DTYPE_CODE[x["q"].dtype]
    gate = L.GATE_DECAY_VEC if x["g"].dim() == 4 else L.GATE_LOG
    y = torch.full((B, T, Hv, D), float("nan"), device=dev, dtype=x["q"].dtype)
    S = torch.full((B, Hv, D, D), float("nan"), device=dev)
    ptrs = [x[n].data_ptr() for n in ("q", "k", "v", "g", "beta", "S0")]
    m = None if mask is None else mask.data_ptr()
    form = L.FORM_AUTO if form is None else form
    if noalloc:
        rc = lib.gdn_fwd_noalloc(*ptrs, m, y.data_ptr(), S.data_ptr(), B, T, Hk, Hv, D, D, code, code, gate,
                                 form, None)
    else:
        n_ws = lib.gdn_fwd_workspace_bytes(B, T, Hk, Hv, D, D, 64, gate, int(mask is not None), form,
                                           code, 0)
        ws = torch.empty(max(n_ws, 1), device=dev, dtype=torch.uint8)
        rc = lib.gdn_fwd(*ptrs, m, y.data_ptr(), S.data_ptr(), None, 0, ws.data_ptr(), n_ws, B, T, Hk, Hv, D, D, 64,
                         code, code, gate, form, None)
    L.check(rc)
    torch.cuda.synchronize()
    return y, S


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_forward_matches_gdn_fwd_twice(dev, dtype):
    # first call: 4 x 32 heads over 1000 tokens (several groups in the fixed scratch); second: a smaller input
    for B, T, seed in ((4, 1000, 1), (2, 300, 2)):
        print(f"gdn_fwd_noalloc {dtype} B={B} T={T} Hk=16 Hv=32 D=128", flush=True)
        x = _inputs(B, T, 16, 32, 128, dtype, dev, seed)
        y0, S0 = _run(x, dev, noalloc=False)
        y1, S1 = _run(x, dev, noalloc=True)
        assert torch.isfinite(y1.float()).all() and torch.isfinite(S1).all()
        assert torch.equal(y0, y1) and torch.equal(S0, S1)


def test_noalloc_vector_gates_on_the_chunked_form_twice(dev):
    """Per-channel gates with bf16 inputs run the chunked form's vector-gate kernels, whose per-chunk decay tiles
    take their share of the fixed scratch: equal to gdn_fwd bit for bit on two calls, the second smaller."""
    import gdn_lib as L
    lib = L.load()
    assert lib.gdn_select_form(32, 128, 128, 0, L.GATE_DECAY_VEC, L.FORM_AUTO, L.BF16) == L.FORM_CHUNK
    for B, T, seed in ((4, 700, 4), (1, 130, 5)):
        print(f"gdn_fwd_noalloc bf16 vector gates B={B} T={T} Hk=16 Hv=32 D=128", flush=True)
        x = _inputs(B, T, 16, 32, 128, torch.bfloat16, dev, seed, vector=True)
        y0, S0 = _run(x, dev, noalloc=False)
        y1, S1 = _run(x, dev, noalloc=True)
        assert torch.isfinite(y1.float()).all() and torch.isfinite(S1).all()
        assert torch.equal(y0, y1) and torch.equal(S0, S1)


def test_noalloc_recurrent_form_and_limits(dev):
    """A masked call runs the recurrent form (no scratch), equal to gdn_fwd's recurrent form.  The refusals (a masked
    call that asks for the chunked form, a one-chunk group beyond the fixed scratch) are host-side checks, tested on
    the CPU (tests/test_abi_cpu.py)."""
    import gdn_lib as L
    x = _inputs(2, 70, 2, 4, 128, torch.float32, dev, 3)
    mask = torch.ones(2, 70, dtype=torch.uint8, device=dev)
    mask[:, 50:] = 0
    for _ in range(2):
        y0, S0 = _run(x, dev, noalloc=False, mask=mask, form=L.FORM_RECURRENT)
        y1, S1 = _run(x, dev, noalloc=True, mask=mask)
        assert torch.equal(y0, y1) and torch.equal(S0, S1)


def test_noalloc_forward_under_graph_capture(dev):
    """gdn_fwd_noalloc recorded into a HIP graph (torch.cuda.graph capture) after one eager call on the device: each
    replay, over new contents of the captured inputs and with eager work between replays, equals gdn_fwd."""
    import gdn_lib as L
    lib = L.load()
    B, T, Hk, Hv, D = 2, 300, 16, 32, 128
    x = _inputs(B, T, Hk, Hv, D, torch.bfloat16, dev, 11)
    _run(x, dev, noalloc=True)   # the first call on the device looks up the scratch address
    code = L.DTYPE_CODE[torch.bfloat16]
    y = torch.empty((B, T, Hv, D), device=dev, dtype=torch.bfloat16)
    S = torch.empty((B, Hv, D, D), device=dev)
    ptrs = [x[n].data_ptr() for n in ("q", "k", "v", "g", "beta", "S0")]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.gdn_fwd_noalloc(*ptrs, None, y.data_ptr(), S.data_ptr(), B, T, Hk, Hv, D, D, code, code,
                                 L.GATE_LOG, L.FORM_AUTO, L.stream_handle(dev))
    L.check(rc)
    for rep in range(3):
        print(f"graph replay {rep}", flush=True)
        new = _inputs(B, T, Hk, Hv, D, torch.bfloat16, dev, 20 + rep)
        for n in new:
            x[n].copy_(new[n])
        y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        y0, S0 = _run(x, dev, noalloc=False)
        assert torch.equal(y0, y) and torch.equal(S0, S)
