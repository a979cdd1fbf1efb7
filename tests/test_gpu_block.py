"""GPU parity of one whole GDN block (qwen3_5.GatedDeltaNet: projections with LoRA adapters, conv + SiLU, q/k
L2 norm, gates, recurrence, gated RMSNorm, out-projection) forward and backward, against the float64 block oracle
(oracle/gdn_block_oracle.py, pinned against torch autograd on the CPU).

Shapes cover the recurrent form (Dk = Dv = 32) and the chunked form (Dk = Dv = 128).  fp32: normalised max error
<= 1e-4 on the output and every gradient; bf16 weights and activations: <= 3e-2 (every stage rounds its output
to bf16, roughly 4e-3 relative each, and the gradients pass through five such stages).
"""

import numpy as np
import pytest
import torch

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


def build_block(P, h, Hk, Hv, Dk, Dv, dev, dtype, rank, scale):
    import qwen3_5 as Q
    args = Q.ModelArgs(hidden_size=h, linear_num_key_heads=Hk, linear_num_value_heads=Hv,
                       linear_key_head_dim=Dk, linear_value_head_dim=Dv, linear_conv_kernel_dim=4)
    blk = Q.GatedDeltaNet(args)
    t = lambda x: torch.tensor(np.asarray(x, np.float32))
    with torch.no_grad():
        for n in ("qkv", "z", "b", "a"):
            getattr(blk, "in_proj_" + n).weight.copy_(t(P["W_" + n]))
        blk.out_proj.weight.copy_(t(P["W_out"]))
        blk.conv1d.weight.copy_(t(P["conv_w"])[:, None, :])
        blk.A_log.copy_(t(P["A_log"]))
        blk.dt_bias.copy_(t(P["dt_bias"]))
        blk.norm.weight.copy_(t(P["norm_w"]))
    if rank:
        Q.freeze(blk)
        for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj"):
            lora = Q.LoRALinear(getattr(blk, n), rank, scale)
            key = n.replace("in_proj_", "").replace("out_proj", "out")
            with torch.no_grad():
                lora.lora_a.copy_(t(P["A_" + key]))
                lora.lora_b.copy_(t(P["B_" + key]))
            setattr(blk, n, lora)
    blk = blk.to(device=dev, dtype=dtype)
    blk.train()
    return blk


def run_block(P, x, dout, dims, dev, dtype, rank, scale):
    h, Hk, Hv, Dk, Dv = dims
    blk = build_block(P, h, Hk, Hv, Dk, Dv, dev, dtype, rank, scale)
    tx = torch.tensor(x, device=dev, dtype=dtype, requires_grad=True)
    out = blk(tx)
    params = dict(blk.named_parameters())
    names = [n for n, p in params.items() if p.requires_grad]
    grads = torch.autograd.grad(out, [tx] + [params[n] for n in names],
                                torch.tensor(dout, device=dev, dtype=dtype))
    torch.cuda.synchronize()
    got = {"x": grads[0]}
    got.update(dict(zip(names, grads[1:])))
    return out.detach().float().cpu().numpy(), {k: v.detach().float().cpu().numpy() for k, v in got.items()}


def lora_key(name):
    # "in_proj_qkv.lora_a" -> "A_qkv"; "out_proj.lora_b" -> "B_out"
    mod, leaf = name.split(".")
    key = mod.replace("in_proj_", "").replace("out_proj", "out")
    return ("A_" if leaf == "lora_a" else "B_") + key


@pytest.mark.parametrize("D,T,B", [(32, 100, 2), (128, 130, 1)])
def test_block_fp32_full_gradients(dev, D, T, B):
    """All parameters trainable (no adapters): every gradient of the block."""
    h, Hk, Hv = 48, 2, 4
    P = BO.make_block_params(h, Hk, Hv, D, D, rank=0, seed=D, w_std=0.2)
    r = np.random.default_rng(D + 1)
    x, dout = r.standard_normal((B, T, h)).astype(np.float32), r.standard_normal((B, T, h)).astype(np.float32)
    print(f"block fp32 D={D} T={T} B={B}", flush=True)
    out, got = run_block(P, x, dout, (h, Hk, Hv, D, D), dev, torch.float32, 0, 0.0)
    want_out, want = BO.block_vjp(x, P, dout, Hk, Hv, D, D)
    assert nerr(out, want_out) <= 1e-4
    pairs = {"x": "x", "conv1d.weight": "conv_w", "A_log": "A_log", "dt_bias": "dt_bias", "norm.weight": "norm_w",
             "in_proj_qkv.weight": "W_qkv", "in_proj_z.weight": "W_z", "in_proj_b.weight": "W_b",
             "in_proj_a.weight": "W_a", "out_proj.weight": "W_out"}
    for mine, theirs in pairs.items():
        g = got[mine].reshape(want[theirs].shape)
        assert nerr(g, want[theirs]) <= 1e-4, (mine, nerr(g, want[theirs]))


@pytest.mark.parametrize("D,T,B", [(32, 70, 1), (128, 200, 2)])
def test_block_lora_fp32(dev, D, T, B):
    """LoRA adapters on the five projections with random B: gradients of x and of every A and B."""
    h, Hk, Hv, rank, scale = 40, 2, 4, 4, 2.0
    P = BO.make_block_params(h, Hk, Hv, D, D, rank=rank, lora_scale=scale, b_std=0.05, seed=7, w_std=0.2)
    r = np.random.default_rng(8)
    x, dout = r.standard_normal((B, T, h)).astype(np.float32), r.standard_normal((B, T, h)).astype(np.float32)
    print(f"block lora fp32 D={D} T={T}", flush=True)
    out, got = run_block(P, x, dout, (h, Hk, Hv, D, D), dev, torch.float32, rank, scale)
    want_out, want = BO.block_vjp(x, P, dout, Hk, Hv, D, D)
    assert nerr(out, want_out) <= 1e-4
    assert set(got) == {"x"} | {f"{m}.lora_{ab}" for m in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a",
                                                             "out_proj") for ab in "ab"}
    for name, g in got.items():
        key = "x" if name == "x" else lora_key(name)
        assert nerr(g, want[key]) <= 1e-4, (name, nerr(g, want[key]))


def test_block_lora_init_gives_zero_a_gradient(dev):
    """LoRA B = 0 at initialisation: grad(A) is exactly zero on the GPU too, grad(B) is not."""
    h, Hk, Hv, D, rank = 40, 2, 4, 128, 4
    P = BO.make_block_params(h, Hk, Hv, D, D, rank=rank, b_std=0.0, seed=9, w_std=0.2)
    r = np.random.default_rng(10)
    x, dout = r.standard_normal((1, 64, h)).astype(np.float32), r.standard_normal((1, 64, h)).astype(np.float32)
    _, got = run_block(P, x, dout, (h, Hk, Hv, D, D), dev, torch.float32, rank, 2.0)
    for name, g in got.items():
        if name.endswith("lora_a"):
            assert not np.any(g), name
        elif name.endswith("lora_b"):
            assert np.abs(g).max() > 0, name


def test_block_lora_bf16(dev):
    """bf16 weights and activations at the block's real head layout (Dk = Dv = 128, 2:1 GQA), small hidden size."""
    h, Hk, Hv, D, rank, scale, T = 256, 4, 8, 128, 8, 2.0, 192
    P = BO.make_block_params(h, Hk, Hv, D, D, rank=rank, lora_scale=scale, b_std=0.05, seed=11, w_std=0.05)
    # the module holds bf16 weights: give the oracle the same rounded values
    P = {k: (torch.tensor(v).bfloat16().float().numpy() if isinstance(v, np.ndarray) else v) for k, v in P.items()}
    r = np.random.default_rng(12)
    bf = lambda a: torch.tensor(a).bfloat16().float().numpy()
    x, dout = bf(r.standard_normal((2, T, h))), bf(r.standard_normal((2, T, h)))
    out, got = run_block(P, x, dout, (h, Hk, Hv, D, D), dev, torch.bfloat16, rank, scale)
    want_out, want = BO.block_vjp(x, P, dout, Hk, Hv, D, D)
    assert nerr(out, want_out) <= 3e-2, nerr(out, want_out)
    for name, g in got.items():
        key = "x" if name == "x" else lora_key(name)
        assert nerr(g, want[key]) <= 3e-2, (name, nerr(g, want[key]))


def test_block_config4_full_size(dev, monkeypatch):
    """The block configuration itself: B=2, T=8192, hidden 2048, Hk=16, Hv=32, D=128, bf16 weights and activations,
    LoRA rank 16 on the five projections (A ~ N(0, 0.02), B = 0), gradients to the adapters and the input.  At this
    size: grad(A) is exactly zero and every gradient finite (B = 0); the chunked and the recurrent form of the
    recurrence (each pinned against the oracle above and in the recurrence tests) agree on the output, dx and every
    grad(B); and the output's first 256 tokens equal the block run on those tokens alone (causality), which the
    float64 block oracle pins."""
    h, Hk, Hv, D, rank, scale, B, T = 2048, 16, 32, 128, 16, 2.0, 2, 8192
    P = BO.make_block_params(h, Hk, Hv, D, D, rank=rank, lora_scale=scale, b_std=0.0, seed=21, w_std=0.02)
    P = {k: (torch.tensor(v).bfloat16().float().numpy() if isinstance(v, np.ndarray) else v) for k, v in P.items()}
    r = np.random.default_rng(22)
    bf = lambda a: torch.tensor(a).bfloat16().float().numpy()
    x = bf(r.standard_normal((B, T, h)).astype(np.float32))
    dout = bf(r.standard_normal((B, T, h)).astype(np.float32))
    dims = (h, Hk, Hv, D, D)
    print("block B=2 T=8192 hidden 2048 bf16 LoRA 16: chunked form", flush=True)
    out_c, g_c = run_block(P, x, dout, dims, dev, torch.bfloat16, rank, scale)
    for name, g in g_c.items():
        assert np.all(np.isfinite(g)), name
        if name.endswith("lora_a"):
            assert not np.any(g), name
    assert np.all(np.isfinite(out_c))
    monkeypatch.setenv("GDN_FORM", "recurrent")
    print("  recurrent form", flush=True)
    out_r, g_r = run_block(P, x, dout, dims, dev, torch.bfloat16, rank, scale)
    monkeypatch.delenv("GDN_FORM")
    errs = {"out": nerr(out_c, out_r)}
    errs.update({n: nerr(g_c[n], g_r[n]) for n in g_c if not n.endswith("lora_a")})
    print("  chunked vs recurrent", {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= 3e-2, (n, e)
    print("  the first 256 tokens alone, and the float64 block oracle", flush=True)
    out_p, _ = run_block(P, x[:, :256], dout[:, :256], dims, dev, torch.bfloat16, rank, scale)
    want, _ = BO.block_forward(x[:, :256], P, Hk, Hv, D, D)
    e_pre, e_orc = nerr(out_c[:, :256], out_p), nerr(out_p, want)
    print(f"  prefix {e_pre:.1e}, oracle {e_orc:.1e}", flush=True)
    assert e_pre <= 1e-2 and e_orc <= 3e-2
