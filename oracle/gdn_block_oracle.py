"""CPU oracle for one whole GDN block, forward and VJP, with LoRA on the projections.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import this
module, and only as the checker.  The product path never imports it.

The forward follows the order of one block in ``engine/src/gdn_layer.c:18-58`` (``engine/include/gdn_layer.h:
31-43``), over a whole sequence instead of one token:

    qkv = W_qkv x;  z = W_z x;  b = W_b x;  a = W_a x
    c = conv_silu(qkv)                         (causal depthwise, K taps)
    q, k, v = split(c);  q, k L2-normalised per head (q scaled by Dk^-1/2)
    decay, beta = gates(a, b, A_log, dt_bias)
    y = delta-rule recurrence from S0 = 0
    o = rmsnorm(y_h) * w * silu(z_h) per value head
    out = W_out o

Each linear W is ``W + scale * B A`` when it carries a LoRA adapter (A [r, in], B [out, r]).  The VJP composes
the pieces' backward functions of ``oracle/gdn_oracle.py`` in reverse order; all arithmetic is float64.

Pinned by ``tests/test_oracle.py::test_block_vjp_matches_torch_autograd`` against torch float64 autograd of an
independent torch statement of the same block (``tests/naive_torch.py::gdn_block``).
"""

from __future__ import annotations

import numpy as np

from . import gdn_oracle as O

PROJ = ("qkv", "z", "b", "a", "out")


def effective(P: dict, name: str) -> np.ndarray:
    """W + scale * B A for projection ``name`` (no adapter: W)."""
    W = np.asarray(P["W_" + name], np.float64)
    if ("A_" + name) in P:
        W = W + P["lora_scale"] * np.asarray(P["B_" + name], np.float64) @ np.asarray(P["A_" + name], np.float64)
    return W


def block_forward(x, P, Hk, Hv, Dk, Dv, eps=1e-6, chunk=64):
    """x [B,T,h] -> (out [B,T,h], cache of the intermediates the VJP reads)."""
    x = np.asarray(x, np.float64)
    B, T, _ = x.shape
    W = {n: effective(P, n) for n in PROJ}
    qkv, z, b, a = (x @ W[n].T for n in ("qkv", "z", "b", "a"))
    conv_w = np.asarray(P["conv_w"], np.float64)
    c, _ = O.conv_silu(qkv, conv_w)
    kd = Hk * Dk
    q = c[..., :kd].reshape(B, T, Hk, Dk)
    k = c[..., kd:2 * kd].reshape(B, T, Hk, Dk)
    v = c[..., 2 * kd:].reshape(B, T, Hv, Dv)
    qn, kn = O.l2norm(q, eps, Dk ** -0.5), O.l2norm(k, eps, 1.0)
    A_log, dt = np.asarray(P["A_log"], np.float64), np.asarray(P["dt_bias"], np.float64)
    decay, beta = O.gates(a, b, A_log, dt)
    S0 = np.zeros((B, Hv, Dv, Dk))
    y, S, bounds = O.forward(qn, kn, v, decay, beta, S0, None, chunk)
    zh = z.reshape(B, T, Hv, Dv)
    nw = np.asarray(P["norm_w"], np.float64)
    # float64 throughout (O.rmsnorm rounds the rms to float32 as engine/src/ops.c does)
    o = (y / np.sqrt((y * y).mean(-1, keepdims=True) + eps) * nw * O.silu(zh)).reshape(B, T, Hv * Dv)
    out = o @ W["out"].T
    cache = dict(x=x, W=W, qkv=qkv, z=zh, b=b, a=a, q=q, k=k, v=v, qn=qn, kn=kn, decay=decay, beta=beta,
                 S0=S0, bounds=bounds, y=y, o=o, conv_w=conv_w, A_log=A_log, dt=dt, nw=nw)
    return out, cache


def block_vjp(x, P, dout, Hk, Hv, Dk, Dv, eps=1e-6, chunk=64):
    """Returns (out, grads) with grads a dict: 'x', 'W_<p>' (of the effective weight), 'A_<p>' / 'B_<p>' for
    adapters, 'conv_w', 'A_log', 'dt_bias', 'norm_w'."""
    out, C = block_forward(x, P, Hk, Hv, Dk, Dv, eps, chunk)
    dout = np.asarray(dout, np.float64)
    B, T, _ = dout.shape
    W = C["W"]
    g = {}
    g["W_out"] = dout.reshape(-1, dout.shape[-1]).T @ C["o"].reshape(-1, C["o"].shape[-1])
    do = (dout @ W["out"]).reshape(B, T, Hv, Dv)
    dy, dz, g["norm_w"] = O.gated_rmsnorm_bwd(C["y"], C["z"], C["nw"], do, eps)
    dq, dk, dv, ddecay, dbeta, _ = O.backward(C["qn"], C["kn"], C["v"], C["decay"], C["beta"], C["S0"], None,
                                              C["bounds"], dy, np.zeros_like(C["S0"]), chunk)
    dq = O.l2norm_bwd(C["q"], dq, eps, Dk ** -0.5)
    dk = O.l2norm_bwd(C["k"], dk, eps, 1.0)
    da, db, g["A_log"], g["dt_bias"] = O.gates_bwd(C["a"], C["b"], C["A_log"], C["dt"], ddecay, dbeta)
    dc = np.concatenate([dq.reshape(B, T, -1), dk.reshape(B, T, -1), dv.reshape(B, T, -1)], -1)
    dqkv, g["conv_w"] = O.conv_silu_bwd(C["qkv"], C["conv_w"], dc)
    dproj = {"qkv": dqkv, "z": dz.reshape(B, T, -1), "b": db, "a": da}
    x2 = C["x"].reshape(-1, C["x"].shape[-1])
    dx = np.zeros_like(C["x"])
    for n, d in dproj.items():
        dx += d @ W[n]
        g["W_" + n] = d.reshape(-1, d.shape[-1]).T @ x2
    g["x"] = dx
    s = P.get("lora_scale", 0.0)
    for n in PROJ:
        if ("A_" + n) in P:
            A, Bm = np.asarray(P["A_" + n], np.float64), np.asarray(P["B_" + n], np.float64)
            g["A_" + n] = s * Bm.T @ g["W_" + n]
            g["B_" + n] = s * g["W_" + n] @ A.T
    return out, g


def make_block_params(h, Hk, Hv, Dk, Dv, K=4, rank=0, lora_scale=2.0, b_std=0.0, seed=0, w_std=0.02):
    """Random block weights: projections ~ N(0, w_std); conv ~ N(0, 0.5/sqrt(K)); A_log ~ log U(1, 16);
    dt_bias 0; norm weight 1 + N(0, 0.1).  With rank > 0, LoRA A ~ N(0, 0.02) and B ~ N(0, b_std) (0: B = 0)
    on the in/out projections."""
    r = np.random.default_rng(seed)
    conv_dim = 2 * Hk * Dk + Hv * Dv
    P = {"W_qkv": r.standard_normal((conv_dim, h)) * w_std, "W_z": r.standard_normal((Hv * Dv, h)) * w_std,
         "W_b": r.standard_normal((Hv, h)) * w_std, "W_a": r.standard_normal((Hv, h)) * w_std,
         "W_out": r.standard_normal((h, Hv * Dv)) * w_std,
         "conv_w": r.standard_normal((conv_dim, K)) * (0.5 / np.sqrt(K)),
         "A_log": np.log(r.uniform(1.0, 16.0, Hv)), "dt_bias": np.zeros(Hv),
         "norm_w": 1.0 + 0.1 * r.standard_normal(Dv)}
    if rank:
        P["lora_scale"] = lora_scale
        for n in PROJ:
            W = P["W_" + n]
            P["A_" + n] = r.standard_normal((rank, W.shape[1])) * 0.02
            P["B_" + n] = r.standard_normal((W.shape[0], rank)) * b_std
    return {k: (v.astype(np.float32) if isinstance(v, np.ndarray) else v) for k, v in P.items()}
