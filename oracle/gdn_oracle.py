"""CPU oracle for the Gated DeltaNet forward + VJP path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import this
module, and only as the checker.  The product path (``moe-stream-mac_amd/``) never imports it and has no
CPU fallback.

This is a NumPy restatement of the reference's arithmetic, one function per reference function:

* ``decay_view``        <- ``tools/gdn_vjp.py:174-179``  (``_decay``)
* ``step_parts``        <- ``tools/gdn_vjp.py:238-256``  (``_step_parts``; restates mlx-lm
                           ``_gated_delta_step_ops``: ``y`` always reads the candidate state)
* ``repeat_heads``      <- ``tools/gdn_vjp.py:259-263``
* ``collapse_heads``    <- ``tools/gdn_vjp.py:266-270``
* ``forward``           <- ``tools/gdn_vjp.py:182-235``  (``_run_chunk``, ``_copy_boundary``, ``_forward``)
* ``chunk_vjp``         <- ``tools/gdn_vjp.py:273-320``  (``_chunk_vjp``, the hand-derived adjoint)
* ``backward``          <- ``tools/gdn_vjp.py:426-474``  (``_backward``, impl="staged")
* ``gated_delta_chunked`` / ``gated_delta_chunked_vjp``
                        <- ``tools/gdn_vjp.py:503-528`` (public entry; state defaults to fp32 zeros)
* ``gated_delta_ops_checkpointed`` <- ``tools/gdn_checkpoint.py:53-95`` (same forward, chunked by ``chunk``)
* ``compute_g`` / ``gates``  <- ``engine/include/gdn.h:20-25``, ``engine/src/gdn.c:51-61``
                                (mlx-lm ``compute_g`` returns the multiplicative decay)
* ``l2norm``            <- ``engine/include/gdn.h:17-18``, ``engine/src/gdn.c:40-49``
* ``conv_silu``         <- ``engine/include/gdn.h:7-15``, ``engine/src/gdn.c:15-38`` (whole sequence)
* ``rmsnorm`` / ``silu_mul`` <- ``engine/include/ops.h:7-11``, ``engine/src/ops.c``
* ``gated_rmsnorm``     <- ``engine/src/gdn_layer.c:47-55`` (rmsnorm(y)*silu(z) per value head)

The backward functions of the elementwise pieces (``*_bwd``) are derived here from those forward specs;
the reference has no backward for them (its training path relies on MLX autodiff).

How each function is pinned (the checks live in ``tests/test_oracle.py``):

* forward / step_parts: the reference's MLX-generated fixture ``engine/tests/fixtures/gdn_recurrence.bin``
  and the reference C ``gdn_recurrent_step`` compiled from source into ``oracle/_ref``.
* chunk_vjp / backward: torch float64 autograd of an independently written naive recurrence
  (mask, vector gate, GQA, nonzero S0, chunk sizes), float64 central finite differences, and
  closed-form special cases (T=1, beta=0, decay=0).
* gates / l2norm / conv_silu / rmsnorm / silu_mul: the reference fixtures ``gdn_gates.bin``,
  ``gdn_l2norm.bin``, ``gdn_conv.bin``, ``ops_rmsnorm.bin``, ``ops_silu_mul.bin`` and the reference C.
* the ``*_bwd`` functions: torch float64 autograd and finite differences of the forward spec.

Layouts follow the reference: q, k ``[B,T,Hk,Dk]``; v ``[B,T,Hv,Dv]``; g ``[B,T,Hv]`` (scalar decay) or
``[B,T,Hv,Dk]`` (vector decay along the key axis); beta ``[B,T,Hv]``; state ``[B,Hv,Dv,Dk]``;
mask ``[B,T]`` bool (True keeps the candidate state).
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np

DEFAULT_CHUNK = 64


# --------------------------------------------------------------------------------------------------------
# Core recurrence (tools/gdn_vjp.py)
# --------------------------------------------------------------------------------------------------------

def decay_view(g_t: np.ndarray) -> np.ndarray:
    """Per-step decay broadcast to the state shape (tools/gdn_vjp.py:174-179).

    ``g_t`` is one time step: ``[B,Hv]`` (scalar gate) or ``[B,Hv,Dk]`` (vector gate along the key axis).
    """
    if g_t.ndim == 2:
        return g_t[..., None, None]
    if g_t.ndim == 3:
        return g_t[..., None, :]
    raise ValueError(f"Unsupported gating shape {g_t.shape}")


def step_parts(q, k, v, g, beta, state, mask):
    """One step (tools/gdn_vjp.py:238-256).  Returns (candidate, next_state, a, residual, delta).

    a = state*decay; residual = v - a@k; delta = residual*beta; candidate = a + k (x) delta;
    next_state = mask ? candidate : state.
    """
    a = state * decay_view(g)
    residual = v - (a * k[..., None, :]).sum(axis=-1)
    delta = residual * beta[..., None]
    candidate = a + k[..., None, :] * delta[..., None]
    if mask is None:
        next_state = candidate
    else:
        next_state = np.where(mask[:, None, None, None], candidate, state)
    return candidate, next_state, a, residual, delta


def repeat_heads(q, k, value_heads):
    """GQA repeat: value head h reads key head h // (Hv/Hk) (tools/gdn_vjp.py:259-263, :217-222)."""
    repeat = value_heads // q.shape[2]
    if repeat > 1:
        return np.repeat(q, repeat, axis=-2), np.repeat(k, repeat, axis=-2)
    return q, k


def collapse_heads(gradient, key_heads, repeat):
    """Sum dq/dk over the value heads that share a key head (tools/gdn_vjp.py:266-270)."""
    if repeat == 1:
        return gradient
    batch, timesteps, _, dim = gradient.shape
    return gradient.reshape(batch, timesteps, key_heads, repeat, dim).sum(axis=3)


def _run_chunk(q, k, v, g, beta, state, mask):
    """Per-step loop over one chunk (tools/gdn_vjp.py:182-198); y reads the candidate state."""
    outputs = []
    for t in range(q.shape[1]):
        step_mask = None if mask is None else mask[:, t]
        candidate, state, _, _, _ = step_parts(
            q[:, t], k[:, t], v[:, t], g[:, t], beta[:, t], state, step_mask)
        outputs.append((candidate * q[:, t][..., None, :]).sum(axis=-1))
    if not outputs:
        return np.zeros(v.shape[:1] + (0,) + v.shape[2:], dtype=state.dtype), state
    return np.stack(outputs, axis=1), state


def forward(q, k, v, g, beta, state, mask, chunk):
    """Chunked forward keeping chunk-boundary states (tools/gdn_vjp.py:205-235).

    Returns (y, final_state, boundaries) with boundaries ``[ceil(T/chunk)+1, B,Hv,Dv,Dk]``.
    """
    batch, timesteps, key_heads, _ = q.shape
    value_heads = v.shape[2]
    repeat = value_heads // key_heads
    if repeat * key_heads != value_heads:
        raise ValueError("q/k head count must divide the value head count")
    q, k = repeat_heads(q, k, value_heads)
    outputs = []
    boundaries = [state.copy()]
    for start in range(0, timesteps, chunk):
        end = min(start + chunk, timesteps)
        chunk_mask = None if mask is None else mask[:, start:end]
        output, state = _run_chunk(q[:, start:end], k[:, start:end], v[:, start:end],
                                   g[:, start:end], beta[:, start:end], state, chunk_mask)
        outputs.append(output)
        boundaries.append(state.copy())
    y = np.concatenate(outputs, axis=1) if outputs else np.zeros(v.shape, dtype=state.dtype)
    return y, state, np.stack(boundaries, axis=0)


def chunk_vjp(q, k, v, g, beta, initial_state, mask, dy, dstate):
    """Reverse pass over one chunk (tools/gdn_vjp.py:273-320).

    q, k already repeated to the value heads.  Returns (dq, dk, dv, dg, dbeta, dstate_in); dq/dk are per
    value head.  Adjoint equations (tools/gdn_vjp.py:8-21):
      dS~ = dy (x) q + m dS;  dq = S~^T dy;  u = dS~ k;  dbeta = sum_v u r;  dv = e = beta u;
      dA = dS~ - e (x) k;  dk = sum_v (dS~ delta - A e);  dS_prev = dA decay + (1-m) dS;
      dg = sum_{v,k} dA S_prev (scalar gate) or sum_v dA S_prev (vector gate).
    """
    states = [initial_state]
    for t in range(q.shape[1]):
        step_mask = None if mask is None else mask[:, t]
        states.append(step_parts(q[:, t], k[:, t], v[:, t], g[:, t], beta[:, t], states[-1],
                                 step_mask)[1])
    dq, dk, dv, dg, dbeta = [], [], [], [], []
    for t in range(q.shape[1] - 1, -1, -1):
        step_mask = None if mask is None else mask[:, t]
        selector = 1.0 if step_mask is None else step_mask[:, None, None, None].astype(dstate.dtype)
        candidate, _, a, residual, delta = step_parts(
            q[:, t], k[:, t], v[:, t], g[:, t], beta[:, t], states[t], step_mask)
        ds_candidate = dy[:, t, ..., None] * q[:, t, ..., None, :]
        ds_candidate = ds_candidate + selector * dstate
        dq.append((dy[:, t, ..., None] * candidate).sum(axis=-2))
        ddelta = (ds_candidate * k[:, t, ..., None, :]).sum(axis=-1)
        dbeta.append((ddelta * residual).sum(axis=-1))
        e = ddelta * beta[:, t, ..., None]
        dv.append(e)
        dk.append((ds_candidate * delta[..., None] - a * e[..., None]).sum(axis=-2))
        da = ds_candidate - e[..., None] * k[:, t, ..., None, :]
        if g.ndim == 3:
            dg.append((da * states[t]).sum(axis=(-2, -1)))
        else:
            dg.append((da * states[t]).sum(axis=-2))
        dstate = da * decay_view(g[:, t]) + (1.0 - selector) * dstate
    return (np.stack(dq[::-1], axis=1), np.stack(dk[::-1], axis=1), np.stack(dv[::-1], axis=1),
            np.stack(dg[::-1], axis=1), np.stack(dbeta[::-1], axis=1), dstate)


def backward(q, k, v, g, beta, state, mask, boundaries, dy, dstate, chunk):
    """Reverse chunk loop, impl="staged" (tools/gdn_vjp.py:426-474).

    Returns (dq, dk, dv, dg, dbeta, dstate0) with dq/dk collapsed to the key heads.
    """
    batch, timesteps, key_heads, key_dim = q.shape
    value_heads = v.shape[2]
    repeat = value_heads // key_heads
    q, k = repeat_heads(q, k, value_heads)
    grads = {n: [] for n in ("q", "k", "v", "g", "b")}
    starts = list(range(0, timesteps, chunk))
    for index in range(len(starts) - 1, -1, -1):
        start = starts[index]
        end = min(start + chunk, timesteps)
        chunk_mask = None if mask is None else mask[:, start:end]
        dq, dk, dv, dg, dbeta, dstate = chunk_vjp(
            q[:, start:end], k[:, start:end], v[:, start:end], g[:, start:end],
            beta[:, start:end], boundaries[index], chunk_mask, dy[:, start:end], dstate)
        for n, x in zip(("q", "k", "v", "g", "b"), (dq, dk, dv, dg, dbeta)):
            grads[n].append(x)
    cat = {n: (np.concatenate(x[::-1], axis=1) if x else None) for n, x in grads.items()}
    if cat["q"] is None:   # T == 0
        return (np.zeros(q.shape[:2] + (key_heads, key_dim), dstate.dtype),
                np.zeros(q.shape[:2] + (key_heads, key_dim), dstate.dtype),
                np.zeros(v.shape, dstate.dtype), np.zeros(g.shape, dstate.dtype),
                np.zeros(beta.shape, dstate.dtype), dstate)
    dq = collapse_heads(cat["q"], key_heads, repeat)
    dk = collapse_heads(cat["k"], key_heads, repeat)
    return dq, dk, cat["v"], cat["g"], cat["b"], dstate


def _as(x, dtype):
    return None if x is None else np.asarray(x, dtype=dtype)


def gated_delta_chunked(q, k, v, g, beta, state=None, mask=None, chunk=DEFAULT_CHUNK,
                        dtype=np.float32):
    """Forward of the public entry point (tools/gdn_vjp.py:503-528).  Returns (y, final_state)."""
    if chunk <= 0:
        raise ValueError("chunk must be a positive integer")
    q, k, v, g, beta = (_as(x, dtype) for x in (q, k, v, g, beta))
    if state is None:
        state = np.zeros((q.shape[0], v.shape[2], v.shape[3], q.shape[3]), dtype=dtype)
    y, final_state, _ = forward(q, k, v, g, beta, _as(state, dtype), mask, chunk)
    return y, final_state


def gated_delta_chunked_vjp(q, k, v, g, beta, state, mask, dy, dstate, chunk=DEFAULT_CHUNK,
                            dtype=np.float32):
    """Forward + VJP.  Returns ((y, final_state), (dq, dk, dv, dg, dbeta, dstate0))."""
    if chunk <= 0:
        raise ValueError("chunk must be a positive integer")
    q, k, v, g, beta, dy = (_as(x, dtype) for x in (q, k, v, g, beta, dy))
    if state is None:
        state = np.zeros((q.shape[0], v.shape[2], v.shape[3], q.shape[3]), dtype=dtype)
    state = _as(state, dtype)
    dstate = np.zeros_like(state) if dstate is None else _as(dstate, dtype)
    y, final_state, boundaries = forward(q, k, v, g, beta, state, mask, chunk)
    grads = backward(q, k, v, g, beta, state, mask, boundaries, dy, dstate, chunk)
    return (y, final_state), grads


def gated_delta_ops_checkpointed(q, k, v, g, beta, state=None, mask=None, chunk=DEFAULT_CHUNK,
                                 dtype=np.float32):
    """tools/gdn_checkpoint.py:53-95: the same recurrence run in checkpointed chunks (forward)."""
    return gated_delta_chunked(q, k, v, g, beta, state, mask, chunk, dtype)


# --------------------------------------------------------------------------------------------------------
# Gates, L2 norm, causal conv, gated RMSNorm (engine/include/gdn.h, engine/include/ops.h)
# --------------------------------------------------------------------------------------------------------

def softplus(t):
    """Stable softplus, engine/include/gdn.h:23 (t > 20 ? t : log1p(exp(t)))."""
    t = np.asarray(t)
    return np.where(t > 20, t, np.log1p(np.exp(np.minimum(t, 20))))


def compute_g(A_log, a, dt_bias):
    """Multiplicative decay exp(-exp(A_log) * softplus(a + dt_bias)) (engine/include/gdn.h:20-25)."""
    return np.exp(-np.exp(A_log) * softplus(a + dt_bias))


def gates(a, b, A_log, dt_bias):
    """(decay, beta) as gdn_gates (engine/src/gdn.c:51-61)."""
    return compute_g(A_log, a, dt_bias), 1.0 / (1.0 + np.exp(-b))


def gates_bwd(a, b, A_log, dt_bias, d_decay, d_beta, allow_neg_eigval=False):
    """Backward of gates over [..., Hv] inputs.  Returns (da, db, dA_log, ddt_bias).

    decay = exp(-exp(A_log) sp(x)), x = a + dt_bias:  d/dx = -decay exp(A_log) sigmoid(x) (sp' = sigmoid,
    and exactly 1 on the t > 20 branch);  d/dA_log = -decay exp(A_log) sp(x).  beta = s sigmoid(b):
    d/db = s sigmoid(b)(1 - sigmoid(b)) with s = 2 when allow_neg_eigval.
    """
    x = a + dt_bias
    sp = softplus(x)
    dec = compute_g(A_log, a, dt_bias)
    e = np.exp(A_log)
    sig_x = np.where(x > 20, 1.0, 1.0 / (1.0 + np.exp(-np.minimum(x, 20))))
    dx = d_decay * (-dec * e * sig_x)
    sb = 1.0 / (1.0 + np.exp(-b))
    scale = 2.0 if allow_neg_eigval else 1.0
    db = d_beta * scale * sb * (1.0 - sb)
    red = tuple(range(dx.ndim - 1))
    dA_log = (d_decay * (-dec * e * sp)).sum(axis=red)
    ddt = dx.sum(axis=red)
    return dx, db, dA_log, ddt


def l2norm(x, eps=1e-6, scale=1.0):
    """scale * x / sqrt(sum x^2 + eps) over the last axis, sum in float64 (engine/src/gdn.c:40-49)."""
    x = np.asarray(x)
    ss = (x.astype(np.float64) ** 2).sum(axis=-1, keepdims=True)
    return (x * (scale / np.sqrt(ss + eps)).astype(x.dtype)).astype(x.dtype)


def l2norm_bwd(x, dy, eps=1e-6, scale=1.0):
    """Backward of l2norm: with n = sqrt(sum x^2 + eps), y = s x / n,
    dx = s/n * (dy - x (x . dy) / n^2)."""
    x64 = np.asarray(x, np.float64)
    dy64 = np.asarray(dy, np.float64)
    n2 = (x64 ** 2).sum(axis=-1, keepdims=True) + eps
    n = np.sqrt(n2)
    dot = (x64 * dy64).sum(axis=-1, keepdims=True)
    return scale / n * (dy64 - x64 * dot / n2)


def silu(x):
    return x / (1.0 + np.exp(-x))


def conv_silu(x, w):
    """Causal depthwise conv + SiLU over a whole sequence (engine/include/gdn.h:7-15).

    x: [B,T,C]; w: [C,K] (w[c, K-1] multiplies the current input).  Zero initial conv state.
    out[b,t,c] = silu(sum_j w[c,j] * x[b, t-(K-1)+j, c]) with x at negative t = 0.
    """
    B, T, C = x.shape
    K = w.shape[1]
    xp = np.concatenate([np.zeros((B, K - 1, C), x.dtype), x], axis=1)
    pre = np.zeros((B, T, C), dtype=np.result_type(x, w))
    for j in range(K):
        pre += w[:, j] * xp[:, j:j + T]
    return silu(pre), pre


def conv_silu_bwd(x, w, dout):
    """Backward of conv_silu.  Returns (dx, dw) with dw [C,K]."""
    B, T, C = x.shape
    K = w.shape[1]
    _, pre = conv_silu(x, w)
    s = 1.0 / (1.0 + np.exp(-pre))
    dpre = dout * s * (1.0 + pre * (1.0 - s))
    xp = np.concatenate([np.zeros((B, K - 1, C), x.dtype), x], axis=1)
    dxp = np.zeros_like(xp, dtype=dpre.dtype)
    dw = np.zeros((C, K), dtype=dpre.dtype)
    for j in range(K):
        dxp[:, j:j + T] += w[:, j] * dpre
        dw[:, j] = (dpre * xp[:, j:j + T]).sum(axis=(0, 1))
    return dxp[:, K - 1:], dw


def rmsnorm(x, w, eps=1e-6):
    """x / sqrt(mean(x^2) + eps) * w over the last axis, mean in float64 (engine/src/ops.c op_rmsnorm)."""
    x = np.asarray(x)
    ms = (x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    rms = np.sqrt(ms + eps).astype(np.float32)
    return (x / rms * w).astype(np.result_type(x, w))


def silu_mul(gate, up):
    """silu(gate) * up (engine/include/ops.h:10-11)."""
    return gate / (1.0 + np.exp(-gate)) * up


def gated_rmsnorm(y, z, w, eps=1e-6):
    """Gated RMSNorm of engine/src/gdn_layer.c:47-55: rmsnorm(y_h, w) * silu(z_h) per value head."""
    return silu_mul(z, rmsnorm(y, w, eps))


def gated_rmsnorm_bwd(y, z, w, dout, eps=1e-6):
    """Backward of gated_rmsnorm over the last axis.  Returns (dy, dz, dw) in float64.

    r = 1/sqrt(mean y^2 + eps); n = y r; out = n w silu(z).
    dn = dout w silu(z); dy = r (dn - y r^2 mean(dn y)); dz = dout n w silu'(z); dw = sum dout n silu(z).
    """
    y = np.asarray(y, np.float64)
    z = np.asarray(z, np.float64)
    w = np.asarray(w, np.float64)
    dout = np.asarray(dout, np.float64)
    D = y.shape[-1]
    r = 1.0 / np.sqrt((y ** 2).mean(axis=-1, keepdims=True) + eps)
    n = y * r
    sz = 1.0 / (1.0 + np.exp(-z))
    silz = z * sz
    dn = dout * w * silz
    dy = r * (dn - y * r * r * (dn * y).sum(axis=-1, keepdims=True) / D)
    dz = dout * n * w * sz * (1.0 + z * (1.0 - sz))
    dw = (dout * n * silz).reshape(-1, D).sum(axis=0)
    return dy, dz, dw


# --------------------------------------------------------------------------------------------------------
# Synthetic inputs for the measured workloads
# --------------------------------------------------------------------------------------------------------

def make_inputs(B, T, Hk, Hv, D, seed=0, s0_std=0.0, dtype=np.float32):
    """Seeded inputs: q,k ~ N(0,1) L2-normalised per head (eps 1e-6), q scaled by D^-1/2; v ~ N(0,1);
    beta = sigmoid(N(0,1)); log-decay = -exp(A_log) softplus(a + dt_bias), A_log ~ U(log 1, log 16) per
    head, a ~ N(0,1), dt_bias = 0; S0 ~ N(0, s0_std) (zeros when s0_std == 0); dO ~ N(0,1).

    Returns a dict with q, k, v, beta, g_log (log decay), decay, state, dy.  One numpy Generator per
    tensor, seeded ``seed*100 + i`` in that fixed order.
    """
    rngs = [np.random.default_rng(seed * 100 + i) for i in range(8)]
    q = rngs[0].standard_normal((B, T, Hk, D))
    k = rngs[1].standard_normal((B, T, Hk, D))
    q = l2norm(q, 1e-6, 1.0 / math.sqrt(D))
    k = l2norm(k, 1e-6, 1.0)
    v = rngs[2].standard_normal((B, T, Hv, D))
    beta = 1.0 / (1.0 + np.exp(-rngs[3].standard_normal((B, T, Hv))))
    A_log = rngs[4].uniform(math.log(1.0), math.log(16.0), size=(Hv,))
    a = rngs[5].standard_normal((B, T, Hv))
    g_log = -np.exp(A_log) * softplus(a)
    state = (rngs[6].standard_normal((B, Hv, D, D)) * s0_std if s0_std > 0
             else np.zeros((B, Hv, D, D)))
    dy = rngs[7].standard_normal((B, T, Hv, D))
    out = dict(q=q, k=k, v=v, beta=beta, g_log=g_log, decay=np.exp(g_log), state=state, dy=dy,
               A_log=A_log, a=a)
    return {n: np.asarray(x, dtype=dtype) for n, x in out.items()}
