"""torch.autograd bridge to the block ops around the recurrence: causal depthwise conv1d + SiLU, per-head q/k L2
norm, gates, and gated RMSNorm * SiLU(z), each a HIP kernel pair called through the C ABI.

These are the steps one GDN block runs around the delta rule (``engine/src/gdn_layer.c:29-55``, the sequence
form of ``engine/include/gdn.h:7-25``), with hand-derived backwards; the reference gets these backwards from MLX
autodiff of the mlx-lm ops (``tools/gdn_vjp.py:554-560``).  Tensors must live on a ROCm device; there is no CPU
path.
"""

from __future__ import annotations

from typing import Optional

import torch

import gdn_lib as L

Array = torch.Tensor


def _require_cuda(*tensors: Optional[Array]) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError("the GDN block ops run on a ROCm GPU only; got tensors on " + str(dev))
    for t in tensors:
        if t is not None and t.device != dev:
            raise ValueError("all inputs must be on the same device")
    return dev


def _code(t: Array) -> int:
    try:
        return L.DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; use float32, bfloat16 or float16") from None


def _workspace(nbytes: int, dev: torch.device) -> Array:
    return torch.empty((max(int(nbytes), 1),), dtype=torch.uint8, device=dev)


# ------------------------------------------------------------------------------------------------ gates


class _Gates(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, A_log, dt_bias, log_space, allow_neg_eigval):
        dev = _require_cuda(a, b, A_log, dt_bias)
        Hv = a.shape[-1]
        if b.shape != a.shape or A_log.shape != (Hv,) or dt_bias.shape != (Hv,):
            raise ValueError(f"gates expect a, b [..., Hv] and A_log, dt_bias [Hv]; got {tuple(a.shape)}, "
                             f"{tuple(b.shape)}, {tuple(A_log.shape)}, {tuple(dt_bias.shape)}")
        a = a.contiguous()
        b = b.to(a.dtype).contiguous()
        A32, d32 = A_log.float().contiguous(), dt_bias.float().contiguous()
        tokens = a.numel() // Hv
        g = torch.empty(a.shape, dtype=torch.float32, device=dev)
        beta = torch.empty(a.shape, dtype=torch.float32, device=dev)
        lib = L.load()
        L.check(lib.gdn_gates_fwd(L.ptr(a), L.ptr(b), L.ptr(A32), L.ptr(d32), L.ptr(g), L.ptr(beta), tokens, Hv,
                                  _code(a), int(log_space), int(allow_neg_eigval), L.stream_handle(dev)))
        ctx.save_for_backward(a, b, A32, d32, g)
        ctx.meta = (bool(log_space), bool(allow_neg_eigval), A_log.dtype, dt_bias.dtype)
        return g, beta

    @staticmethod
    def backward(ctx, dg, dbeta):
        a, b, A32, d32, g = ctx.saved_tensors
        log_space, neg, A_dtype, d_dtype = ctx.meta
        dev = a.device
        Hv = a.shape[-1]
        tokens = a.numel() // Hv
        dg = torch.zeros_like(g) if dg is None else dg.float().contiguous()
        dbeta = torch.zeros_like(g) if dbeta is None else dbeta.float().contiguous()
        da, db = torch.empty_like(a), torch.empty_like(b)
        dA = torch.empty((Hv,), dtype=torch.float32, device=dev)
        ddt = torch.empty((Hv,), dtype=torch.float32, device=dev)
        lib = L.load()
        nws = lib.gdn_gates_bwd_workspace_bytes(tokens, Hv)
        ws = _workspace(nws, dev)
        L.check(lib.gdn_gates_bwd(L.ptr(a), L.ptr(b), L.ptr(A32), L.ptr(d32), L.ptr(g), L.ptr(dg), L.ptr(dbeta),
                                  L.ptr(da), L.ptr(db), L.ptr(dA), L.ptr(ddt), L.ptr(ws), nws, tokens, Hv, _code(a),
                                  _code(a), int(log_space), int(neg), L.stream_handle(dev)))
        return da, db, dA.to(A_dtype), ddt.to(d_dtype), None, None


def gates(a: Array, b: Array, A_log: Array, dt_bias: Array, *, log_space: bool = False,
          allow_neg_eigval: bool = False) -> tuple[Array, Array]:
    """(g, beta) with g = exp(l) (or l itself when log_space), l = -exp(A_log) softplus(a + dt_bias), and
    beta = sigmoid(b) (x2 when allow_neg_eigval); gdn_gates of engine/include/gdn.h:20-25 over every token.
    Both outputs are float32, shaped like a."""
    return _Gates.apply(a, b, A_log, dt_bias, log_space, allow_neg_eigval)


# ------------------------------------------------------------------------------------------------ l2 norm


class _L2Norm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, scale, eps):
        dev = _require_cuda(x)
        x = x.contiguous()
        D = x.shape[-1]
        rows = x.numel() // D if D else 0
        y = torch.empty_like(x)
        L.check(L.load().gdn_l2norm_fwd(L.ptr(x), L.ptr(y), rows, D, float(eps), float(scale), _code(x),
                                        L.stream_handle(dev)))
        ctx.save_for_backward(x)
        ctx.meta = (float(scale), float(eps))
        return y

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        scale, eps = ctx.meta
        dy = dy.contiguous()
        D = x.shape[-1]
        rows = x.numel() // D if D else 0
        dx = torch.empty_like(x)
        L.check(L.load().gdn_l2norm_bwd(L.ptr(x), L.ptr(dy), L.ptr(dx), rows, D, eps, scale, _code(x), _code(dy),
                                        L.stream_handle(x.device)))
        return dx, None, None


def l2norm(x: Array, scale: float = 1.0, eps: float = 1e-6) -> Array:
    """scale * x / sqrt(sum x^2 + eps) over the last axis (gdn_l2norm, engine/include/gdn.h:17-18)."""
    return _L2Norm.apply(x, scale, eps)


def normalize_qk(q: Array, k: Array, inv_scale: float, eps: float = 1e-6) -> tuple[Array, Array]:
    """Per-head q/k normalisation of one GDN block: q scaled by inv_scale, k by 1
    (engine/src/gdn_layer.c:35-39)."""
    return l2norm(q, inv_scale, eps), l2norm(k, 1.0, eps)


# ------------------------------------------------------------------------------------------------ conv1d + SiLU


def _conv_weight(w: Array, C: int) -> tuple[Array, int]:
    """[C, K] or torch's depthwise Conv1d weight [C, 1, K] -> contiguous fp32 [C, K]."""
    if w.dim() == 3 and w.shape[1] == 1:
        w = w[:, 0, :]
    if w.dim() != 2 or w.shape[0] != C:
        raise ValueError(f"conv weight must be [C, K] or [C, 1, K] with C = {C}; got {tuple(w.shape)}")
    return w.float().contiguous(), w.shape[1]


class _ConvSiLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, state_in, want_state):
        dev = _require_cuda(x, w, state_in)
        if x.dim() != 3:
            raise ValueError(f"conv input must be [B, T, C]; got {tuple(x.shape)}")
        B, T, C = x.shape
        w32, K = _conv_weight(w, C)
        x = x.contiguous()
        s_in = None if state_in is None else state_in.float().contiguous()
        if s_in is not None and s_in.shape != (B, K - 1, C):
            raise ValueError(f"conv state must be [B, K-1, C] = {(B, K - 1, C)}; got {tuple(s_in.shape)}")
        out = torch.empty_like(x)
        s_out = torch.empty((B, K - 1, C), dtype=torch.float32, device=dev) if want_state else None
        L.check(L.load().gdn_conv_silu_fwd(L.ptr(x), L.ptr(w32), L.ptr(s_in), L.ptr(out), L.ptr(s_out), B, T, C, K,
                                           _code(x), L.stream_handle(dev)))
        ctx.save_for_backward(x, w32, s_in)
        ctx.w_shape, ctx.w_dtype = w.shape, w.dtype
        if s_out is not None:
            ctx.mark_non_differentiable(s_out)
        return out, s_out

    @staticmethod
    def backward(ctx, dout, _ds):
        x, w32, s_in = ctx.saved_tensors
        B, T, C = x.shape
        K = w32.shape[1]
        dev = x.device
        dout = torch.zeros_like(x) if dout is None else dout.contiguous()
        dx = torch.empty_like(x)
        dw = torch.empty((C, K), dtype=torch.float32, device=dev)
        lib = L.load()
        nws = lib.gdn_conv_silu_bwd_workspace_bytes(B, T, C, K)
        ws = _workspace(nws, dev)
        L.check(lib.gdn_conv_silu_bwd(L.ptr(x), L.ptr(w32), L.ptr(s_in), L.ptr(dout), L.ptr(dx), L.ptr(dw),
                                      L.ptr(ws), nws, B, T, C, K, _code(x), _code(dout), L.stream_handle(dev)))
        return dx, dw.reshape(ctx.w_shape).to(ctx.w_dtype), None, None


def conv_silu(x: Array, w: Array, state: Optional[Array] = None, *, return_state: bool = False):
    """Causal depthwise conv over time + SiLU, the sequence form of gdn_conv_step (engine/include/gdn.h:7-15).

    x [B, T, C]; w [C, K] or [C, 1, K] (w[c, K-1] multiplies the current input); state [B, K-1, C] holds the
    K-1 inputs before x (oldest first; None = zeros).  Returns out [B, T, C], and with return_state also the
    state after x (float32, not differentiable).  No gradient flows into ``state``."""
    out, s = _ConvSiLU.apply(x, w, state, return_state)
    return (out, s) if return_state else out


def _aligned16(t: Array) -> Array:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _ConvQKV(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, state_in, heads, q_scale, eps, want_state):
        Hk, Dk, Hv, Dv = heads
        dev = _require_cuda(x, w, state_in)
        if x.dim() != 3 or x.shape[-1] != 2 * Hk * Dk + Hv * Dv:
            raise ValueError(f"conv input must be [B, T, 2*Hk*Dk + Hv*Dv]; got {tuple(x.shape)}")
        B, T, C = x.shape
        w32, K = _conv_weight(w, C)
        x = _aligned16(x)
        s_in = None if state_in is None else state_in.float().contiguous()
        if s_in is not None and s_in.shape != (B, K - 1, C):
            raise ValueError(f"conv state must be [B, K-1, C] = {(B, K - 1, C)}; got {tuple(s_in.shape)}")
        q = torch.empty((B, T, Hk, Dk), dtype=x.dtype, device=dev)
        k = torch.empty((B, T, Hk, Dk), dtype=x.dtype, device=dev)
        v = torch.empty((B, T, Hv, Dv), dtype=x.dtype, device=dev)
        s_out = torch.empty((B, K - 1, C), dtype=torch.float32, device=dev) if want_state else None
        L.check(L.load().gdn_conv_qkv_fwd(L.ptr(x), L.ptr(w32), L.ptr(s_in), L.ptr(q), L.ptr(k), L.ptr(v),
                                          L.ptr(s_out), B, T, Hk, Dk, Hv, Dv, K, float(q_scale), float(eps),
                                          _code(x), L.stream_handle(dev)))
        ctx.save_for_backward(x, w32, s_in)
        ctx.meta = (heads, float(q_scale), float(eps), w.shape, w.dtype)
        if s_out is not None:
            ctx.mark_non_differentiable(s_out)
        return q, k, v, s_out

    @staticmethod
    def backward(ctx, dq, dk, dv, _ds):
        x, w32, s_in = ctx.saved_tensors
        (Hk, Dk, Hv, Dv), q_scale, eps, w_shape, w_dtype = ctx.meta
        B, T, C = x.shape
        K = w32.shape[1]
        dev = x.device
        gd = next((g.dtype for g in (dq, dk, dv) if g is not None), x.dtype)
        fill = lambda g, shape: (torch.zeros(shape, dtype=gd, device=dev) if g is None else _aligned16(g.to(gd)))
        dq, dk = fill(dq, (B, T, Hk, Dk)), fill(dk, (B, T, Hk, Dk))
        dv = fill(dv, (B, T, Hv, Dv))
        dx = torch.empty_like(x)
        dw = torch.empty((C, K), dtype=torch.float32, device=dev)
        lib = L.load()
        nws = lib.gdn_conv_silu_bwd_workspace_bytes(B, T, C, K)
        ws = _workspace(nws, dev)
        L.check(lib.gdn_conv_qkv_bwd(L.ptr(x), L.ptr(w32), L.ptr(s_in), L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(dx),
                                     L.ptr(dw), L.ptr(ws), nws, B, T, Hk, Dk, Hv, Dv, K, q_scale, eps, _code(x),
                                     _code(dq), L.stream_handle(dev)))
        return dx, dw.reshape(w_shape).to(w_dtype), None, None, None, None, None


def conv_qkv(x: Array, w: Array, Hk: int, Dk: int, Hv: int, Dv: int, q_scale: float, eps: float = 1e-6,
             state: Optional[Array] = None, *, return_state: bool = False):
    """Steps 2-4 of one block (engine/src/gdn_layer.c:29-39) on x [B, T, 2*Hk*Dk + Hv*Dv]: causal depthwise conv
    + SiLU, split into q, k [B, T, Hk, Dk] and v [B, T, Hv, Dv], q and k L2-normalised per head (q scaled by
    q_scale).  One fused kernel pair where the shape allows (K = 4, 16-byte vector lanes per head), else the
    separate conv and L2-norm kernels.  ``state``/``return_state`` as in ``conv_silu``."""
    try:
        q, k, v, s = _ConvQKV.apply(x, w, state, (Hk, Dk, Hv, Dv), q_scale, eps, return_state)
    except L.GDNError as e:
        if e.status != L.GDN_ERR_UNSUPPORTED:
            raise
        out, s = _ConvSiLU.apply(x, w, state, return_state)
        B, T, _ = x.shape
        kd = Hk * Dk
        q = out[..., :kd].reshape(B, T, Hk, Dk)
        k = out[..., kd:2 * kd].reshape(B, T, Hk, Dk)
        v = out[..., 2 * kd:].reshape(B, T, Hv, Dv)
        q, k = normalize_qk(q, k, q_scale, eps)
    return (q, k, v, s) if return_state else (q, k, v)


# ------------------------------------------------------------------------------------------------ gated RMSNorm


class _GatedRMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, z, w, eps):
        dev = _require_cuda(y, z, w)
        if z.shape != y.shape or w.shape != y.shape[-1:]:
            raise ValueError(f"gated RMSNorm expects y, z [..., D] and w [D]; got {tuple(y.shape)}, "
                             f"{tuple(z.shape)}, {tuple(w.shape)}")
        y, z = y.contiguous(), z.contiguous()
        w32 = w.float().contiguous()
        D = y.shape[-1]
        rows = y.numel() // D if D else 0
        out = torch.empty_like(y)
        L.check(L.load().gdn_gated_rmsnorm_fwd(L.ptr(y), L.ptr(z), L.ptr(w32), L.ptr(out), rows, D, float(eps),
                                               _code(y), _code(z), L.stream_handle(dev)))
        ctx.save_for_backward(y, z, w32)
        ctx.meta = (float(eps), w.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        y, z, w32 = ctx.saved_tensors
        eps, w_dtype = ctx.meta
        dev = y.device
        D = y.shape[-1]
        rows = y.numel() // D if D else 0
        dout = dout.contiguous()
        dy, dz = torch.empty_like(y), torch.empty_like(z)
        dw = torch.empty((D,), dtype=torch.float32, device=dev)
        lib = L.load()
        nws = lib.gdn_gated_rmsnorm_bwd_workspace_bytes(rows, D)
        ws = _workspace(nws, dev)
        L.check(lib.gdn_gated_rmsnorm_bwd(L.ptr(y), L.ptr(z), L.ptr(w32), L.ptr(dout), L.ptr(dy), L.ptr(dz),
                                          L.ptr(dw), L.ptr(ws), nws, rows, D, eps, _code(y), _code(z), _code(dout),
                                          L.stream_handle(dev)))
        return dy, dz, dw.to(w_dtype), None


def gated_rmsnorm(y: Array, z: Array, w: Array, eps: float = 1e-6) -> Array:
    """y / sqrt(mean(y^2) + eps) * w * silu(z) over the last axis (op_rmsnorm then op_silu_mul per value head,
    engine/include/ops.h:7-11, engine/src/gdn_layer.c:47-55).  Output has y's dtype."""
    return _GatedRMSNorm.apply(y, z, w, eps)
