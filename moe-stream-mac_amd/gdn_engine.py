"""torch.autograd bridge to the HIP engine: one Function whose forward runs ``gdn_fwd`` (saving chunk
snapshots) and whose backward runs ``gdn_bwd``.

This is the device-side replacement of the reference's ``mx.custom_function`` pair
(``tools/gdn_vjp.py:477-500``): the forward keeps ceil(T/chunk)-1 boundary states (the reference keeps
ceil(T/chunk)+1 including S0 and S_T, ``:205-235``), and the backward recomputes every state inside a
chunk from its boundary, like ``_chunk_vjp`` (``:273-320``) and ``mx.checkpoint`` in
``tools/gdn_checkpoint.py:39-50``.  Tensors must live on a ROCm device; there is no CPU path.
"""

from __future__ import annotations

import os
from typing import Optional

import torch

import gdn_lib as L


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError("the GDN engine runs on a ROCm GPU only; got tensors on " + str(dev))
    for t in tensors:
        if t is not None and t.device != dev:
            raise ValueError("all GDN inputs must be on the same device")
    return dev


def gate_kind_for(g: torch.Tensor, log_gate: bool) -> int:
    if g.dim() == 3:
        return L.GATE_LOG if log_gate else L.GATE_DECAY
    if g.dim() == 4:
        return L.GATE_LOG_VEC if log_gate else L.GATE_DECAY_VEC
    raise ValueError(f"Unsupported gating shape {tuple(g.shape)}")


def _saved_bytes(lib, B, T, Hk, Hv, Dk, Dv, chunk, gate, has_mask, form, in_code) -> int:
    return int(lib.gdn_saved_bytes(B, T, Hk, Hv, Dk, Dv, chunk, gate, has_mask, form, in_code))


class _GDNRecurrence(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, g, beta, state, mask, chunk, log_gate, out_dtype, need_saved, form,
                backward_error=None):
        # an output that the loss does not use reaches backward as None instead of a zero tensor filled for it
        # (the library takes a NULL exit-state cotangent as zero)
        ctx.set_materialize_grads(False)
        dev = _require_device(q, k, v, g, beta, state)
        B, T, Hk, Dk = q.shape
        Hv, Dv = v.shape[2], v.shape[3]
        in_dtype = q.dtype
        gate = gate_kind_for(g, log_gate)
        lib = L.load()
        has_mask = int(mask is not None)
        resolved = int(lib.gdn_select_form(Hv, Dk, Dv, has_mask, gate, form, L.DTYPE_CODE[in_dtype]))
        if resolved < 0:
            L.check(resolved)
        y = torch.empty((B, T, Hv, Dv), device=dev, dtype=out_dtype)
        state_T = torch.empty((B, Hv, Dv, Dk), device=dev, dtype=torch.float32)
        in_code = L.DTYPE_CODE[in_dtype]
        n_saved = _saved_bytes(lib, B, T, Hk, Hv, Dk, Dv, chunk, gate, has_mask, form, in_code) if need_saved else 0
        # a forward-only call keeps nothing (saved = NULL); the saved buffer of a training call may still be empty
        # (T <= chunk), which is passed as a real pointer so that the library sees a training call
        saved = torch.empty((max(n_saved, 1) if need_saved else 0,), device=dev, dtype=torch.uint8)
        n_ws = int(lib.gdn_fwd_workspace_bytes(B, T, Hk, Hv, Dk, Dv, chunk, gate, has_mask, form, in_code,
                                               int(need_saved)))
        ws = torch.empty((n_ws,), device=dev, dtype=torch.uint8) if n_ws else None
        L.check(lib.gdn_fwd(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(g), L.ptr(beta), L.ptr(state),
                            L.ptr(mask), L.ptr(y), L.ptr(state_T), L.ptr(saved) if need_saved else None, n_saved,
                            L.ptr(ws), n_ws, B, T, Hk, Hv, Dk, Dv, chunk, in_code, L.DTYPE_CODE[out_dtype],
                            gate, form, L.stream_handle(dev)))
        del ws
        ctx.save_for_backward(q, k, v, g, beta, state, mask, saved)
        ctx.meta = (chunk, gate, form)
        ctx.backward_error = backward_error
        return y, state_T

    @staticmethod
    def backward(ctx, dy, dstate_T):
        if ctx.backward_error is not None:
            raise ValueError(ctx.backward_error)
        q, k, v, g, beta, state, mask, saved = ctx.saved_tensors
        chunk, gate, form = ctx.meta
        dev = q.device
        B, T, Hk, Dk = q.shape
        Hv, Dv = v.shape[2], v.shape[3]
        lib = L.load()
        has_mask = int(mask is not None)
        if dy is None:
            dy = torch.zeros((B, T, Hv, Dv), device=dev, dtype=torch.float32)
        dy = dy.contiguous()
        if dy.dtype not in L.DTYPE_CODE or (q.dtype == torch.bfloat16 and dy.dtype == torch.float16):
            # the chunked form with bf16 inputs reads a bf16 or fp32 cotangent
            dy = dy.float()
        dy = _aligned(dy)
        dstate_T = None if dstate_T is None else dstate_T.contiguous().float()
        grad_dtype = q.dtype
        dq = torch.empty((B, T, Hk, Dk), device=dev, dtype=grad_dtype)
        dk = torch.empty_like(dq)
        dv = torch.empty((B, T, Hv, Dv), device=dev, dtype=grad_dtype)
        dg = torch.empty(g.shape, device=dev, dtype=torch.float32)
        dbeta = torch.empty((B, T, Hv), device=dev, dtype=torch.float32)
        dS0 = torch.empty((B, Hv, Dv, Dk), device=dev, dtype=torch.float32)
        ws_bytes = int(lib.gdn_bwd_workspace_bytes(B, T, Hk, Hv, Dk, Dv, chunk, gate, has_mask, form,
                                                   L.DTYPE_CODE[q.dtype]))
        ws = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
        L.check(lib.gdn_bwd(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(g), L.ptr(beta), L.ptr(state), L.ptr(mask),
                            L.ptr(saved), saved.numel(), L.ptr(dy),
                            L.ptr(dstate_T), L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(dg), L.ptr(dbeta),
                            L.ptr(dS0), L.ptr(ws), ws_bytes, B, T, Hk, Hv, Dk, Dv, chunk,
                            L.DTYPE_CODE[q.dtype], L.DTYPE_CODE[dy.dtype], L.DTYPE_CODE[grad_dtype], gate,
                            form, L.stream_handle(dev)))
        return dq, dk, dv, dg, dbeta, dS0, None, None, None, None, None, None, None


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """The kernels read rows with 16-byte loads: a contiguous view at an unaligned offset is copied."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _prep(q, k, v, g, beta, state, mask):
    common = torch.promote_types(torch.promote_types(q.dtype, k.dtype), v.dtype)
    if common not in L.DTYPE_CODE:
        common = torch.float32
    q, k, v = (_aligned(x.to(common).contiguous()) for x in (q, k, v))
    g = g.to(torch.float32).contiguous()
    beta = beta.to(torch.float32).contiguous()
    state = state.to(torch.float32).contiguous()
    if mask is not None:
        mask = mask.to(device=q.device, dtype=torch.uint8).contiguous()
    return q, k, v, g, beta, state, mask


def check_shapes(q, k, v, g, beta, state, mask) -> None:
    """Shape checks raising the reference's exception types."""
    if q.dim() != 4 or k.shape != q.shape:
        raise ValueError("q and k must both be [B, T, Hk, Dk]")
    B, T, Hk, Dk = q.shape
    if v.dim() != 4 or v.shape[:2] != (B, T):
        raise ValueError("v must be [B, T, Hv, Dv]")
    Hv, Dv = v.shape[2], v.shape[3]
    if Hv % Hk:
        raise ValueError("q/k head count must divide the value head count")
    if g.dim() not in (3, 4):
        raise ValueError(f"Unsupported gating shape {tuple(g.shape)}")
    want_g = (B, T, Hv) if g.dim() == 3 else (B, T, Hv, Dk)
    if tuple(g.shape) != want_g:
        raise ValueError(f"Unsupported gating shape {tuple(g.shape)}")
    if tuple(beta.shape) != (B, T, Hv):
        raise ValueError("beta must be [B, T, Hv]")
    if tuple(state.shape) != (B, Hv, Dv, Dk):
        raise ValueError("state must be [B, Hv, Dv, Dk]")
    if mask is not None and tuple(mask.shape) != (B, T):
        raise ValueError("mask must be [B, T]")


def default_form() -> int:
    """Form requested by default: GDN_FORM=auto|recurrent|chunk in the environment, else auto."""
    name = os.environ.get("GDN_FORM", "auto").strip().lower()
    if name not in L.FORMS:
        raise ValueError(f"GDN_FORM must be one of {sorted(L.FORMS)}, got {name!r}")
    return L.FORMS[name]


def recurrence(q, k, v, g, beta, state, mask=None, chunk: int = 64, log_gate: bool = False,
               output_dtype: Optional[torch.dtype] = None, need_grad: Optional[bool] = None,
               form: Optional[str] = None, backward_error: Optional[str] = None):
    """(y, final_state) of the delta-rule recurrence with a HIP forward and VJP.

    ``g`` is the multiplicative decay ([B,T,Hv] or [B,T,Hv,Dk]) or, with ``log_gate``, the log decay.
    ``y`` defaults to the dtype the reference's arithmetic promotes to (fp32 with an fp32 state).
    ``need_grad=False`` runs the forward-only path (no autograd graph).  ``form`` is "auto" (default, or the
    GDN_FORM environment variable), "recurrent" or "chunk".  ``backward_error``, when given, is raised as a
    ``ValueError`` by the backward (the forward runs).
    """
    if chunk <= 0:
        raise ValueError("chunk must be a positive integer")
    check_shapes(q, k, v, g, beta, state, mask)
    _require_device(q, k, v, g, beta, state)
    out_dtype = output_dtype
    if out_dtype is None:
        out_dtype = q.dtype
        for t in (k, v, g, beta, state):
            out_dtype = torch.promote_types(out_dtype, t.dtype)
        if out_dtype not in L.DTYPE_CODE:
            out_dtype = torch.float32
    grads_wanted = torch.is_grad_enabled() and any(
        t.requires_grad for t in (q, k, v, g, beta, state))
    if need_grad is None:
        need_grad = grads_wanted
    form_code = default_form() if form is None else L.FORMS[form]
    pq, pk, pv, pg, pb, ps, pm = _prep(q, k, v, g, beta, state, mask)
    if not (need_grad and grads_wanted) and q.shape[1] == 1 and pm is None:
        # one token, no gradient: the decode step (gdn_recurrent_step's counterpart)
        with torch.no_grad():
            state_T = torch.empty_like(ps)
            y = decode_step(pq[:, 0], pk[:, 0], pv[:, 0], pg[:, 0], pb[:, 0], ps, state_T, log_gate, out_dtype)
        return y[:, None], state_T
    if not (need_grad and grads_wanted):
        with torch.no_grad():
            return _GDNRecurrence.forward(_NoCtx(), pq, pk, pv, pg, pb, ps, pm, chunk, log_gate, out_dtype,
                                          False, form_code)
    y, state_T = _GDNRecurrence.apply(pq, pk, pv, pg, pb, ps, pm, chunk, log_gate, out_dtype, True, form_code,
                                      backward_error)
    return y, state_T


def decode_step(q, k, v, g, beta, state_in, state_out, log_gate: bool = False,
                out_dtype: Optional[torch.dtype] = None):
    """One token of B sequences: q, k [B, Hk, Dk], v [B, Hv, Dv], g [B, Hv] (or [B, Hv, Dk]), beta [B, Hv];
    reads state_in [B, Hv, Dv, Dk] fp32 (None = zeros) and writes state_out (which may be state_in: in place).
    Returns y [B, Hv, Dv].  Forward only (engine/include/gdn.h:27-38)."""
    dev = _require_device(q, k, v, g, beta, state_out)
    B, Hk, Dk = q.shape
    Hv, Dv = v.shape[1], v.shape[2]
    if state_out.dtype != torch.float32 or not state_out.is_contiguous() or \
            tuple(state_out.shape) != (B, Hv, Dv, Dk):
        raise ValueError("state_out must be a contiguous float32 [B, Hv, Dv, Dk] tensor")
    if state_in is not None:
        state_in = state_in.to(torch.float32).contiguous()
    gate = gate_kind_for(g[:, None], log_gate)
    out_dtype = out_dtype or q.dtype
    if out_dtype not in L.DTYPE_CODE:
        out_dtype = torch.float32
    y = torch.empty((B, Hv, Dv), device=dev, dtype=out_dtype)
    lib = L.load()
    # the contiguous copies stay referenced until the launch is enqueued (a copy freed earlier could hand its
    # memory to the next one)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    g, beta = g.float().contiguous(), beta.float().contiguous()
    L.check(lib.gdn_decode_step(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(g), L.ptr(beta), L.ptr(state_in),
                                L.ptr(state_out), L.ptr(y), B, Hk, Hv, Dk, Dv, L.DTYPE_CODE[q.dtype],
                                L.DTYPE_CODE[out_dtype], gate, L.stream_handle(dev)))
    return y


class _NoCtx:
    """Stand-in ctx for calling the forward without building an autograd node."""

    def save_for_backward(self, *args):
        pass

    def set_materialize_grads(self, value):
        pass

