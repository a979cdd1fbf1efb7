"""Independent float64 torch statement of the delta-rule recurrence, for pinning the oracle's hand-derived
backward with torch autograd (a library routine).  Written from the recurrence's definition
(engine/include/gdn.h:217-226 plus the mask rule of tools/gdn_vjp.py:3-6), not from the oracle's code."""

import torch


def recurrence(q, k, v, g, beta, state, mask=None):
    """q,k [B,T,Hk,Dk]; v [B,T,Hv,Dv]; g [B,T,Hv] or [B,T,Hv,Dk] decay; beta [B,T,Hv];
    state [B,Hv,Dv,Dk]; mask [B,T] bool.  Returns (y [B,T,Hv,Dv], final state)."""
    B, T, Hk, Dk = q.shape
    Hv = v.shape[2]
    rep = Hv // Hk
    S = state
    ys = []
    for t in range(T):
        qt = q[:, t].repeat_interleave(rep, dim=1)
        kt = k[:, t].repeat_interleave(rep, dim=1)
        gt = g[:, t]
        dec = gt[:, :, None, None] if gt.dim() == 2 else gt[:, :, None, :]
        A = S * dec
        kv = torch.einsum("bhij,bhj->bhi", A, kt)
        delta = (v[:, t] - kv) * beta[:, t, :, None]
        cand = A + delta[:, :, :, None] * kt[:, :, None, :]
        ys.append(torch.einsum("bhij,bhj->bhi", cand, qt))
        S = cand if mask is None else torch.where(mask[:, t, None, None, None], cand, S)
    if T == 0:
        return v.new_zeros(v.shape), S
    return torch.stack(ys, dim=1), S


def vjp(q, k, v, g, beta, state, mask, dy, dstate):
    """Returns (y, S_T, dq, dk, dv, dg, dbeta, dS0) in float64 via torch autograd."""
    xs = [torch.as_tensor(x, dtype=torch.float64).clone().requires_grad_(True)
          for x in (q, k, v, g, beta, state)]
    m = None if mask is None else torch.as_tensor(mask, dtype=torch.bool)
    y, S = recurrence(*xs, m)
    loss = (y * torch.as_tensor(dy, dtype=torch.float64)).sum() + \
        (S * torch.as_tensor(dstate, dtype=torch.float64)).sum()
    grads = torch.autograd.grad(loss, xs, allow_unused=True)
    grads = [torch.zeros_like(x) if gr is None else gr for x, gr in zip(xs, grads)]
    return [t.detach().numpy() for t in (y, S, *grads)]
