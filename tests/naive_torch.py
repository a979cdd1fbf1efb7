"""Independent float64 torch statement of the delta-rule recurrence, for pinning the oracle's hand-derived
backward with torch autograd (a library routine).  Written from the recurrence's definition
(engine/include/gdn.h:27-38 plus the mask rule of tools/gdn_vjp.py:3-6), not from the oracle's code."""

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


def gdn_block(x, P, Hk, Hv, Dk, Dv, eps=1e-6):
    """One GDN block over a sequence in float64 torch ops, written from engine/src/gdn_layer.c:18-58:
    projections (W + scale B A when a LoRA adapter is present), causal depthwise conv + SiLU, per-head L2 norm
    (q scaled by Dk^-1/2), gates, the recurrence from a zero state, rmsnorm(y) * w * silu(z), out-projection.
    P maps names to float64 tensors (those requiring grad are differentiated by the caller)."""
    import torch.nn.functional as F

    def W(n):
        w = P["W_" + n]
        if ("A_" + n) in P:
            w = w + P["lora_scale"] * P["B_" + n] @ P["A_" + n]
        return w

    B, T, _ = x.shape
    qkv, z, b, a = (F.linear(x, W(n)) for n in ("qkv", "z", "b", "a"))
    K = P["conv_w"].shape[1]
    pre = F.conv1d(qkv.transpose(1, 2), P["conv_w"][:, None, :], padding=K - 1, groups=qkv.shape[-1])[..., :T]
    c = F.silu(pre).transpose(1, 2)
    kd = Hk * Dk
    q = c[..., :kd].reshape(B, T, Hk, Dk)
    k = c[..., kd:2 * kd].reshape(B, T, Hk, Dk)
    v = c[..., 2 * kd:].reshape(B, T, Hv, Dv)
    q = q * (Dk ** -0.5) / torch.sqrt((q * q).sum(-1, keepdim=True) + eps)
    k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + eps)
    t = a + P["dt_bias"]
    sp = torch.where(t > 20, t, torch.log1p(torch.exp(torch.clamp(t, max=20.0))))
    decay = torch.exp(-torch.exp(P["A_log"]) * sp)
    beta = torch.sigmoid(b)
    y, _ = recurrence(q, k, v, decay, beta, x.new_zeros((B, Hv, Dv, Dk)))
    zh = z.reshape(B, T, Hv, Dv)
    n = y / torch.sqrt((y * y).mean(-1, keepdim=True) + eps)
    o = (n * P["norm_w"] * F.silu(zh)).reshape(B, T, Hv * Dv)
    return F.linear(o, W("out"))
