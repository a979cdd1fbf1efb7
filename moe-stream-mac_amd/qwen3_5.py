"""Torch Qwen3.5 model pieces around the GDN hot path: the module whose global ``gated_delta_update`` the
``install()`` functions rebind, exactly as the reference rebinds ``mlx_lm.models.qwen3_5.gated_delta_update``
(``tools/gdn_vjp.py:566-574``, ``tools/gdn_checkpoint.py:145-153``, ``tools/frozen_gdn.py:54-62``).

``GatedDeltaNet`` follows the order of one GDN block in ``engine/include/gdn_layer.h:31-43``: in-projections
-> causal depthwise conv1d + SiLU -> split q/k/v -> q/k L2 norm -> gates -> recurrence -> gated RMSNorm *
SiLU(z) -> out-projection.  The recurrence call resolves ``gated_delta_update`` from this module's globals
at call time with ``use_kernel=not self.training`` (the mlx-lm call site, ``qwen3_5.py:183-193``).

``TextModel`` / ``Model`` are small decoder stacks (GDN or causal attention mixer + SwiGLU MLP) used to
exercise install()/frozen-layer dispatch and LoRA gradients; the MoE and full-attention details of the real
model are outside the GDN path and are not modelled.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

import gdn_block
from gated_delta import gated_delta_update, normalize_qk  # noqa: F401  (rebound by install())

Array = torch.Tensor


@dataclass
class ModelArgs:
    hidden_size: int = 64
    intermediate_size: int = 128
    num_hidden_layers: int = 4
    num_attention_heads: int = 4
    vocab_size: int = 1000
    rms_norm_eps: float = 1e-6
    linear_num_value_heads: int = 4
    linear_num_key_heads: int = 2
    linear_key_head_dim: int = 8
    linear_value_head_dim: int = 8
    linear_conv_kernel_dim: int = 4
    full_attention_interval: int = 2
    layer_types: list = field(default_factory=list)

    def __post_init__(self):
        if not self.layer_types:
            self.layer_types = [
                "full_attention" if (i + 1) % self.full_attention_interval == 0 else "linear_attention"
                for i in range(self.num_hidden_layers)]


class RMSNormGated(nn.Module):
    """rmsnorm(y) * w * silu(z) over the value head dim, eps 1e-6 (engine/src/gdn_layer.c:47-55)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, y: Array, z: Array) -> Array:
        return gdn_block.gated_rmsnorm(y, z, self.weight, self.eps)


class GatedDeltaNet(nn.Module):
    def __init__(self, args: ModelArgs):
        super().__init__()
        self.Hk, self.Hv = args.linear_num_key_heads, args.linear_num_value_heads
        self.Dk, self.Dv = args.linear_key_head_dim, args.linear_value_head_dim
        self.key_dim, self.value_dim = self.Hk * self.Dk, self.Hv * self.Dv
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.K = args.linear_conv_kernel_dim
        h = args.hidden_size
        self.in_proj_qkv = nn.Linear(h, self.conv_dim, bias=False)
        self.in_proj_z = nn.Linear(h, self.value_dim, bias=False)
        self.in_proj_b = nn.Linear(h, self.Hv, bias=False)
        self.in_proj_a = nn.Linear(h, self.Hv, bias=False)
        self.conv1d = nn.Conv1d(self.conv_dim, self.conv_dim, self.K, groups=self.conv_dim, bias=False,
                                padding=self.K - 1)
        self.A_log = nn.Parameter(torch.log(torch.empty(self.Hv).uniform_(1.0, 16.0)))
        self.dt_bias = nn.Parameter(torch.zeros(self.Hv))
        self.norm = RMSNormGated(self.Dv, args.rms_norm_eps)
        self.out_proj = nn.Linear(self.value_dim, h, bias=False)

    def forward(self, x: Array, mask: Optional[Array] = None, cache: Optional["GDNCache"] = None) -> Array:
        """x [B, T, hidden] -> [B, T, hidden].  With a cache (mlx-lm's two-entry cache: the conv state, then the
        recurrent state) the call continues the sequences the cache holds and leaves their states after x in it:
        a prefill, then one call per decoded token."""
        B, T, _ = x.shape
        projs = (self.in_proj_qkv, self.in_proj_z, self.in_proj_b, self.in_proj_a)
        if all(isinstance(m, LoRALinear) and m.base.bias is None for m in projs):
            qkv, z, b, a = lora_group(x, projs)  # the four adapters share one pass over x
        else:
            qkv, z, b, a = (m(x) for m in projs)
        z = z.reshape(B, T, self.Hv, self.Dv)
        if mask is not None:
            qkv = qkv * mask[..., None].to(qkv.dtype)
        # conv + SiLU, split, per-head q/k L2 norm (q scaled by Dk^-1/2): one fused kernel pair
        conv_state = None if cache is None else cache[0]
        q, k, v, *conv_next = gdn_block.conv_qkv(qkv, self.conv1d.weight, self.Hk, self.Dk, self.Hv, self.Dv,
                                                 self.Dk ** -0.5, 1e-6, state=conv_state,
                                                 return_state=cache is not None)
        update = globals()["gated_delta_update"]
        state = None if cache is None else cache[1]
        out, state_next = update(q, k, v, a, b, self.A_log, self.dt_bias, state, mask,
                                 use_kernel=not self.training)
        if cache is not None:
            cache[0], cache[1] = conv_next[0], state_next
        out = self.norm(out.to(z.dtype), z)
        return self.out_proj(out.reshape(B, T, -1))


class GDNCache:
    """Decode state of one GatedDeltaNet layer, indexed like mlx-lm's ArraysCache(2): [0] the conv state
    [B, K-1, conv_dim] fp32 (the last K-1 conv inputs, oldest first), [1] the recurrent state [B, Hv, Dv, Dk] fp32.
    Both start as None (zeros)."""

    def __init__(self):
        self.entries: list[Optional[Array]] = [None, None]

    def __getitem__(self, i: int) -> Optional[Array]:
        return self.entries[i]

    def __setitem__(self, i: int, value: Optional[Array]) -> None:
        self.entries[i] = value


class KVCache:
    """Keys and values seen so far by one Attention layer, [B, T_past, heads, head_dim] each."""

    def __init__(self):
        self.k: Optional[Array] = None
        self.v: Optional[Array] = None


class Attention(nn.Module):
    """Plain causal softmax attention standing in for the full-attention layers."""

    def __init__(self, args: ModelArgs):
        super().__init__()
        h = args.hidden_size
        self.nh = args.num_attention_heads
        self.qkv = nn.Linear(h, 3 * h, bias=False)
        self.o_proj = nn.Linear(h, h, bias=False)

    def forward(self, x: Array, mask: Optional[Array] = None, cache: Optional[KVCache] = None) -> Array:
        B, T, H = x.shape
        q, k, v = self.qkv(x).float().reshape(B, T, 3, self.nh, H // self.nh).unbind(2)
        past = 0
        if cache is not None:
            if cache.k is not None:
                past = cache.k.shape[1]
                k, v = torch.cat([cache.k, k], 1), torch.cat([cache.v, v], 1)
            cache.k, cache.v = k, v
        att = torch.einsum("bqhd,bkhd->bhqk", q, k) / math.sqrt(H // self.nh)
        causal = torch.ones(T, past + T, dtype=torch.bool, device=x.device).tril(past)
        att = att.masked_fill(~causal, float("-inf")).softmax(-1)
        out = torch.einsum("bhqk,bkhd->bqhd", att, v).reshape(B, T, H).to(x.dtype)
        return self.o_proj(out)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: Array) -> Array:
        xf = x.float()
        return (xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + self.eps) * self.weight).to(x.dtype)


class DecoderLayer(nn.Module):
    def __init__(self, args: ModelArgs, layer_type: str):
        super().__init__()
        self.is_linear = layer_type == "linear_attention"
        if self.is_linear:
            self.linear_attn = GatedDeltaNet(args)
        else:
            self.self_attn = Attention(args)
        h = args.hidden_size
        self.input_layernorm = RMSNorm(h, args.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(h, args.rms_norm_eps)
        self.gate_up = nn.Linear(h, 2 * args.intermediate_size, bias=False)
        self.down = nn.Linear(args.intermediate_size, h, bias=False)

    def make_cache(self):
        return GDNCache() if self.is_linear else KVCache()

    def forward(self, x: Array, mask: Optional[Array] = None, cache=None) -> Array:
        mixer = self.linear_attn if self.is_linear else self.self_attn
        x = x + mixer(self.input_layernorm(x), mask, cache)
        gate, up = self.gate_up(self.post_attention_layernorm(x)).chunk(2, dim=-1)
        return x + self.down(F.silu(gate) * up)


class TextModel(nn.Module):
    def __init__(self, args: ModelArgs):
        super().__init__()
        self.args = args
        self.embed_tokens = nn.Embedding(args.vocab_size, args.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(args, t) for t in args.layer_types)
        self.norm = RMSNorm(args.hidden_size, args.rms_norm_eps)

    def make_cache(self) -> list:
        """One cache per decoder layer (GDNCache for linear attention, KVCache for attention)."""
        return [layer.make_cache() for layer in self.layers]

    def forward(self, tokens: Array, mask: Optional[Array] = None, cache: Optional[list] = None) -> Array:
        x = self.embed_tokens(tokens)
        for i, layer in enumerate(self.layers):
            x = layer(x, mask, None if cache is None else cache[i])
        return self.norm(x)


class Model(nn.Module):
    def __init__(self, args: ModelArgs):
        super().__init__()
        self.model = TextModel(args)
        self.lm_head = nn.Linear(args.hidden_size, args.vocab_size, bias=False)

    @property
    def layers(self):
        return self.model.layers

    def make_cache(self) -> list:
        return self.model.make_cache()

    def forward(self, tokens: Array, mask: Optional[Array] = None, cache: Optional[list] = None) -> Array:
        return self.lm_head(self.model(tokens, mask, cache))


Qwen3_5TextModel = TextModel


def _mm(a: Array, b: Array, alpha: float = 1.0) -> Array:
    """alpha * a @ b with alpha applied inside the GEMM (one rounding)."""
    if alpha == 1.0:
        return a @ b
    return torch.addmm(a.new_empty(a.shape[0], b.shape[1]), a, b, beta=0, alpha=alpha)


class _LoRAGroupFn(torch.autograd.Function):
    """y_i = x W_i^T + s_i (x A_i^T) B_i^T for LoRA projections i that share the input x, with no pass of its own
    over any [tokens, features] tensor: the adapters' A products come from one GEMM over x, each adapter GEMM
    accumulates into its base output in place, and the backward accumulates dx in one buffer (beta = 1 GEMMs)
    and takes every dA from one GEMM over x.  Arguments: x, the scales, then W_i, A_i, B_i per projection."""

    @staticmethod
    def forward(ctx, x: Array, scales: tuple, *wab: Array):
        n = len(scales)
        Ws, As, Bs = wab[0::3], wab[1::3], wab[2::3]
        x2 = x.reshape(-1, x.shape[-1])
        ranks = tuple(a.shape[0] for a in As)
        a_cat = torch.cat(As) if n > 1 else As[0]
        u = x2 @ a_cat.t()  # [tokens, sum of ranks]
        outs, o = [], 0
        for W, B, s, r in zip(Ws, Bs, scales, ranks):
            y = x2 @ W.t()
            y.addmm_(u[:, o:o + r], B.t(), alpha=s)
            outs.append(y.view(*x.shape[:-1], W.shape[0]))
            o += r
        ctx.scales, ctx.ranks, ctx.xshape = scales, ranks, x.shape
        ctx.save_for_backward(x2, u, a_cat, *Ws, *Bs)
        return tuple(outs)

    @staticmethod
    def backward(ctx, *dys: Array):
        x2, u, a_cat, *rest = ctx.saved_tensors
        n = len(ctx.scales)
        Ws, Bs = rest[:n], rest[n:]
        need = ctx.needs_input_grad  # x, scales, then W_i, A_i, B_i
        grads: list = [None] * (3 * n)
        dx, du_parts, o = None, [], 0
        for i, (dy, W, B, s, r) in enumerate(zip(dys, Ws, Bs, ctx.scales, ctx.ranks)):
            if dy is None:
                du_parts.append(u.new_zeros(u.shape[0], r))
                o += r
                continue
            dy2 = dy.reshape(-1, dy.shape[-1])
            if need[0]:
                if dx is None:
                    dx = dy2 @ W
                else:
                    dx.addmm_(dy2, W)
            if need[2 + 3 * i]:
                grads[3 * i] = dy2.t() @ x2
            if need[4 + 3 * i]:
                grads[3 * i + 2] = _mm(dy2.t(), u[:, o:o + r], s)
            du_parts.append(_mm(dy2, B, s))
            o += r
        du = torch.cat(du_parts, 1) if n > 1 else du_parts[0]  # s_i (dy_i B_i), [tokens, sum of ranks]
        if need[0]:
            if dx is None:
                dx = du @ a_cat
            else:
                dx.addmm_(du, a_cat)
        if any(need[3 + 3 * i] for i in range(n)):
            da = du.t() @ x2
            o = 0
            for i, r in enumerate(ctx.ranks):
                if need[3 + 3 * i]:
                    grads[3 * i + 1] = da[o:o + r]
                o += r
        return (dx.view(ctx.xshape) if dx is not None else None, None, *grads)


def lora_group(x: Array, mods) -> tuple:
    """The outputs of LoRALinear modules without bias that share the input x (see _LoRAGroupFn)."""
    wab = []
    for m in mods:
        wab += [m.base.weight.to(x.dtype), m.lora_a.to(x.dtype), m.lora_b.to(x.dtype)]
    return _LoRAGroupFn.apply(x, tuple(float(m.scale) for m in mods), *wab)


class LoRALinear(nn.Module):
    """y = W x + scale * B(A x) with A ~ N(0, std), B = 0; W frozen."""

    def __init__(self, base: nn.Linear, rank: int, scale: float, std: float = 0.02):
        super().__init__()
        self.base = base
        self.base.weight.requires_grad_(False)
        self.lora_a = nn.Parameter(torch.randn(rank, base.in_features) * std)
        self.lora_b = nn.Parameter(torch.zeros(base.out_features, rank))
        self.scale = scale

    @property
    def weight(self):
        return self.base.weight

    def forward(self, x: Array) -> Array:
        if self.base.bias is None:
            return lora_group(x, (self,))[0]
        u = F.linear(x, self.lora_a.to(x.dtype)).flatten(0, -2)
        y = torch.addmm(self.base(x).flatten(0, -2), u, self.lora_b.to(x.dtype).t(), alpha=self.scale)
        return y.view(*x.shape[:-1], y.shape[-1])


def freeze(module: nn.Module) -> None:
    for p in module.parameters():
        p.requires_grad_(False)


def linear_to_lora_layers(model: Model, num_layers: int, rank: int = 2, scale: float = 2.0) -> None:
    """Freeze the model and put LoRA adapters on every Linear of the last ``num_layers`` decoder layers
    (the convention of mlx_lm.tuner.utils.linear_to_lora_layers used by the reference tests)."""
    freeze(model)
    for layer in list(model.layers)[-num_layers:]:
        for name, mod in list(layer.named_modules()):
            for child_name, child in list(mod.named_children()):
                if isinstance(child, nn.Linear):
                    setattr(mod, child_name, LoRALinear(child, rank, scale))
