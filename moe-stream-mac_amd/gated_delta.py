"""Torch counterpart of the mlx-lm ``gated_delta`` functions the reference builds on (third-party
``mlx_lm/models/gated_delta.py``: ``compute_g``, ``gated_delta_ops``, ``gated_delta_update``; call sites
``tools/gdn_vjp.py:194,558``, ``tools/gdn_checkpoint.py:32,135``), running on the HIP engine.

``gated_delta_update`` is the un-patched update bound into ``qwen3_5``: ``use_kernel=True`` is the
forward-only inference path (no snapshots, no autograd graph), ``use_kernel=False`` the differentiable
recurrence.  The arithmetic is the per-step rule of ``engine/include/gdn.h:27-38`` (``engine/src/gdn.c:63-108``).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

import gdn_block
import gdn_engine

Array = torch.Tensor


def compute_g(A_log: Array, a: Array, dt_bias: Array) -> Array:
    """Multiplicative decay exp(-exp(A_log) * softplus(a + dt_bias)) (engine/include/gdn.h:20-25), float32,
    on the fused gates kernel."""
    return gdn_block.gates(a, a, A_log, dt_bias)[0]


def gates(a: Array, b: Array, A_log: Array, dt_bias: Array, allow_neg_eigval: bool = False,
          lower_bound: float | None = None) -> tuple[Array, Array]:
    """(decay, beta) of the update functions (tools/gdn_vjp.py:554-558): beta = sigmoid(b), x2 when
    allow_neg_eigval; decay = compute_g(A_log, a, dt_bias).  One fused HIP kernel forward and backward."""
    if lower_bound is not None:
        raise NotImplementedError("lower_bound gates are not supported by this engine")
    return gdn_block.gates(a, b, A_log, dt_bias, allow_neg_eigval=allow_neg_eigval)


def normalize_qk(q: Array, k: Array, inv_scale: float, eps: float = 1e-6) -> tuple[Array, Array]:
    """q <- inv_scale * q / sqrt(sum q^2 + eps), k <- k / sqrt(sum k^2 + eps) (engine/include/gdn.h:17-18,
    engine/src/gdn_layer.c:35-39), on the L2-norm kernel."""
    return gdn_block.normalize_qk(q, k, inv_scale, eps)


def _default_state(q: Array, v: Array, state: Optional[Array]) -> Array:
    if state is not None:
        return state
    B, _, _, Dk = q.shape
    Hv, Dv = v.shape[-2:]
    return torch.zeros((B, Hv, Dv, Dk), dtype=torch.float32, device=q.device)


def gated_delta_ops(q: Array, k: Array, v: Array, g: Array, beta: Array, state: Optional[Array] = None,
                    mask: Optional[Array] = None) -> tuple[Array, Array]:
    """Differentiable recurrence over the whole sequence (the ops loop the reference tests compare with)."""
    return gdn_engine.recurrence(q, k, v, g, beta, _default_state(q, v, state), mask, chunk=64)


def gated_delta_kernel(q: Array, k: Array, v: Array, g: Array, beta: Array, state: Optional[Array] = None,
                       mask: Optional[Array] = None) -> tuple[Array, Array]:
    """Forward-only recurrence (inference kernel; used for frozen layers, tools/frozen_gdn.py:19-25)."""
    return gdn_engine.recurrence(q, k, v, g, beta, _default_state(q, v, state), mask, chunk=64,
                                 need_grad=False)


def gated_delta_update(
    q: Array,
    k: Array,
    v: Array,
    a: Array,
    b: Array,
    A_log: Array,
    dt_bias: Array,
    state: Optional[Array] = None,
    mask: Optional[Array] = None,
    *,
    use_kernel: bool = True,
    lower_bound: float | None = None,
    allow_neg_eigval: bool = False,
) -> tuple[Array, Array]:
    """Gates from (a, b, A_log, dt_bias), then the recurrence (mlx-lm ``gated_delta_update`` contract)."""
    g, beta = gates(a, b, A_log, dt_bias, allow_neg_eigval, lower_bound)
    if use_kernel:
        return gated_delta_kernel(q, k, v, g, beta, state, mask)
    return gated_delta_ops(q, k, v, g, beta, state, mask)


def l2_inv_scale(dim: int) -> float:
    return 1.0 / math.sqrt(dim)
