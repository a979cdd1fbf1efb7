"""Activation-checkpointed GDN recurrence for Qwen3.5, on MI355X.

Drop-in for the reference's ``tools/gdn_checkpoint.py``: the forward keeps only the state at every
``chunk``-th token and the backward recomputes each chunk from it (the contract of ``mx.checkpoint`` per
chunk, ``tools/gdn_checkpoint.py:39-50,81-95``).  The recompute runs inside the HIP backward kernel, so no
per-chunk autodiff graph is ever built.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Optional

import torch

import gated_delta
import gdn_engine
import gdn_hf
import qwen3_5

DEFAULT_CHUNK = 64
Array = torch.Tensor
UpdateFunction = Callable[..., tuple[Array, Array]]

_ORIGINAL_UPDATE: Optional[UpdateFunction] = None


def gated_delta_ops_checkpointed(
    q: Array,
    k: Array,
    v: Array,
    g: Array,
    beta: Array,
    state: Optional[Array] = None,
    mask: Optional[Array] = None,
    chunk: int = DEFAULT_CHUNK,
) -> tuple[Array, Array]:
    """Run the recurrence in checkpointed time chunks (tools/gdn_checkpoint.py:53-95).

    Inputs follow ``gated_delta_ops``; each chunk retains its entry state and is recomputed in backward.
    """
    if chunk <= 0:
        raise ValueError("chunk must be a positive integer")
    batch, timesteps, key_heads, key_dim = q.shape
    value_heads, value_dim = v.shape[-2:]
    if state is None:
        state = torch.zeros((batch, value_heads, value_dim, key_dim), dtype=torch.float32, device=q.device)
    return gdn_engine.recurrence(q, k, v, g, beta, state, mask, chunk)


def _checkpointed_update(
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
    """Drop-in for ``gated_delta_update`` on the checkpoint path (tools/gdn_checkpoint.py:98-142)."""
    if use_kernel:
        if _ORIGINAL_UPDATE is None:
            raise RuntimeError("gdn_checkpoint.install() has not been called")
        return _ORIGINAL_UPDATE(
            q, k, v, a, b, A_log, dt_bias, state, mask,
            use_kernel=use_kernel, lower_bound=lower_bound, allow_neg_eigval=allow_neg_eigval,
        )
    g, beta = gated_delta.gates(a, b, A_log, dt_bias, allow_neg_eigval, lower_bound)
    if state is None:
        batch, _, _, key_dim = q.shape
        value_heads, value_dim = v.shape[-2:]
        state = torch.zeros((batch, value_heads, value_dim, key_dim), dtype=torch.float32, device=q.device)
    return gated_delta_ops_checkpointed(q, k, v, g, beta, state, mask)


def install() -> None:
    """Patch Qwen3.5's imported update alias for its training path only (tools/gdn_checkpoint.py:145-153)."""
    global _ORIGINAL_UPDATE
    if qwen3_5.gated_delta_update is _checkpointed_update:
        return
    _ORIGINAL_UPDATE = qwen3_5.gated_delta_update
    gdn_hf.route_training_calls(_checkpointed_update, owner="gdn_checkpoint", chunk=DEFAULT_CHUNK)
