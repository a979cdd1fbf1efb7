"""Chunk-bounded forward + hand-written VJP of the Qwen3.5 Gated DeltaNet recurrence, on MI355X.

Drop-in for the reference's ``tools/gdn_vjp.py``: same public names, arguments, defaults, return tuples and
exceptions, on ``torch.Tensor`` living on a ROCm device.  Per step (``tools/gdn_vjp.py:3-6``)::

    A = S_prev * decay;  r = v - A @ k;  delta = beta * r;  S~ = A + k (x) delta;  y = S~ @ q
    S_t = mask ? S~ : S_prev

and the backward is the reverse-time adjoint of ``tools/gdn_vjp.py:8-21``.  All three ``impl`` strings run
the same HIP engine (``libgdn_mi355x.so``): the forward keeps one state snapshot per ``chunk`` tokens and
the backward recomputes the states inside each chunk, in registers, instead of storing them.
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


def gated_delta_chunked(
    q: Array,
    k: Array,
    v: Array,
    g: Array,
    beta: Array,
    state: Optional[Array] = None,
    mask: Optional[Array] = None,
    chunk: int = DEFAULT_CHUNK,
    impl: str = "staged",
    *,
    output_dtype: Optional[torch.dtype] = None,
) -> tuple[Array, Array]:
    """Run GDN with saved chunk boundaries and a hand-written reverse pass (tools/gdn_vjp.py:503-528).

    q, k ``[B,T,Hk,Dk]``; v ``[B,T,Hv,Dv]``; g the decay ``[B,T,Hv]`` or ``[B,T,Hv,Dk]``; beta
    ``[B,T,Hv]``; state ``[B,Hv,Dv,Dk]`` (fp32 zeros when None); mask ``[B,T]`` bool.
    Returns ``(y, final_state)``.  ``output_dtype`` (keyword only, not in the reference) overrides the
    dtype of ``y``, which otherwise follows the reference's promotion (fp32 with an fp32 state).
    """
    if chunk <= 0:
        raise ValueError("chunk must be a positive integer")
    if impl not in ("chunked", "staged", "kernel"):
        raise ValueError("impl must be 'chunked', 'staged', or 'kernel'")
    backward_error = None
    if impl == "kernel":
        # The reference's kernel impl accepts only these inputs, and checks them when the backward runs
        # (tools/gdn_vjp.py:391-394): a forward-only call with other inputs succeeds.
        if q.shape[-1] % 32:
            backward_error = "impl='kernel' requires key_dim divisible by 32"
        elif q.dtype != k.dtype or q.dtype != v.dtype:
            backward_error = "impl='kernel' requires q, k, and v to share a dtype"
    batch, _, _, key_dim = q.shape
    value_heads, value_dim = v.shape[-2:]
    if state is None:
        state = torch.zeros((batch, value_heads, value_dim, key_dim), dtype=torch.float32, device=q.device)
    return gdn_engine.recurrence(q, k, v, g, beta, state, mask, chunk, output_dtype=output_dtype,
                                 backward_error=backward_error)


def _vjp_update(
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
    """Drop-in for ``gated_delta_update`` (tools/gdn_vjp.py:531-563)."""
    if use_kernel:
        if _ORIGINAL_UPDATE is None:
            raise RuntimeError("gdn_vjp.install() has not been called")
        return _ORIGINAL_UPDATE(
            q, k, v, a, b, A_log, dt_bias, state, mask,
            use_kernel=use_kernel, lower_bound=lower_bound,
            allow_neg_eigval=allow_neg_eigval
        )
    g, beta = gated_delta.gates(a, b, A_log, dt_bias, allow_neg_eigval, lower_bound)
    # the reference picks the kernel impl by key_dim alone (tools/gdn_vjp.py:562)
    impl = "kernel" if q.shape[-1] % 32 == 0 else "staged"
    return gated_delta_chunked(q, k, v, g, beta, state, mask, impl=impl)


def install() -> None:
    """Patch Qwen3.5 training calls while preserving its inference update (tools/gdn_vjp.py:566-574).

    Rebinds ``qwen3_5.gated_delta_update`` (idempotently; the previous binding serves ``use_kernel=True``)
    and, when transformers is importable, HF Qwen3.5's module-level chunk rule.
    """
    global _ORIGINAL_UPDATE
    if qwen3_5.gated_delta_update is _vjp_update:
        return
    _ORIGINAL_UPDATE = qwen3_5.gated_delta_update
    gdn_hf.route_training_calls(_vjp_update, owner="gdn_vjp", chunk=DEFAULT_CHUNK)
