"""Routing of model-side GDN calls to the engine, shared by ``gdn_vjp.install`` and
``gdn_checkpoint.install``.

Two targets are rebound, both module globals resolved at call time:

* ``qwen3_5.gated_delta_update`` in this package (the mlx-lm contract the reference patches,
  ``tools/gdn_vjp.py:566-574``);
* ``torch_chunk_gated_delta_rule`` in the HF ``transformers`` Qwen3.5 modeling modules, when they are
  importable, through an adapter that converts their convention (log-space gate, q/k normalised inside,
  state ``[B,H,Dk,Dv]``) to this engine's.  The single-token decode rule is left untouched, as the
  reference leaves the inference update untouched.
"""

from __future__ import annotations

import contextvars
import importlib
from typing import Any, Callable, Optional

import torch

import gated_delta
import gdn_engine
import qwen3_5

original_update = gated_delta.gated_delta_update

_HF_MODULES = ("transformers.models.qwen3_5.modeling_qwen3_5",
               "transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
_HF_ORIGINALS: dict[str, Callable] = {}
_ROUTE: dict[str, Any] = {"owner": None, "chunk": 64}

# Set while a frozen (forward-only) GDN layer runs; see frozen_gdn.
FORCE_FORWARD_ONLY: contextvars.ContextVar[bool] = contextvars.ContextVar("gdn_force_forward_only",
                                                                          default=False)


def _hf_chunk_rule(query, key, value, g, beta, chunk_size=64, initial_state=None, output_final_state=False,
                   use_qk_l2norm_in_kernel=False, **kwargs):
    """HF ``torch_chunk_gated_delta_rule`` signature on the HIP engine (HF modeling_qwen3_5.py:248-327)."""
    if kwargs.get("cu_seqlens") is not None:
        raise NotImplementedError("packed sequences (cu_seqlens) are not supported by the GDN engine")
    Dk = query.shape[-1]
    if use_qk_l2norm_in_kernel:
        query, key = gated_delta.normalize_qk(query, key, Dk ** -0.5, 1e-6)
    else:
        query = query * (Dk ** -0.5)
    B, T, H, _ = query.shape
    Dv = value.shape[-1]
    state = (torch.zeros((B, H, Dv, Dk), dtype=torch.float32, device=query.device) if initial_state is None
             else initial_state.transpose(-1, -2))
    y, S = gdn_engine.recurrence(query, key, value, g, beta, state, None, chunk=_ROUTE["chunk"],
                                 log_gate=True, output_dtype=query.dtype,
                                 need_grad=False if FORCE_FORWARD_ONLY.get() else None)
    return y, (S.transpose(-1, -2) if output_final_state else None)


def _hf_modules() -> list:
    mods = []
    for name in _HF_MODULES:
        try:
            mods.append(importlib.import_module(name))
        except Exception:
            continue
    return mods


def route_training_calls(update: Callable, owner: str, chunk: int = 64) -> None:
    """Rebind ``qwen3_5.gated_delta_update`` to ``update`` and HF's chunk rule to the engine adapter."""
    if qwen3_5.gated_delta_update is not update:
        qwen3_5.gated_delta_update = update
    _ROUTE["owner"] = owner
    _ROUTE["chunk"] = chunk
    for mod in _hf_modules():
        if getattr(mod, "torch_chunk_gated_delta_rule", None) is not _hf_chunk_rule:
            _HF_ORIGINALS[mod.__name__] = mod.torch_chunk_gated_delta_rule
            mod.torch_chunk_gated_delta_rule = _hf_chunk_rule


def hf_original(module_name: str) -> Optional[Callable]:
    return _HF_ORIGINALS.get(module_name)
