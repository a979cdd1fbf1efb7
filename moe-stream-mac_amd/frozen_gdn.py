"""Use the forward-only GDN path for frozen lower decoder layers (drop-in for ``tools/frozen_gdn.py``).

Layers below the first decoder layer with a trainable parameter need no gradient, so their GDN calls are
forced onto the inference path (``use_kernel=True``: forward-only HIP kernel, no snapshots, no autograd
node).  The marker is a ContextVar, so it is thread/task local and survives ``model.train()``
(``tools/frozen_gdn.py:12-36``).
"""

from __future__ import annotations

from contextvars import ContextVar
from typing import Any, Callable, Optional

import torch.nn as nn

import gdn_hf
import qwen3_5

MARKER = "_frozen_gdn_kernel"
_ACTIVE_MARKED_GDN: ContextVar[bool] = ContextVar("frozen_gdn_kernel_active", default=False)
_ORIGINAL_UPDATE: Optional[Callable[..., Any]] = None
_ORIGINAL_GDN_CALL: Optional[Callable[..., Any]] = None


def _marked_update(*args: Any, **kwargs: Any) -> Any:
    if _ORIGINAL_UPDATE is None:
        raise RuntimeError("frozen_gdn.install() has not patched the update")
    if _ACTIVE_MARKED_GDN.get():
        kwargs["use_kernel"] = True
    return _ORIGINAL_UPDATE(*args, **kwargs)


def _marked_gdn_call(module: nn.Module, *args: Any, **kwargs: Any) -> Any:
    if _ORIGINAL_GDN_CALL is None:
        raise RuntimeError("frozen_gdn.install() has not patched GatedDeltaNet")
    if not getattr(module, MARKER, False):
        return _ORIGINAL_GDN_CALL(module, *args, **kwargs)
    token = _ACTIVE_MARKED_GDN.set(True)
    hf_token = gdn_hf.FORCE_FORWARD_ONLY.set(True)
    try:
        return _ORIGINAL_GDN_CALL(module, *args, **kwargs)
    finally:
        gdn_hf.FORCE_FORWARD_ONLY.reset(hf_token)
        _ACTIVE_MARKED_GDN.reset(token)


def _decoder_layers(model: nn.Module) -> list[nn.Module]:
    if not isinstance(model, (qwen3_5.Model, qwen3_5.TextModel, qwen3_5.Qwen3_5TextModel)):
        raise TypeError("frozen_gdn supports only qwen3_5-family models")
    return list(model.layers)


def _has_trainable_parameters(module: nn.Module) -> bool:
    return any(p.requires_grad for p in module.parameters())


def _patch_qwen3_5() -> None:
    global _ORIGINAL_UPDATE, _ORIGINAL_GDN_CALL
    if qwen3_5.gated_delta_update is not _marked_update:
        _ORIGINAL_UPDATE = qwen3_5.gated_delta_update
        qwen3_5.gated_delta_update = _marked_update
    if qwen3_5.GatedDeltaNet.forward is not _marked_gdn_call:
        _ORIGINAL_GDN_CALL = qwen3_5.GatedDeltaNet.forward
        qwen3_5.GatedDeltaNet.forward = _marked_gdn_call


def install(model: nn.Module) -> None:
    """Mark frozen GDN layers below the first trainable decoder layer (tools/frozen_gdn.py:65-83)."""
    layers = _decoder_layers(model)
    if not _has_trainable_parameters(model):
        raise ValueError("frozen_gdn requires at least one trainable parameter")
    first_trainable = next(
        (index for index, layer in enumerate(layers) if _has_trainable_parameters(layer)), len(layers))
    _patch_qwen3_5()
    for index, layer in enumerate(layers):
        gdn = getattr(layer, "linear_attn", None)
        if isinstance(gdn, qwen3_5.GatedDeltaNet):
            setattr(gdn, MARKER, index < first_trainable)
