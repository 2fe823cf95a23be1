"""generate() hooks that put the paged KV cache under Hugging Face decoding.

Counterparts of the reference's ``_patch_generate_with_paged_kv`` and ``patch_inference``
(python/barqtrain/patch_models.py:235-261,319-329), the only parts of its model patching that
sit on the KV-cache path.  The wrapper records on the model whether the last ``generate`` call
ran on the paged cache (``_barqtrain_last_generate_used_paged_kv``), whether the model can
(``_barqtrain_paged_kv_supported``) and that it is wrapped
(``_barqtrain_generate_paged_kv_patched``).
"""

from __future__ import annotations

import os
import types
from typing import Optional

import torch


def _patch_generate_with_paged_kv(model: torch.nn.Module, model_label: str) -> torch.nn.Module:
    """Wrap ``model.generate`` so each call may receive a paged cache (idempotent)."""
    if getattr(model, "_barqtrain_generate_paged_kv_patched", False) or not hasattr(model, "generate"):
        return model

    # Looked up through the module at call time so they stay patchable.
    from barqtrain_amd import kv_cache

    inner_generate = model.generate

    def generate(self, *args, **kwargs):
        call_kwargs, used = kv_cache.maybe_prepare_paged_kv_generate_kwargs(self, args, kwargs)
        self._barqtrain_last_generate_used_paged_kv = used
        return inner_generate(*args, **call_kwargs)

    model.generate = types.MethodType(generate, model)
    model._barqtrain_generate_paged_kv_patched = True
    model._barqtrain_paged_kv_supported = kv_cache.paged_kv_supported_for_model(model)
    if model._barqtrain_paged_kv_supported:
        print(f"BarqTrain: Enabled paged KV-cache injection for {model_label}")
    return model


def _attention_backend() -> Optional[str]:
    """Attention implementation for decode: SDPA (on ROCm PyTorch it dispatches to the AMD
    flash / memory-efficient kernels); flash_attention_2 only if that package is importable."""
    import importlib.util

    if torch.cuda.is_available() and importlib.util.find_spec("flash_attn") is not None:
        return "flash_attention_2"
    if hasattr(torch.nn.functional, "scaled_dot_product_attention"):
        return "sdpa"
    return None


def _configure_attention_backend(model: torch.nn.Module, model_label: str) -> Optional[str]:
    config = getattr(model, "config", None)
    backend = _attention_backend()
    if config is None or backend is None:
        return None
    if getattr(config, "_attn_implementation", None) != backend:
        config._attn_implementation = backend
        if hasattr(config, "attn_implementation"):
            config.attn_implementation = backend
        print(f"BarqTrain: Enabled {backend} attention backend for {model_label}")
    return backend


def patch_inference(model: torch.nn.Module, paged_attention: Optional[bool] = None) -> torch.nn.Module:
    """Decode-time patches: attention backend choice plus the paged-cache generate hook.
    paged_attention (default: the BARQTRAIN_PAGED_ATTENTION switch, off) routes attention
    through "barq_paged", which reads K/V from the cache pages instead of a gathered copy."""
    label = getattr(getattr(model, "config", None), "model_type", None) or "model"
    if paged_attention is None:
        paged_attention = os.environ.get("BARQTRAIN_PAGED_ATTENTION", "0").strip().lower() in {"1", "true", "yes", "on"}
    if paged_attention and torch.cuda.is_available():
        from barqtrain_amd.attention import enable_paged_attention

        enable_paged_attention(model)
        print(f"BarqTrain: Enabled paged decode attention for {label}")
    else:
        _configure_attention_backend(model, label)
    return _patch_generate_with_paged_kv(model, label)


__all__ = ["patch_inference"]
