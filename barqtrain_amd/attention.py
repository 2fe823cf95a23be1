"""Attention that reads K and V from the paged cache's pages, as a transformers attention
implementation (``"barq_paged"``).

A ``BarqPagedKVCache`` built with ``fused_attention=True`` appends in ``update`` and returns, in
place of materialised K/V, zero-stride views that name their cache layer.  The attention
function registered here finds the layer on the key view and, for decode (``G * T <= 16`` query
rows per kv head, no padding mask, head_dim 64, 128 or 256), runs the pool's decode-attention kernel:
softmax(Q K^T) V is computed from the pages through the block table, so the per-step gather of
the whole history (and its write and re-read) disappears.  Prefill, padded batches and other
head sizes take the gathered K/V through torch's fused SDPA kernels (flash or memory-efficient,
grouped-query heads without copies, bottom-right causal); host tensors, and shapes no fused
kernel takes, an fp32 attention.  Calls without a paged cache go to transformers' SDPA path.
Layers with options the kernel does not implement -- logit soft-capping (Gemma 2), attention
sinks (``s_aux``, gpt-oss), dropout, or a sliding window that cuts the row -- attend over the
gathered K/V: a sliding window alone (whose mask transformers builds) through fused SDPA, the
others through the fp32 attention, which applies each option as the models' own attention does.

The kernel's numbers are fp32 throughout (scores from exact bf16/fp16 products, fp32 softmax and
P.V), so logits track an fp32 reference more closely than the default bf16 attention does.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

ATTN_IMPLEMENTATION = "barq_paged"
_KERNEL_MAX_ROWS = 16


def paged_kv_view(layer, like: torch.Tensor, seq: int) -> torch.Tensor:
    """A ``[batch, kv_heads, seq, head_dim]`` zero-stride view carrying the cache layer."""
    base = getattr(layer, "_fused_base", None)
    if base is None or base.dtype != like.dtype or base.device != like.device:
        base = torch.zeros((), dtype=like.dtype, device=like.device)
        layer._fused_base = base
    view = base.expand(like.shape[0], like.shape[1], seq, like.shape[3])
    view._barq_paged_layer = layer
    return view


def _fp32_attention(query, key, value, attention_mask, scale, softcap=None, sinks=None, sliding_window=None,
                    dropout=0.0):
    """Reference-precision attention over gathered K/V: q [B, Hq, T, D], k/v [B, Hkv, S, D];
    bottom-right causal when no mask is given; returns [B, T, Hq, D] in the query's dtype.
    Options as the models that use them apply them: `softcap` caps the scaled scores to
    softcap * tanh(s / softcap) before the mask (Gemma 2); `sinks` [Hq] is one extra logit per
    head that takes part in the softmax and is then dropped (gpt-oss); `sliding_window` W lets
    query position q see key positions k with q - W < k <= q (transformers' sliding-window
    overlay); `dropout` drops probabilities (training only)."""
    B, Hq, T, D = query.shape
    group = Hq // key.shape[1]
    q = query.float()
    k = key.float().repeat_interleave(group, dim=1)
    v = value.float().repeat_interleave(group, dim=1)
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    if softcap is not None:
        scores = torch.tanh(scores / softcap) * softcap
    S = k.shape[2]
    pos = torch.arange(S, device=q.device)
    qpos = S - T + torch.arange(T, device=q.device)
    if attention_mask is None:
        scores = scores.masked_fill(pos[None, :] > qpos[:, None], float("-inf"))
    elif attention_mask.dtype == torch.bool:
        scores = scores.masked_fill(~attention_mask[..., :S], float("-inf"))
    else:
        scores = scores + attention_mask[..., :S].float()
    if sliding_window is not None:
        scores = scores.masked_fill(pos[None, :] <= qpos[:, None] - sliding_window, float("-inf"))
    if sinks is not None:
        sink = sinks.float().to(q.device).reshape(1, Hq, 1, 1).expand(B, Hq, T, 1)
        probs = torch.softmax(torch.cat([scores, sink], dim=-1), dim=-1)[..., :-1]
    else:
        probs = torch.softmax(scores, dim=-1).nan_to_num(0.0)
    if dropout:
        probs = F.dropout(probs, p=dropout, training=True)
    return torch.matmul(probs, v).transpose(1, 2).contiguous().to(query.dtype)


def _sdpa_attention(query, key, value, attention_mask, scale):
    """Fused SDPA over gathered K/V (q [B, Hq, T, D], k/v [B, Hkv, S, D]) with the same masking
    as _fp32_attention; returns [B, T, Hq, D], or None when no fused kernel takes the shapes.
    Only the flash and memory-efficient kernels are allowed: the math fallback runs batched
    bf16 products over transposed views."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from torch.nn.attention.bias import causal_lower_right

    T, S = query.shape[2], key.shape[2]
    if attention_mask is None:
        mask = causal_lower_right(T, S) if T > 1 else None
    elif attention_mask.dtype == torch.bool:
        mask = attention_mask[..., :S]
    else:
        mask = attention_mask[..., :S].to(query.dtype)
    group = query.shape[1] // key.shape[1]
    # Grouped heads natively where a kernel takes them (ROCm's fused kernels do not with a mask),
    # else K/V expanded to the query heads.
    attempts = (True, False) if attention_mask is None else (False,)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        for gqa in attempts:
            k, v = (key, value) if gqa or group == 1 else (key.repeat_interleave(group, 1),
                                                         value.repeat_interleave(group, 1))
            try:
                out = F.scaled_dot_product_attention(query, k, v, attn_mask=mask, scale=scale,
                                                     enable_gqa=gqa and group > 1)
            except RuntimeError:
                continue
            return out.transpose(1, 2).contiguous()
    return None


def _gathered_attention(query, key, value, attention_mask, scale):
    if query.is_cuda and query.dtype in (torch.bfloat16, torch.float16):
        out = _sdpa_attention(query, key, value, attention_mask, scale)
        if out is not None:
            return out
    return _fp32_attention(query, key, value, attention_mask, scale)


def paged_attention_forward(module: torch.nn.Module, query: torch.Tensor, key: torch.Tensor,
                            value: torch.Tensor, attention_mask: Optional[torch.Tensor],
                            scaling: Optional[float] = None, dropout: float = 0.0, **kwargs):
    """transformers attention interface: returns ``(attn_output [B, T, Hq, D], None)``."""
    layer = getattr(key, "_barq_paged_layer", None)
    if layer is None:
        from transformers.integrations.sdpa_attention import sdpa_attention_forward

        return sdpa_attention_forward(module, query, key, value, attention_mask, scaling=scaling,
                                      dropout=dropout, **kwargs)
    softcap, sinks, window = kwargs.get("softcap"), kwargs.get("s_aux"), kwargs.get("sliding_window")
    if not module_training(module):
        dropout = 0.0
    # A window cuts the row only when some query sees fewer positions than it holds.
    window_cuts = window is not None and key.shape[2] > int(window)
    options = softcap is not None or sinks is not None or bool(dropout)
    pool = layer.pool
    _, q_heads, tokens, head_dim = query.shape
    scale = scaling if scaling is not None else 1.0 / math.sqrt(head_dim)
    rows = (q_heads // pool.kv_heads) * tokens
    kernel_ok = (not options and not window_cuts and attention_mask is None and rows <= _KERNEL_MAX_ROWS
                 and pool.on_gpu and (not getattr(pool, "quantized", False) or pool.page_size % 16 == 0)
                 and pool.dtype in (torch.bfloat16, torch.float16) and pool.head_dim in (64, 128, 256))
    if kernel_ok:
        return pool.attend(query, scale).transpose(1, 2), None
    k, v = layer.current_tensors()
    if options or (window_cuts and attention_mask is None):
        return _fp32_attention(query, k, v, attention_mask, scale, softcap=softcap, sinks=sinks,
                               sliding_window=window if window_cuts else None, dropout=dropout), None
    # no option, or a window that the mask transformers built already applies
    return _gathered_attention(query, k, v, attention_mask, scale), None


def module_training(module) -> bool:
    """Dropout applies while the attention module trains (as in the models' own attention)."""
    return bool(getattr(module, "training", False))


def register() -> str:
    """Make ``"barq_paged"`` a transformers attention implementation (idempotent); its masks are
    built like SDPA's (none for an unpadded decode step)."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

    AttentionInterface.register(ATTN_IMPLEMENTATION, paged_attention_forward)
    AttentionMaskInterface.register(ATTN_IMPLEMENTATION, sdpa_mask)
    return ATTN_IMPLEMENTATION


def enable_paged_attention(model: torch.nn.Module) -> torch.nn.Module:
    """Route the model's attention through ``"barq_paged"`` and mark it so that paged caches
    created for its generate() calls return page views instead of gathered K/V."""
    register()
    config = getattr(model, "config", None)
    if config is not None:
        config._attn_implementation = ATTN_IMPLEMENTATION
    model._barqtrain_paged_attention = True
    return model


__all__ = ["ATTN_IMPLEMENTATION", "enable_paged_attention", "paged_attention_forward", "register"]
