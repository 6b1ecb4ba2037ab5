"""Talker-side KV import and the audio-Q1 position counter.

The talker (Qwen3-TTS-shaped: 28 layers, 8 KV heads, head_dim 128, bf16)
prefills its prefix with HF and then decodes one codec frame per step from
native KV storage. These helpers take an HF ``DynamicCache`` into a
:class:`kvrt.cache.KVRTCache` and advance the per-response position counter:

* ``dynamic_cache_kv_layers`` — validate and borrow the exact bf16 layer
  tensors of an HF cache without casting or cloning
  (duplex_kernel/native_qwen_talker.py:350-392);
* ``import_dynamic_cache`` — reset the slot, then one kvrt import launch per
  layer (native_qwen_talker.py:781-874 -> qwen_talker.cu:1060-1110: memset
  of the arena, then the prefix copy);
* ``advance_audio_q1_position`` — next causal Q1 position, failing closed
  past the response budget (native_qwen_talker.py:395-401).
"""
from __future__ import annotations

from typing import Any

import torch

from .cache import KVRTCache

TALKER_NUM_LAYERS = 28
TALKER_NUM_KV_HEADS = 8
TALKER_HEAD_DIM = 128


def dynamic_cache_kv_layers(cache: Any, *, num_layers: int = TALKER_NUM_LAYERS,
                            kv_heads: int = TALKER_NUM_KV_HEADS, head_dim: int = TALKER_HEAD_DIM,
                            ) -> tuple[int, list[tuple[torch.Tensor, torch.Tensor]]]:
    """(sequence length, [(K, V)] per layer) of an HF cache, validated.

    Every layer must hold contiguous bf16 K and V of shape
    [1, kv_heads, S, head_dim] on one device, with S = ``get_seq_length()``
    >= 1. Raises ``ValueError`` otherwise; the returned tensors are the
    cache's own (no copy).
    """
    layers = getattr(cache, "layers", None)
    get_len = getattr(cache, "get_seq_length", None)
    if not isinstance(layers, (list, tuple)) or not callable(get_len):
        raise ValueError("talker cache must expose DynamicCache.layers and get_seq_length()")
    if len(layers) != num_layers:
        raise ValueError(f"talker DynamicCache must hold {num_layers} layers, got {len(layers)}")
    try:
        seq = int(get_len())
    except (TypeError, ValueError, RuntimeError) as exc:
        raise ValueError("talker DynamicCache has an invalid sequence length") from exc
    if seq <= 0:
        raise ValueError("talker DynamicCache must hold at least one prefix token")
    want = (1, kv_heads, seq, head_dim)
    out = []
    for i, layer in enumerate(layers):
        k, v = getattr(layer, "keys", None), getattr(layer, "values", None)
        if not isinstance(k, torch.Tensor) or not isinstance(v, torch.Tensor):
            raise ValueError(f"DynamicCache layer {i} holds no K/V tensors")
        if tuple(k.shape) != want or tuple(v.shape) != want:
            raise ValueError(f"unexpected DynamicCache shape at layer {i}: K={tuple(k.shape)} "
                             f"V={tuple(v.shape)} expected={want}")
        if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
            raise ValueError(f"DynamicCache layer {i} must be BF16")
        if k.device != v.device:
            raise ValueError(f"DynamicCache K/V on different devices at layer {i}")
        if not k.is_contiguous() or not v.is_contiguous():
            raise ValueError(f"DynamicCache layer {i} must be contiguous")
        out.append((k, v))
    return seq, out


def import_dynamic_cache(cache: Any, target: KVRTCache) -> int:
    """Import every layer of an HF talker cache into ``target`` (a KVRTCache
    whose runtime has the talker topology); returns the imported length."""
    rt = target.runtime
    spec = rt.layers[0]
    seq, layers = dynamic_cache_kv_layers(cache, num_layers=len(rt.layers), kv_heads=spec.kv_heads,
                                          head_dim=spec.head_dim)
    if seq > rt.capacity:
        raise ValueError(f"prefix of {seq} tokens exceeds the runtime capacity {rt.capacity}")
    for i, (k, v) in enumerate(layers):
        if not k.is_cuda:
            raise ValueError(f"DynamicCache layer {i} is not on the GPU (kvrt has no CPU path)")
    target.reset()
    for i, (k, v) in enumerate(layers):
        if rt._owner(i) == i:
            rt.import_(target.slot, i, k, v)
    target.adopt()
    return seq


def advance_audio_q1_position(current_position: int, limit_position: int) -> int:
    """The next Q1 position; ``RuntimeError`` once the response budget is spent."""
    current_position, limit_position = int(current_position), int(limit_position)
    if current_position < 0 or limit_position <= current_position:
        raise RuntimeError("audio frame limit of the response reached")
    return current_position + 1


__all__ = ["TALKER_HEAD_DIM", "TALKER_NUM_KV_HEADS", "TALKER_NUM_LAYERS", "advance_audio_q1_position",
           "dynamic_cache_kv_layers", "import_dynamic_cache"]
