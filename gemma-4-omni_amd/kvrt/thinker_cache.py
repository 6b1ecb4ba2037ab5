"""Exact token-prefix reuse for the thinker cache, with the copy on kvrt kernels.

Same names and behaviour as the reference module
``duplex_kernel/thinker_cache.py`` (andr-lab/gemma-4-omni): the longest
common prefix of two token-id sequences decides how many committed positions
a new decode branch can reuse; those positions are copied into a fresh,
empty cache of the same physical shape, and every layer's length is set to
the copied count. Validation fails closed with ``CachePrefixCopyError``
before anything is copied.

Two cache kinds are accepted:

* transformers ``StaticCache`` objects whose layers are full-attention
  ``StaticLayer`` instances on the GPU (the reference's only kind): the K/V
  rows move with the kvrt row-copy kernel;
* :class:`kvrt.cache.KVRTCache` slots of one runtime: one kvrt prefix-copy
  launch per layer.

``select_audio_thinker_cache_bucket`` (duplex_kernel/engine.py:588-630) picks
the static capacity a branch is created with.
"""
from __future__ import annotations

from dataclasses import dataclass
from numbers import Integral
from typing import Sequence

import torch

from .cache import KVRTCache
from .runtime import copy_rows


class CachePrefixCopyError(RuntimeError):
    """The cache pair does not satisfy the prefix-copy contract."""


@dataclass(frozen=True)
class CachePrefixCopyResult:
    copied_tokens: int
    copied_bytes: int
    layer_count: int


def longest_common_prefix_length(left: Sequence[int], right: Sequence[int]) -> int:
    """Number of leading token ids equal in both sequences.
    Reference: duplex_kernel/thinker_cache.py:28-34."""
    n = 0
    for a, b in zip(left, right):
        if int(a) != int(b):
            break
        n += 1
    return n


def _cache_length(cache: object) -> int:
    fn = getattr(cache, "get_seq_length", None)
    if not callable(fn):
        raise CachePrefixCopyError("cache has no get_seq_length()")
    try:
        value = fn()
    except Exception as exc:  # fail closed on any read error
        raise CachePrefixCopyError(f"get_seq_length() failed: {exc}") from exc
    if isinstance(value, torch.Tensor):
        if value.numel() != 1:
            raise CachePrefixCopyError("get_seq_length() must return a scalar")
        return int(value.item())
    return int(value)


def static_cache_sequence_length(cache: object) -> int:
    """Committed positions of a cache, or ``CachePrefixCopyError``.
    Reference: duplex_kernel/thinker_cache.py:54-56."""
    return _cache_length(cache)


def _is_full_static_layer(layer: object) -> bool:
    from transformers.cache_utils import StaticLayer

    return isinstance(layer, StaticLayer) and not bool(getattr(layer, "is_sliding", False))


def static_cache_storage_bytes(cache: object) -> int:
    """Allocated K/V bytes, unused static capacity included.
    Reference: duplex_kernel/thinker_cache.py:59-76."""
    if isinstance(cache, KVRTCache):
        rt = cache.runtime
        total = 0
        for i, spec in enumerate(rt.layers):
            if rt._owner(i) != i:
                continue
            k, v, _, _ = rt.storage(i)
            total += (k[cache.slot].numel() + v[cache.slot].numel()) * k.element_size() \
                if spec.layout != "paged" else 0
        return total
    layers = getattr(cache, "layers", None)
    if not isinstance(layers, (list, tuple)) or not layers:
        raise CachePrefixCopyError("cache exposes no measurable layers")
    total = 0
    for i, layer in enumerate(layers):
        if not _is_full_static_layer(layer):
            raise CachePrefixCopyError(f"layer {i} is not a full-attention StaticLayer")
        if not bool(getattr(layer, "is_initialized", False)):
            continue
        keys, values = getattr(layer, "keys", None), getattr(layer, "values", None)
        if not isinstance(keys, torch.Tensor) or not isinstance(values, torch.Tensor):
            raise CachePrefixCopyError(f"layer {i} K/V storage is unreadable")
        total += keys.numel() * keys.element_size() + values.numel() * values.element_size()
    return total


def _copy_kvrt(source: KVRTCache, target: KVRTCache, n: int) -> CachePrefixCopyResult:
    if source.runtime is not target.runtime:
        raise CachePrefixCopyError("source and target must be slots of one KVRuntime")
    rt = source.runtime
    src_len = _cache_length(source)
    if n > src_len:
        raise CachePrefixCopyError(f"token_count={n} exceeds source cache length={src_len}")
    owned = [i for i in range(len(rt.layers)) if rt._owner(i) == i]
    for i in owned:
        if rt.layers[i].layout == "paged":
            raise CachePrefixCopyError(f"layer {i} is paged: prefix copy needs CONTIG or RING storage")
        if source.get_seq_length(i) != src_len:
            raise CachePrefixCopyError(f"layer {i} length differs from the source cache length")
        if target.get_seq_length(i) != 0:
            raise CachePrefixCopyError(f"target layer {i} is not empty")
    target.generation = rt.copy_prefix(source.slot, target.slot, n, generation=source.generation)
    copied = sum(2 * rt.layers[i].kv_heads * n * rt.layers[i].head_dim * 2 for i in owned)
    if _cache_length(target) != n:
        raise CachePrefixCopyError("target length does not match the copied prefix")
    return CachePrefixCopyResult(copied_tokens=n, copied_bytes=copied, layer_count=len(owned))


def copy_static_cache_prefix(source_cache: object, target_cache: object, token_count: int) -> CachePrefixCopyResult:
    """Copy the first ``token_count`` positions of every layer into an empty,
    matching cache and set its lengths to ``token_count``.

    Reference: duplex_kernel/thinker_cache.py:83-190 (per-layer
    ``keys[:, :, :n].copy_()`` plus ``cumulative_length`` fill).
    """
    if isinstance(token_count, bool) or not isinstance(token_count, int) or token_count < 0:
        raise ValueError("token_count must be a non-negative int")
    if source_cache is target_cache:
        raise CachePrefixCopyError("source and target must be isolated caches")
    if token_count == 0:
        return CachePrefixCopyResult(copied_tokens=0, copied_bytes=0, layer_count=0)
    if isinstance(source_cache, KVRTCache) or isinstance(target_cache, KVRTCache):
        if not (isinstance(source_cache, KVRTCache) and isinstance(target_cache, KVRTCache)):
            raise CachePrefixCopyError("source and target must both be KVRTCache slots")
        return _copy_kvrt(source_cache, target_cache, token_count)

    src_layers = getattr(source_cache, "layers", None)
    dst_layers = getattr(target_cache, "layers", None)
    if not isinstance(src_layers, (list, tuple)) or not isinstance(dst_layers, (list, tuple)):
        raise CachePrefixCopyError("source/target must expose cache layers")
    if not src_layers or len(src_layers) != len(dst_layers):
        raise CachePrefixCopyError("source/target layer counts differ")
    src_len = _cache_length(source_cache)
    if token_count > src_len:
        raise CachePrefixCopyError(f"token_count={token_count} exceeds source cache length={src_len}")

    pairs = []
    for i, (s, t) in enumerate(zip(src_layers, dst_layers)):
        if not _is_full_static_layer(s) or not _is_full_static_layer(t):
            raise CachePrefixCopyError(f"layer {i} is not a full-attention StaticLayer")
        if type(s) is not type(t):
            raise CachePrefixCopyError(f"source/target layer types differ at index {i}")
        if s.get_seq_length() != src_len:
            raise CachePrefixCopyError(f"layer {i} length differs from the source cache length")
        if t.get_seq_length() != 0:
            raise CachePrefixCopyError(f"target layer {i} is not empty")
        if not s.is_initialized or s.keys is None or s.values is None:
            raise CachePrefixCopyError(f"source layer {i} is not initialised")
        if token_count > int(s.keys.shape[-2]):
            raise CachePrefixCopyError(f"source layer {i} does not hold the whole prefix")
        if int(s.max_cache_len) != int(t.max_cache_len):
            raise CachePrefixCopyError(f"StaticLayer capacity differs at index {i}")
        if tuple(s.keys.shape) != tuple(s.values.shape):
            raise CachePrefixCopyError(f"source K/V shapes differ at index {i}")
        if s.keys.dim() != 4:
            raise CachePrefixCopyError(f"source K/V are not rank 4 at index {i}")
        if not s.keys.is_cuda:
            raise CachePrefixCopyError(f"source layer {i} is not on the GPU (kvrt has no CPU path)")
        pairs.append((s, t))

    copied = 0
    for i, (s, t) in enumerate(pairs):
        try:
            if not t.is_initialized:
                shape = s.keys.shape
                empty = torch.empty((shape[0], shape[1], 0, shape[3]), device=s.keys.device, dtype=s.keys.dtype)
                t.lazy_initialization(empty, empty)
            for a, b in ((t.keys, s.keys), (t.values, s.values)):
                if tuple(a.shape) != tuple(b.shape) or a.device != b.device or a.dtype != b.dtype:
                    raise CachePrefixCopyError(f"StaticLayer storage incompatible at index {i}")
            copy_rows(s.keys, t.keys, token_count)
            copy_rows(s.values, t.values, token_count)
            t.cumulative_length.fill_(token_count)
            per_row = s.keys.shape[0] * s.keys.shape[1] * s.keys.shape[3]
            copied += token_count * per_row * (s.keys.element_size() + s.values.element_size())
        except CachePrefixCopyError:
            raise
        except Exception as exc:
            raise CachePrefixCopyError(f"StaticLayer copy failed at index {i}: {exc}") from exc

    if _cache_length(target_cache) != token_count:
        raise CachePrefixCopyError("target length does not match the copied prefix")
    return CachePrefixCopyResult(copied_tokens=token_count, copied_bytes=copied, layer_count=len(pairs))


AUDIO_THINKER_CACHE_BUCKETS = (512, 1024, 2048, 4096)


def select_audio_thinker_cache_bucket(prefill_tokens: int, output_budget: int, *,
                                      max_cache_len: int = AUDIO_THINKER_CACHE_BUCKETS[-1]) -> int:
    """Smallest static capacity holding the prefill plus the whole generation
    budget; never truncates. Reference: duplex_kernel/engine.py:591-630."""
    for name, value in (("prefill_tokens", prefill_tokens), ("output_budget", output_budget),
                        ("max_cache_len", max_cache_len)):
        if isinstance(value, bool) or not isinstance(value, Integral):
            raise TypeError(f"{name} must be an integer")
        if int(value) < 1:
            raise ValueError(f"{name} must be at least 1")
    need = int(prefill_tokens) + int(output_budget)
    usable = [b for b in AUDIO_THINKER_CACHE_BUCKETS if b <= int(max_cache_len)]
    for bucket in usable:
        if need <= bucket:
            return bucket
    raise ValueError(
        f"thinker prompt + budget exceed the static-cache buckets ({prefill_tokens} + {output_budget} = {need}; "
        f"largest usable {usable[-1] if usable else 0}, largest supported {AUDIO_THINKER_CACHE_BUCKETS[-1]})"
    )


__all__ = [
    "AUDIO_THINKER_CACHE_BUCKETS",
    "CachePrefixCopyError",
    "CachePrefixCopyResult",
    "copy_static_cache_prefix",
    "longest_common_prefix_length",
    "select_audio_thinker_cache_bucket",
    "static_cache_sequence_length",
    "static_cache_storage_bytes",
]
