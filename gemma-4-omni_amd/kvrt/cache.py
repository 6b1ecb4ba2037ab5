"""HF-cache-shaped views of kvrt storage, and the gather / attend entry points.

``KVRTCache`` is one slot (session or stream) of a :class:`KVRuntime` dressed
as a transformers ``Cache``: ``.layers[i].keys/.values``, ``update``,
``get_seq_length``, ``crop``, iteration over ``(K, V)`` pairs and
``copy.deepcopy``. The reference's KV helpers (duplex_kernel/kv_cache.py,
duplex_kernel/thinker_cache.py) and its HF attention call sites operate on
exactly that surface, so they run unchanged over device-resident kvrt storage:

* ``update`` is the append of HF ``DynamicLayer.update``
  (transformers cache_utils.py ``torch.cat(dim=-2)``) or, with an explicit
  ``cache_position``, the positional write of ``_SlotKVCache.update``
  (duplex_kernel/future_prefix.py:523-571) — one kvrt kernel either way;
* ``crop`` / ``truncate`` are length edits (kv_cache.py:205-216 sliced and
  copied; here no KV byte moves);
* ``copy.deepcopy`` copies the slot into a free slot of the same runtime on
  the GPU (kv_cache.py:60 deep-copies the prefix once per session).

``gather`` and ``attend`` are the two functions the reference expresses only
through padding buffers and SDPA (shape_stable_listener.py:28-69, :241-251).

Everything here enqueues kvrt kernels on the current torch stream; there is no
PyTorch or CPU compute path behind any of it.
"""
from __future__ import annotations

from typing import Any, Iterator, Sequence

import torch

from .runtime import KVRuntime, attend_tensors, copy_rows


class KVRTCacheLayer:
    """One layer of a :class:`KVRTCache` (the HF ``CacheLayerMixin`` surface)."""

    is_compileable = False

    def __init__(self, cache: "KVRTCache", index: int) -> None:
        self._cache = cache
        self.layer_idx = int(index)

    @property
    def _spec(self):
        rt = self._cache.runtime
        return rt.layers[rt._owner(self.layer_idx)]

    @property
    def is_initialized(self) -> bool:
        return True

    @property
    def is_sliding(self) -> bool:
        return self._spec.window > 0

    @property
    def sliding_window(self) -> int:
        return self._spec.window

    @property
    def max_cache_len(self) -> int:
        return self._cache.runtime.capacity

    @property
    def cumulative_length(self) -> int:
        return self.get_seq_length()

    @property
    def keys(self) -> torch.Tensor:
        return self._cache.runtime.layer_view(self._cache.slot, self.layer_idx)[0]

    @property
    def values(self) -> torch.Tensor:
        return self._cache.runtime.layer_view(self._cache.slot, self.layer_idx)[1]

    def get_seq_length(self) -> int:
        return self._cache.get_seq_length(self.layer_idx)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, cache_kwargs: dict | None = None,
               *args: Any, **kwargs: Any) -> tuple[torch.Tensor, torch.Tensor]:
        return self._cache.update(key_states, value_states, self.layer_idx, cache_kwargs)

    def crop(self, tokens: int) -> None:
        self._cache._crop_layer(self.layer_idx, int(tokens))


class KVRTCache:
    """One slot of a :class:`KVRuntime` with the transformers ``Cache`` surface.

    Owns its slot: the slot returns to the runtime's free list when the cache
    is released or garbage-collected.
    """

    is_compileable = False

    def __init__(self, runtime: KVRuntime, slot: int | None = None) -> None:
        self.runtime = runtime
        self._owns_slot = slot is None
        self.slot = runtime.acquire_slot() if slot is None else int(slot)
        self.layers = [KVRTCacheLayer(self, i) for i in range(len(runtime.layers))]
        # the slot's generation when this cache took it (or last changed its
        # contents): rollbacks through this cache are refused once the slot
        # holds another session
        self.generation = runtime.slot_generation(self.slot)
        # Gemma shared-KV sources, as the reference keeps them on its
        # DynamicCache (shape_stable_listener.py:222-226, :234-238).
        self.shared_layers: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}

    # ---- transformers Cache surface ---------------------------------------------
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: dict | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Append [1, kv_heads, Q, D] rows (or write them at ``cache_kwargs['cache_position']``).

        Returns the K/V states an HF attention call would see after the update:
        every stored position (global layers) or the last ``W - 1`` stored
        positions plus the new rows (sliding layers, as HF
        ``DynamicSlidingWindowLayer.update`` returns them); after a positional
        write, the slot's whole [1, kv_heads, capacity, D] storage, as
        ``_SlotKVCache.update`` returns its fixed-size tensors
        (future_prefix.py:544-565), which is what the [.., capacity] masks of
        ``get_mask_sizes`` are built for.
        """
        layer_idx = int(layer_idx)
        if key_states.dim() != 4 or key_states.shape[0] != 1:
            raise ValueError("KVRTCache.update takes [1, kv_heads, Q, D] key/value states")
        rt = self.runtime
        spec = rt.layers[rt._owner(layer_idx)]
        before = self.get_seq_length(layer_idx)
        positions = None if cache_kwargs is None else cache_kwargs.get("cache_position")
        returned = None
        if spec.window > 0 and positions is None:
            # HF DynamicSlidingWindowLayer.update returns the retained W - 1
            # positions followed by the new rows. Collect the retained rows
            # before the append (it may overwrite ring rows), then the new rows.
            q = int(key_states.shape[2])
            r = before - max(0, before - (spec.window - 1))
            dt = torch.float32 if spec.dtype == "int8" else torch.bfloat16
            returned = tuple(torch.empty((1, spec.kv_heads, r + q, spec.head_dim), dtype=dt, device=rt.device)
                             for _ in range(2))
            if r > 0:
                rt.gather(layer_idx, [self.slot], start_pos=[before - r], mask_dtype=None,
                          out=(returned[0][:, :, :r], returned[1][:, :, :r]))
            if dt == torch.bfloat16:
                copy_rows(key_states, returned[0][:, :, r:], q)
                copy_rows(value_states, returned[1][:, :, r:], q)
        if positions is None:
            self.runtime.append(layer_idx, key_states, value_states, [self.slot])
        else:
            pos = [int(p) for p in torch.as_tensor(positions).reshape(-1).tolist()]
            if len(pos) != key_states.shape[-2]:
                raise ValueError("cache_position must hold one position per key row")
            if any(p < 0 or p >= self.runtime.capacity for p in pos):
                # _SlotKVCache raises OverflowError here (future_prefix.py:544-549)
                raise OverflowError(f"slot KV position outside [0, {self.runtime.capacity})")
            self.runtime.write_positions(layer_idx, key_states, value_states, [self.slot], [pos])
            k_all, v_all, _, _ = rt.storage(layer_idx)  # CONTIG bf16: zero-copy views
            return k_all[self.slot:self.slot + 1], v_all[self.slot:self.slot + 1]
        if returned is not None and spec.dtype != "int8":
            return returned
        return rt.layer_view(self.slot, layer_idx)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.runtime.seq_length(self.slot, int(layer_idx))

    def get_max_length(self, layer_idx: int = 0) -> int:
        return self.runtime.capacity

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return self.runtime.capacity

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0) -> tuple[int, int]:
        return self.runtime.capacity, 0

    def crop(self, tokens: int) -> None:
        """transformers 5.x ``Cache.crop``: a positive value is the length to keep
        (no-op when not shorter), a negative value the number of positions to
        drop; 0 changes nothing. A length edit on every layer."""
        for layer in range(len(self.layers)):
            if self.runtime._owner(layer) == layer:
                self._crop_layer(layer, int(tokens))

    def _crop_layer(self, layer: int, tokens: int) -> None:
        length = self.get_seq_length(layer)
        if tokens > 0:
            if tokens >= length:
                return
            new_len = tokens
        elif tokens < 0:
            new_len = max(0, length + tokens)
        else:
            return
        self.runtime.truncate(self.slot, new_len, layer=layer, generation=self.generation, expected_len=length)

    def truncate(self, keep_len: int) -> None:
        """Rollback every layer to ``keep_len`` positions (no KV byte moves)."""
        self.runtime.truncate(self.slot, int(keep_len), generation=self.generation)

    def reset(self) -> None:
        """Zero the slot's rows and lengths (``_SlotKVCache.reset``)."""
        self.generation = self.runtime.reset_slot(self.slot)
        self.shared_layers.clear()

    def adopt(self) -> None:
        """Take the slot's current generation after its contents were replaced
        through the runtime (an import or a copy into it)."""
        self.generation = self.runtime.slot_generation(self.slot)

    def __len__(self) -> int:
        return len(self.layers)

    def __getitem__(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.runtime.layer_view(self.slot, int(layer_idx))

    def __iter__(self) -> Iterator[tuple[torch.Tensor, torch.Tensor]]:
        for i in range(len(self.layers)):
            yield self[i]

    def __deepcopy__(self, memo: dict) -> "KVRTCache":
        """An isolated copy in a free slot of the same runtime (a device copy)."""
        owned = [l for l in range(len(self.layers)) if self.runtime._owner(l) == l]
        lengths = {self.get_seq_length(l) for l in owned}
        if len(lengths) != 1:
            raise ValueError("KVRTCache deepcopy needs every layer at one length")
        clone = KVRTCache(self.runtime)
        clone.generation = self.runtime.copy_prefix(self.slot, clone.slot, lengths.pop(), generation=self.generation)
        memo[id(self)] = clone
        return clone

    def release(self) -> None:
        """Return the slot to the runtime (lengths drop to 0)."""
        if self._owns_slot and self.slot is not None and self.runtime._ctx:
            self.runtime.release_slot(self.slot)
        self.slot = None if self._owns_slot else self.slot
        self._owns_slot = False

    def __del__(self) -> None:  # pragma: no cover - interpreter teardown order
        try:
            self.release()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# gather / attend
# ---------------------------------------------------------------------------
def _slots(caches: KVRTCache | Sequence[KVRTCache]) -> tuple[KVRuntime, list[int]]:
    if isinstance(caches, KVRTCache):
        caches = [caches]
    caches = list(caches)
    if not caches:
        raise ValueError("at least one cache is needed")
    rt = caches[0].runtime
    if any(c.runtime is not rt for c in caches):
        raise ValueError("all caches of one call must share a KVRuntime")
    return rt, [c.slot for c in caches]


def gather(caches: KVRTCache | Sequence[KVRTCache], layer_idx: int, target_length: int | None = None,
           mask_dtype: torch.dtype | None = torch.bool, start: Sequence[int] | None = None,
           ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Ragged micro-batch gather: zero-padded K, V [N, kv_heads, Lmax, D] + mask [N, Lmax].

    Semantics of ``_StaticPaddingWorkspace.padded / padded_mask``
    (duplex_kernel/shape_stable_listener.py:38-69): rows past a stream's
    length are zero; the mask tail is ``False`` (bool) or ``finfo.min``
    (float). ``target_length`` defaults to the longest stream.
    """
    rt, slots = _slots(caches)
    return rt.gather(int(layer_idx), slots, lmax=target_length, start_pos=start, mask_dtype=mask_dtype)


def attend(q: torch.Tensor, caches: KVRTCache | Sequence[KVRTCache], layer_idx: int, scale: float,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """GQA decode attention of q [N, Hq, Q, D] over the last Q positions of each cache.

    Causal (and, on sliding layers, windowed) visibility; fp32 softmax and
    accumulation; bf16 output — the semantics of HF ``sdpa_attention_forward``
    with ``repeat_kv`` (shape_stable_listener.py:241-251).
    """
    rt, slots = _slots(caches)
    return rt.attend(int(layer_idx), q, slots, scale, out=out)


def append_attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, caches: KVRTCache | Sequence[KVRTCache],
                  layer_idx: int, scale: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused per-layer decode step: append k, v [N, kv_heads, Q, D], then attend q."""
    rt, slots = _slots(caches)
    return rt.append_attend(int(layer_idx), q, k, v, slots, scale, out=out)


def attend_padded(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lengths: torch.Tensor, scale: float,
                  window: int = 0, out: torch.Tensor | None = None,
                  prefix_attention: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention over a padded batch (the output of :func:`gather`).

    ``lengths`` int32 [N] on the device (e.g. ``mask.sum(1)``); query row i of
    stream b sits at position ``lengths[b] - Q + i``; ``prefix_attention``
    [N, P] hides key j < P of stream b where it is 0 (the listener's
    per-session prefix mask, gemma4_listener_kernels.cuh:517-518).
    """
    return attend_tensors(q, k, v, lengths, scale, window=window, out=out, prefix_attention=prefix_attention)


__all__ = ["KVRTCache", "KVRTCacheLayer", "append_attend", "attend", "attend_padded", "gather"]
