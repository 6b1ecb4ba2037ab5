"""KV-cache session helpers of the duplex loops, over kvrt storage.

Same names, fields and behaviour as the reference module
``duplex_kernel/kv_cache.py`` (andr-lab/gemma-4-omni), so callers switch by
changing the import. The helpers accept the objects the reference accepts —
transformers ``Cache`` objects (``crop`` / ``get_seq_length``), tuples of
``(K, V)`` per layer — plus :class:`kvrt.cache.KVRTCache`, whose storage
stays in HBM:

* ``TurnKVState.truncate_to_prefix`` / ``_slice_kv`` on a ``KVRTCache`` is a
  length edit (kv_cache.py:99-104, :205-216 sliced and copied);
* ``TalkerPrefixKV.store`` of a ``KVRTCache`` is one device copy into a free
  slot of the same runtime (kv_cache.py:58-62 ``copy.deepcopy``);
* tuples of device tensors are sliced / cloned by the kvrt row-copy kernel.

Two functions the reference does not have are exported beside them:
``gather`` (ragged micro-batch gather) and ``attend`` (GQA decode attention).
Tensors on the CPU are refused: kvrt has no CPU path.
"""
from __future__ import annotations

import copy
import logging
from dataclasses import dataclass, field
from typing import Any

import torch

from .cache import KVRTCache, append_attend, attend, gather
from .runtime import copy_rows

logger = logging.getLogger("kvrt.kv_cache")


@dataclass
class TalkerPrefixKV:
    """KV of the talker's stable prefix, computed once per session.

    Reference: duplex_kernel/kv_cache.py:41-67.
    """

    kv: Any | None = None
    last_hidden: torch.Tensor | None = None
    seq_len: int = 0
    dtype: str = "bfloat16"
    device: str = "cuda"

    def is_ready(self) -> bool:
        return self.kv is not None

    def store(self, past_key_values: Any) -> None:
        """Snapshot the prefix KV (an isolated copy) and record its length."""
        self.kv = copy.deepcopy(past_key_values)
        self.seq_len = _kv_seq_len(past_key_values)
        logger.debug("[kvrt] talker prefix stored (seq_len=%d)", self.seq_len)

    def clear(self) -> None:
        self.kv = None
        self.last_hidden = None
        self.seq_len = 0


@dataclass
class TurnKVState:
    """The talker's KV for the current turn: starts at the prefix, grows by
    one codec frame per step, and is rolled back to the prefix at the end of
    the turn or on barge-in. Reference: duplex_kernel/kv_cache.py:70-108."""

    kv: Any | None = None
    frames_generated: int = 0
    prefix_len: int = 0
    device: str = "cuda"

    def start_from_prefix(self, prefix: TalkerPrefixKV) -> None:
        if prefix.is_ready():
            self.kv = prefix.kv
            self.prefix_len = prefix.seq_len
        else:
            self.kv = None
            self.prefix_len = 0
        self.frames_generated = 0

    def append(self, past_key_values: Any) -> None:
        """Adopt the cache object of the current step (the tensors were
        appended by the model's ``update`` call)."""
        self.kv = past_key_values

    def truncate_to_prefix(self) -> None:
        """Roll the turn back to the prefix (a length edit on a KVRTCache)."""
        if self.kv is None or self.prefix_len <= 0:
            return
        self.kv = _slice_kv(self.kv, self.prefix_len)
        self.frames_generated = 0

    def truncate_to_position(self, position: int) -> None:
        """Roll back to ``position`` tokens, never below the prefix.

        ``DuplexKVCacheProxy.rollback_to`` probes for this method
        (duplex_kernel/session.py:912-918) before falling back to
        ``truncate_to_prefix``.
        """
        if self.kv is None:
            return
        keep = max(int(position), self.prefix_len)
        if keep < _kv_seq_len(self.kv):
            self.kv = _slice_kv(self.kv, keep)
        self.frames_generated = max(0, keep - self.prefix_len)

    def clear(self) -> None:
        self.kv = None
        self.frames_generated = 0


@dataclass
class ThinkerContext:
    """Rolling token window of the thinker: system prompt, optional summary
    and the last ``max_turns`` turns within ``max_context_tokens``; older turns
    are evicted first. Host-side bookkeeping only.
    Reference: duplex_kernel/kv_cache.py:111-169."""

    system_prompt: str = ""
    turns: list[list[int]] = field(default_factory=list)
    message_turns: list[dict[str, Any]] = field(default_factory=list)
    max_turns: int = 8
    summary: str = ""
    max_context_tokens: int = 8192

    def set_messages(self, messages: list[dict[str, Any]]) -> None:
        keep = messages[-self.max_turns * 2:]
        self.message_turns = [dict(m) for m in keep]

    def messages(self) -> list[dict[str, Any]]:
        return [dict(m) for m in self.message_turns]

    def add_turn(self, token_ids: list[int]) -> None:
        if token_ids:
            self.turns.append(list(token_ids))
        while len(self.turns) > self.max_turns:
            self.turns.pop(0)
        self._trim_to_budget()

    def _trim_to_budget(self) -> None:
        total = sum(len(t) for t in self.turns)
        while self.turns and total > self.max_context_tokens:
            total -= len(self.turns.pop(0))

    def flatten(self, tokenizer: Any) -> list[int]:
        ids: list[int] = []
        for text in (self.system_prompt, self.summary):
            if text:
                ids.extend(tokenizer.encode(text, add_special_tokens=False))
        for turn in self.turns:
            ids.extend(turn)
        return ids

    def clear_turns(self) -> None:
        self.turns.clear()
        self.message_turns.clear()


# ---------------------------------------------------------------------------
# helpers over past_key_values
# ---------------------------------------------------------------------------
def _require_device(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise TypeError("kvrt: KV tensors must live on the GPU (there is no CPU path)")


def _device_rows(t: torch.Tensor, rows: int) -> torch.Tensor:
    """A fresh contiguous [B, H, rows, D] copy of t[:, :, :rows] (kvrt row copy)."""
    _require_device(t)
    out = torch.empty((t.shape[0], t.shape[1], rows, t.shape[3]), dtype=t.dtype, device=t.device)
    copy_rows(t, out, rows)
    return out


def _clone_kv(past_key_values: Any) -> tuple[tuple[torch.Tensor, torch.Tensor], ...]:
    """Per-layer ``(K, V)`` copies sharing no memory with the input.

    Reference: duplex_kernel/kv_cache.py:175-188 (a wrapper's
    ``past_key_values`` is unwrapped; the flattened ``(K, V)`` tensor pair is
    returned as is).
    """
    if past_key_values is None:
        return ()
    if hasattr(past_key_values, "past_key_values"):
        past_key_values = past_key_values.past_key_values
    if isinstance(past_key_values, tuple) and past_key_values and isinstance(past_key_values[0], torch.Tensor):
        return past_key_values
    out = []
    for layer in past_key_values:
        if isinstance(layer, (list, tuple)) and len(layer) >= 2:
            k, v = layer[0], layer[1]
            out.append((_device_rows(k, k.shape[2]), _device_rows(v, v.shape[2])))
    return tuple(out)


def _kv_seq_len(past_key_values: Any) -> int:
    """Cached positions: ``get_seq_length()`` when the object has it, else the
    key length of the first layer. Reference: duplex_kernel/kv_cache.py:191-202."""
    if past_key_values is None:
        return 0
    if hasattr(past_key_values, "get_seq_length"):
        try:
            return int(past_key_values.get_seq_length())
        except Exception:
            pass
    for layer in past_key_values:
        if isinstance(layer, (list, tuple)) and len(layer) >= 2 and layer[0] is not None:
            return int(layer[0].shape[2])
    return 0


def _slice_kv(past_key_values: Any, keep_len: int) -> Any:
    """Keep the first ``keep_len`` positions.

    Objects with ``crop`` are cropped in place and returned (a length edit on
    a ``KVRTCache``); tuples of ``(K, V)`` become fresh contiguous copies of
    the kept rows. Reference: duplex_kernel/kv_cache.py:205-216.
    """
    if hasattr(past_key_values, "crop"):
        past_key_values.crop(keep_len)
        return past_key_values
    out = []
    for k, v in past_key_values:
        n = int(k.shape[2])
        rows = min(int(keep_len), n) if keep_len >= 0 else max(0, n + int(keep_len))  # Python slice rule
        out.append((_device_rows(k, rows), _device_rows(v, rows)))
    return tuple(out)


def kv_memory_bytes(past_key_values: Any) -> int:
    """Bytes of the K/V tensors (logical views for a ``KVRTCache``).
    Reference: duplex_kernel/kv_cache.py:219-227."""
    total = 0
    for layer in past_key_values:
        if isinstance(layer, (list, tuple)) and len(layer) >= 2:
            for t in layer[:2]:
                if t is not None:
                    total += t.numel() * t.element_size()
    return total


__all__ = [
    "KVRTCache",
    "TalkerPrefixKV",
    "ThinkerContext",
    "TurnKVState",
    "append_attend",
    "attend",
    "gather",
    "kv_memory_bytes",
]
