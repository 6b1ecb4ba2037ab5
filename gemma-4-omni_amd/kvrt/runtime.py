"""Python host side of the kvrt runtime (PyTorch-ROCm tensors in, libkvrt.so out).

``KVRuntime`` owns one kvrt context: per-layer KV storage for ``n_slots``
sessions/streams, host-authoritative lengths (mirrored on the device), the
page pool for paged layers, and the split-K workspace. Every method enqueues
hand-written gfx950 kernels on the current torch stream through the C ABI in
``include/kvrt.h``; there is no PyTorch or CPU fallback behind any method.

Storage is allocated by torch (so HF-shaped views of a contiguous layer are
free) and bound to the context with ``kvrt_create_with_storage``.
"""
from __future__ import annotations

import ctypes
import math
import threading
from dataclasses import dataclass
from typing import Iterable, Sequence

import torch

from . import _lib as L

_DTYPE_CODES = {
    torch.bfloat16: L.DT_BF16,
    torch.int8: L.DT_INT8,
    torch.float32: L.DT_FP32,
    torch.bool: L.DT_BOOL,
    torch.int32: L.DT_INT32,
    torch.int64: L.DT_INT64,
}
_LAYOUTS = {"contig": L.LAYOUT_CONTIG, "ring": L.LAYOUT_RING, "paged": L.LAYOUT_PAGED}


class KVRTError(RuntimeError):
    """A kvrt C-ABI call returned a negative status."""

    def __init__(self, code: int, where: str) -> None:
        self.code = int(code)
        super().__init__(f"{where}: kvrt error {code} ({L.strerror(code)})")


def _check(code: int, where: str) -> None:
    if code != L.KVRT_OK:
        raise KVRTError(code, where)


# Descriptors are a pure function of (data pointer, dtype, shape, strides), so
# they are cached on that key: a decode loop that reuses its buffers skips the
# ctypes field writes (~3 us per tensor). The C side reads a descriptor
# synchronously and never keeps it, and nothing writes one after it is built.
_DESC_CACHE: dict = {}
_DESC_CACHE_MAX = 4096


def tensor_desc(t: torch.Tensor) -> L.KvrtTensor:
    """Strided descriptor of a device tensor (strides in elements)."""
    key = (t.data_ptr(), t.dtype, t.shape, t.stride())
    d = _DESC_CACHE.get(key)
    if d is not None:
        return d
    if t.dtype not in _DTYPE_CODES:
        raise TypeError(f"unsupported dtype {t.dtype}")
    if t.dim() > L.KVRT_MAX_RANK:
        raise ValueError("tensors of rank > 4 are not supported")
    d = L.KvrtTensor()
    d.data = t.data_ptr()
    d.dtype = _DTYPE_CODES[t.dtype]
    d.ndim = t.dim()
    for i, (n, s) in enumerate(zip(t.shape, t.stride())):
        d.dims[i] = int(n)
        d.strides[i] = int(s)
    if len(_DESC_CACHE) >= _DESC_CACHE_MAX:
        _DESC_CACHE.clear()
    _DESC_CACHE[key] = d
    return d


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(device: torch.device) -> int:
    """The current torch stream of ``device`` as a raw HIP stream handle."""
    if _RAW_STREAM is not None:  # the handle without building a Stream object
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return int(_RAW_STREAM(idx))
    return int(torch.cuda.current_stream(device).cuda_stream)


# ctypes int32 arrays of slot lists, cached like the descriptors (read-only on
# the C side).
_SLOT_ARRAYS: dict = {}


def require_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (kvrt has no CPU path)")


@dataclass(frozen=True)
class LayerSpec:
    """One KV layer: layout, dtype, GQA shape, window and aliasing.

    ``layout``: "contig" ([slots, kv_heads, capacity, D]), "ring" (sliding
    window ring of ``ring_rows`` rows) or "paged" (shared page pool).
    ``shared_src >= 0`` makes the layer read another layer's K/V (Gemma-4
    shared-KV layers, native/gemma4_listener_microbatch/generated_topology.h:59-95).
    """

    kv_heads: int
    head_dim: int
    layout: str = "contig"
    dtype: str = "bf16"
    window: int = 0
    ring_rows: int = 0
    shared_src: int = -1

    def to_c(self) -> L.KvrtLayerSpec:
        s = L.KvrtLayerSpec()
        s.layout = _LAYOUTS[self.layout]
        s.dtype = L.DT_INT8 if self.dtype == "int8" else L.DT_BF16
        s.kv_heads = self.kv_heads
        s.head_dim = self.head_dim
        s.window = self.window
        s.ring_rows = self.ring_rows
        s.shared_src = self.shared_src
        s.reserved = 0
        return s


@dataclass(frozen=True)
class TalkerMask:
    """Talker visibility of one slot (absolute cache positions).

    ``[0, prefix_start)`` is the stable text, ``[prefix_start, audio_start)``
    the reserved prefix frames of which ``[prefix_start, prefix_position]``
    are visible, ``[audio_start, audio_position]`` the audio frames so far.
    With Q = 2 query rows (JOINT step) row 0 is the prefix query at
    ``prefix_position`` and row 1 the audio query; with Q = 1 the single row
    is the audio query (terminal / audio-only step, ``prefix_position`` =
    the last visible prefix frame). ``prefix_attention_mode``: 0 audio
    queries see the visible prefix, 1 they do not, 2 they see it with
    ``prefix_log_gate - log(visible_prefix_count)`` (bf16) added to the
    score. Mirrors the arguments of qwen_build_joint_mask /
    qwen_build_audio_only_mask (native/qwen_talker/qwen_talker_kernels.cu:759-807)
    and their checks in duplex_kernel/native_qwen_talker.py:1211-1214.
    """

    prefix_start: int
    audio_start: int
    prefix_position: int
    audio_position: int
    prefix_attention_mode: int = 0
    visible_prefix_count: int = 0
    prefix_log_gate: float = -8.0

    def __post_init__(self) -> None:
        if self.prefix_attention_mode not in (0, 1, 2) or not math.isfinite(float(self.prefix_log_gate)):
            raise ValueError("invalid talker prefix gate: mode must be 0, 1 or 2 and the gate finite")
        if self.prefix_attention_mode == 2 and int(self.visible_prefix_count) <= 0:
            raise ValueError("the gated prefix mode needs visible_prefix_count > 0")
        if not (0 <= self.prefix_start <= self.prefix_position < self.audio_start <= self.audio_position):
            raise ValueError("talker positions must satisfy 0 <= prefix_start <= prefix_position < "
                             "audio_start <= audio_position")

    def to_c(self) -> L.KvrtTalkerMask:
        m = L.KvrtTalkerMask()
        m.prefix_start = int(self.prefix_start)
        m.audio_start = int(self.audio_start)
        m.prefix_position = int(self.prefix_position)
        m.audio_position = int(self.audio_position)
        m.prefix_attention_mode = int(self.prefix_attention_mode)
        m.visible_prefix_count = int(self.visible_prefix_count)
        m.prefix_log_gate = float(self.prefix_log_gate)
        return m


class KVRuntime:
    """One kvrt context: the KV state of ``n_slots`` sessions over ``layers``.

    Launch tuning (``kvrt_config``): ``decode_wgs`` is the split-K workgroup
    target of a decode launch (0: the library default); ``decode_kernel``
    ("auto", "valu", "mfma") picks the kernel of 8- and 16-row bf16 decodes
    (and, forced to "mfma", of int8 ones); ``decode_merge`` ("auto",
    "separate", "last_wg") picks whether a decode's last workgroup per (slot,
    kv head) merges the split-K partials inside the launch or a second kernel
    does.

    Confinement, as the reference binding's (native_listener_microbatch.py:
    1128-1131, gemma4_listener_microbatch_impl.inc:445-473): every call must
    come from the thread that created the runtime, and the context stays on
    the torch stream of its first call. Moving it to another stream raises
    ``KVRTError`` (code -2) while its work may still run there;
    :meth:`synchronize` (or :meth:`health` / :meth:`sync_lengths`) first
    makes the switch legal. Slots carry generations (:meth:`slot_generation`)
    that the lifecycle calls can check.
    """

    def __init__(
        self,
        layers: Sequence[LayerSpec],
        n_slots: int,
        capacity: int,
        *,
        max_q: int = 2,
        block_size: int = 16,
        pool_pages: int = 0,
        pool_seed: int = 0,
        decode_wgs: int = 0,
        decode_kernel: str = "auto",
        decode_merge: str = "auto",
        device: torch.device | str | None = None,
    ) -> None:
        self.lib = L.load()
        self._owner_thread = threading.get_ident()
        self.device = torch.device(device if device is not None else "cuda")
        if self.device.type != "cuda" or not torch.cuda.is_available():
            raise RuntimeError("KVRuntime needs a ROCm GPU (torch.cuda); there is no CPU path")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.layers = list(layers)
        self.n_slots = int(n_slots)
        self.capacity = int(capacity)
        self.max_q = int(max_q)
        self.block_size = int(block_size)
        self.pool_pages = int(pool_pages)
        self._ctx = ctypes.c_void_p()
        cfg = L.KvrtConfig()
        cfg.struct_size = ctypes.sizeof(L.KvrtConfig)
        cfg.n_layers = len(self.layers)
        cfg.n_slots = self.n_slots
        cfg.capacity = self.capacity
        cfg.block_size = self.block_size
        cfg.pool_pages = self.pool_pages
        cfg.max_q = self.max_q
        cfg.pool_seed = int(pool_seed)
        cfg.decode_wgs = int(decode_wgs)
        if decode_kernel not in L.DECODE_KERNELS:
            raise ValueError(f"decode_kernel must be one of {sorted(L.DECODE_KERNELS)}, got {decode_kernel!r}")
        cfg.decode_kernel = L.DECODE_KERNELS[decode_kernel]
        if decode_merge not in L.DECODE_MERGES:
            raise ValueError(f"decode_merge must be one of {sorted(L.DECODE_MERGES)}, got {decode_merge!r}")
        cfg.decode_merge = L.DECODE_MERGES[decode_merge]
        self._cfg = cfg
        specs = (L.KvrtLayerSpec * len(self.layers))(*[s.to_c() for s in self.layers])
        self._specs = specs
        storage = (L.KvrtStorage * len(self.layers))()
        self._store: list[tuple[torch.Tensor, torch.Tensor, torch.Tensor | None, torch.Tensor | None] | None] = []
        with torch.cuda.device(self.device):
            for i, spec in enumerate(self.layers):
                self._store.append(None if spec.shared_src >= 0 else self._alloc_layer(i, storage[i], zero=True))
            torch.cuda.synchronize(self.device)
            _check(self.lib.kvrt_create_with_storage(ctypes.byref(cfg), specs, storage, ctypes.byref(self._ctx)),
                   "kvrt_create_with_storage")
        self._free_slots = list(range(self.n_slots - 1, -1, -1))

    # ---- helpers -------------------------------------------------------------
    def _alloc_layer(self, i: int, entry: L.KvrtStorage, zero: bool):
        """Torch storage of layer i at the current slot count: typed views, with
        the base pointers written to ``entry`` (the views keep the buffers alive)."""
        spec = self.layers[i]
        kvb, scb = ctypes.c_uint64(), ctypes.c_uint64()
        _check(self.lib.kvrt_layer_storage_bytes(ctypes.byref(self._cfg), ctypes.byref(self._specs[i]),
                                                 ctypes.byref(kvb), ctypes.byref(scb)),
               "kvrt_layer_storage_bytes")
        shape = self._storage_shape(spec)
        dt = torch.int8 if spec.dtype == "int8" else torch.bfloat16
        es = 1 if dt == torch.int8 else 2
        make = torch.zeros if zero else torch.empty
        k = make(kvb.value // es, dtype=dt, device=self.device)
        v = make(kvb.value // es, dtype=dt, device=self.device)
        n_el = math.prod(shape)
        entry.k, entry.v = k.data_ptr(), v.data_ptr()
        ks = vs = None
        if spec.dtype == "int8":
            ks_flat = make(scb.value // 4, dtype=torch.float32, device=self.device)
            vs_flat = make(scb.value // 4, dtype=torch.float32, device=self.device)
            n_sc = math.prod(shape[:-1])
            ks, vs = ks_flat[:n_sc].view(shape[:-1]), vs_flat[:n_sc].view(shape[:-1])
            entry.k_scale, entry.v_scale = ks_flat.data_ptr(), vs_flat.data_ptr()
        return k[:n_el].view(shape), v[:n_el].view(shape), ks, vs

    def _storage_shape(self, spec: LayerSpec) -> tuple[int, ...]:
        if spec.layout == "contig":
            return (self.n_slots, spec.kv_heads, self.capacity, spec.head_dim)
        if spec.layout == "ring":
            return (self.n_slots, spec.kv_heads, spec.ring_rows, spec.head_dim)
        return (self.pool_pages, spec.kv_heads, self.block_size, spec.head_dim)

    def _owner(self, layer: int) -> int:
        src = self.layers[layer].shared_src
        return src if src >= 0 else layer

    def _own(self) -> None:
        if threading.get_ident() != self._owner_thread:
            raise RuntimeError("kvrt runtime is confined to the host thread that created it")

    def _bind(self) -> None:
        """Bind the current torch stream (refused while work is in flight on another)."""
        self._own()
        rc = self.lib.kvrt_bind_stream(self._ctx, ctypes.c_void_p(current_stream_handle(self.device)))
        if rc == L.KVRT_ESTATE:
            raise KVRTError(rc, "kvrt_bind_stream: the context's work may still run on its bound stream; "
                                "call synchronize() before using it from another stream")
        _check(rc, "kvrt_bind_stream")

    @staticmethod
    def _slots(slots: Iterable[int]) -> tuple[ctypes.Array, int]:
        key = tuple(map(int, slots))
        hit = _SLOT_ARRAYS.get(key)
        if hit is None:
            hit = ((ctypes.c_int32 * len(key))(*key), len(key))
            if len(_SLOT_ARRAYS) >= _DESC_CACHE_MAX:
                _SLOT_ARRAYS.clear()
            _SLOT_ARRAYS[key] = hit
        return hit

    def storage(self, layer: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
        """Typed views of a layer's K, V (and INT8 scale) storage."""
        st = self._store[self._owner(layer)]
        assert st is not None
        return st

    # ---- slots -----------------------------------------------------------------
    def ensure_capacity(self, n_slots: int) -> int:
        """Grow to at least ``n_slots`` slots; returns the slot count. Existing
        slots keep their rows, lengths, masks and generations; the new ones are
        empty and join the free list. Waits for the context's work; graphs
        captured earlier must be captured again. Mirrors
        NativeGemmaListenerMicrobatch.ensure_capacity
        (duplex_kernel/native_listener_microbatch.py:1217-1268)."""
        self._own()
        n = int(n_slots)
        if n <= self.n_slots:
            return self.n_slots
        old = self.n_slots
        self.n_slots = n
        self._cfg.n_slots = n
        storage = (L.KvrtStorage * len(self.layers))()
        fresh = {}
        try:
            with torch.cuda.device(self.device):
                for i, spec in enumerate(self.layers):
                    if spec.shared_src < 0 and spec.layout != "paged":
                        fresh[i] = self._alloc_layer(i, storage[i], zero=False)  # the library fills them
                _check(self.lib.kvrt_grow_slots(self._ctx, n, storage if fresh else None), "kvrt_grow_slots")
        except Exception:
            self.n_slots = old
            self._cfg.n_slots = old
            raise
        for i, views in fresh.items():
            self._store[i] = views  # the old buffers are released with their views
        self._free_slots = sorted(set(self._free_slots) | set(range(old, n)), reverse=True)
        return n

    def acquire_slot(self) -> int:
        """Take the lowest free slot (session/stream id); raise when none is left."""
        if not self._free_slots:
            raise RuntimeError(f"kvrt: all {self.n_slots} slots are in use")
        return self._free_slots.pop()

    def release_slot(self, slot: int) -> None:
        """Return a slot to the free list; its prefix mask is cleared and its
        lengths drop to 0 (no bytes move)."""
        slot = int(slot)
        if not 0 <= slot < self.n_slots or slot in self._free_slots:
            raise ValueError(f"kvrt: slot {slot} is not in use")
        self.set_prefix_attention(slot, None)
        self.truncate(slot, 0)
        self._free_slots.append(slot)
        self._free_slots.sort(reverse=True)

    # ---- KV operations -----------------------------------------------------
    def import_(self, slot: int, layer: int, k: torch.Tensor, v: torch.Tensor, first_pos: int = 0) -> None:
        """Import an HF layer view [1, kv_heads, S, D] bf16 as positions 0..S-1.

        The layer must be empty and the slot unmasked (a fresh, reset or
        released slot), else ``KVRTError`` code -2; the slot's generation is
        renewed (import_cache_async refuses a primed slot, impl.inc:2595)."""
        require_cuda(k, "k")
        require_cuda(v, "v")
        self._bind()
        kd, vd = tensor_desc(k), tensor_desc(v)
        _check(self.lib.kvrt_import_async(self._ctx, slot, layer, ctypes.byref(kd), ctypes.byref(vd), first_pos),
               "kvrt_import_async")

    def append(self, layer: int, k: torch.Tensor, v: torch.Tensor, slots: Sequence[int]) -> None:
        """Append k, v [n, kv_heads, Q, D] bf16 at each slot's current length."""
        require_cuda(k, "k")
        require_cuda(v, "v")
        self._bind()
        arr, n = self._slots(slots)
        kd, vd = tensor_desc(k), tensor_desc(v)
        _check(self.lib.kvrt_append_async(self._ctx, layer, n, arr, ctypes.byref(kd), ctypes.byref(vd)),
               "kvrt_append_async")

    def write_positions(self, layer: int, k: torch.Tensor, v: torch.Tensor, slots: Sequence[int],
                        positions: Sequence[Sequence[int]]) -> None:
        """Write k, v [n, kv_heads, Q, D] at explicit positions [n][Q] (CONTIG layers).

        Each slot's length becomes max(length, max position + 1). A position
        outside [0, capacity) raises ``KVRTError`` (code -2) and writes nothing.
        """
        require_cuda(k, "k")
        require_cuda(v, "v")
        flat = [int(p) for row in positions for p in row]
        if len(flat) != k.shape[0] * k.shape[2]:
            raise ValueError("positions must hold Q entries per slot")
        if k.shape[2] == 0:
            return  # an empty write changes nothing
        self._bind()
        arr, n = self._slots(slots)
        pos = (ctypes.c_int32 * max(1, len(flat)))(*flat)
        kd, vd = tensor_desc(k), tensor_desc(v)
        _check(self.lib.kvrt_write_positions_async(self._ctx, layer, n, arr, pos, ctypes.byref(kd),
                                                   ctypes.byref(vd)),
               "kvrt_write_positions_async")

    def reset_slot(self, slot: int) -> int:
        """Zero every stored row of a slot, set its lengths to 0, clear its prefix
        mask; returns the slot's new generation (the start of a session)."""
        self._bind()
        _check(self.lib.kvrt_reset_slot_async(self._ctx, int(slot)), "kvrt_reset_slot_async")
        return self.slot_generation(slot)

    def set_prefix_attention(self, slot: int, mask: torch.Tensor | None) -> None:
        """Prefix-attention mask of a slot: key position k < P is visible only where
        ``mask[..., k] != 0`` (int64 / int32 / bool, [1, P] or [P], P <= 512);
        ``None`` clears it. The listener's per-session ``prefix_attention``
        (native_listener_microbatch.py:1340-1414; gemma4_listener_kernels.cuh:517-518).
        """
        self._bind()
        if mask is None:
            _check(self.lib.kvrt_set_prefix_attention_async(self._ctx, int(slot), None),
                   "kvrt_set_prefix_attention_async")
            return
        if not mask.is_cuda:
            mask = mask.to(self.device)
        mask = mask.contiguous()
        md = tensor_desc(mask)
        _check(self.lib.kvrt_set_prefix_attention_async(self._ctx, int(slot), ctypes.byref(md)),
               "kvrt_set_prefix_attention_async")
        # the mask is read on the stream: keep it alive until that work has run
        mask.record_stream(torch.cuda.current_stream(self.device))

    def import_session(self, slot: int, layers: Sequence[tuple[torch.Tensor, torch.Tensor]],
                       prefix_attention: torch.Tensor | None = None) -> int:
        """Start a session in ``slot``: reset it, import one HF layer view
        [1, kv_heads, S, D] per non-shared layer (``layers[i]`` for layer i;
        shared layers' entries are ignored) and set its prefix mask. Returns
        the slot's generation. Mirrors gemma4_listener_batch_import_cache_async
        (gemma4_listener_microbatch_impl.inc:2590-2640)."""
        self.reset_slot(slot)
        for i, kv in enumerate(layers):
            if self._owner(i) != i:
                continue
            self.import_(slot, i, kv[0], kv[1])
        if prefix_attention is not None:
            self.set_prefix_attention(slot, prefix_attention)
        return self.slot_generation(slot)

    # Query rows per kv head (g * Q) above which attention runs on the MFMA
    # prefill kernel instead of the split-K decode kernel.
    DECODE_MAX_ROWS = 16

    def attend(self, layer: int, q: torch.Tensor, slots: Sequence[int], scale: float,
               out: torch.Tensor | None = None) -> torch.Tensor:
        """Attention of q [n, Hq, Q, D] over the last Q positions of each slot.

        Decode shapes (g * Q <= 16 query rows per kv head) take the split-K
        decode kernel; larger chunks (prefill, text appends) the MFMA kernel.
        """
        require_cuda(q, "q")
        spec = self.layers[self._owner(layer)]
        if (q.shape[1] // max(1, spec.kv_heads)) * q.shape[2] > self.DECODE_MAX_ROWS:
            return self.attend_prefill(layer, q, slots, scale, out=out)
        q = q.contiguous()
        out = torch.empty_like(q) if out is None else out
        self._bind()
        arr, n = self._slots(slots)
        qd, od = tensor_desc(q), tensor_desc(out)
        _check(self.lib.kvrt_attend_decode_async(self._ctx, layer, n, arr, ctypes.byref(qd), ctypes.byref(od),
                                                 float(scale)),
               "kvrt_attend_decode_async")
        return out

    def attend_prefill(self, layer: int, q: torch.Tensor, slots: Sequence[int], scale: float,
                       out: torch.Tensor | None = None) -> torch.Tensor:
        """Chunked-prefill attention (MFMA) of q [n, Hq, Q, D] over the last Q positions."""
        require_cuda(q, "q")
        q = q.contiguous()
        out = torch.empty_like(q) if out is None else out
        self._bind()
        arr, n = self._slots(slots)
        qd, od = tensor_desc(q), tensor_desc(out)
        _check(self.lib.kvrt_attend_prefill_async(self._ctx, layer, n, arr, ctypes.byref(qd), ctypes.byref(od),
                                                  float(scale)),
               "kvrt_attend_prefill_async")
        return out

    def attend_talker(self, layer: int, q: torch.Tensor, slots: Sequence[int], scale: float,
                      masks: Sequence["TalkerMask"], out: torch.Tensor | None = None) -> torch.Tensor:
        """Talker attention of q [n, Hq, Q, D] (Q = 2: prefix then audio query;
        Q = 1: audio query) under one :class:`TalkerMask` per slot."""
        require_cuda(q, "q")
        q = q.contiguous()
        out = torch.empty_like(q) if out is None else out
        self._bind()
        arr, n = self._slots(slots)
        if len(masks) != n:
            raise ValueError(f"{len(masks)} talker masks for {n} slots")
        marr = (L.KvrtTalkerMask * max(1, n))()
        for i, m in enumerate(masks):
            marr[i] = m.to_c()
        qd, od = tensor_desc(q), tensor_desc(out)
        _check(self.lib.kvrt_attend_talker_async(self._ctx, layer, n, arr, ctypes.byref(qd), ctypes.byref(od),
                                                 float(scale), marr),
               "kvrt_attend_talker_async")
        return out

    def append_attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      slots: Sequence[int], scale: float, out: torch.Tensor | None = None) -> torch.Tensor:
        """Fused per-layer decode step: append k, v then attend q."""
        require_cuda(q, "q")
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        out = torch.empty_like(q) if out is None else out
        self._bind()
        arr, n = self._slots(slots)
        qd, kd, vd, od = tensor_desc(q), tensor_desc(k), tensor_desc(v), tensor_desc(out)
        _check(self.lib.kvrt_append_attend_async(self._ctx, layer, n, arr, ctypes.byref(qd), ctypes.byref(kd),
                                                 ctypes.byref(vd), ctypes.byref(od), float(scale)),
               "kvrt_append_attend_async")
        return out

    def gather(self, layer: int, slots: Sequence[int], lmax: int | None = None,
               start_pos: Sequence[int] | None = None, mask_dtype: torch.dtype | None = torch.bool,
               out: tuple[torch.Tensor, torch.Tensor] | None = None,
               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
        """Zero-padded batch [n, kv_heads, Lmax, D] (+ mask [n, Lmax]) of n slots.

        ``out`` may supply the K and V destinations (strided views with a
        contiguous last dimension); Lmax is then their third dimension. A third
        element of ``out`` supplies the mask destination [n, Lmax] (of
        ``mask_dtype``), which is then returned instead of a new tensor.
        """
        spec = self.layers[self._owner(layer)]
        slots = [int(s) for s in slots]
        if out is not None:
            lmax = int(out[0].shape[2])
        if lmax is None:
            lens = [self.seq_length(s, layer) for s in slots]
            if start_pos is not None:
                lens = [a - b for a, b in zip(lens, start_pos)]
            elif spec.layout == "ring":
                lens = [min(x, spec.window - 1) for x in lens]
            lmax = max(1, max(lens))
        dt = torch.float32 if spec.dtype == "int8" else torch.bfloat16
        mask = None
        if out is not None:
            out_k, out_v = out[0], out[1]
            require_cuda(out_k, "out_k")
            require_cuda(out_v, "out_v")
            if len(out) > 2 and out[2] is not None:
                mask = out[2]
                require_cuda(mask, "out mask")
                if mask_dtype is not None and mask.dtype != mask_dtype:
                    raise ValueError(f"out mask dtype {mask.dtype} != mask_dtype {mask_dtype}")
                if tuple(mask.shape) != (len(slots), lmax):
                    raise ValueError(f"out mask shape {tuple(mask.shape)} != {(len(slots), lmax)}")
        else:
            out_k = torch.empty((len(slots), spec.kv_heads, lmax, spec.head_dim), dtype=dt, device=self.device)
            out_v = torch.empty_like(out_k)
        if mask is None and mask_dtype is not None:
            mask = torch.empty((len(slots), lmax), dtype=mask_dtype, device=self.device)
        self._bind()
        arr, n = self._slots(slots)
        sp = None if start_pos is None else (ctypes.c_int32 * n)(*[int(x) for x in start_pos])
        kd, vd = tensor_desc(out_k), tensor_desc(out_v)
        md = None if mask is None else ctypes.byref(tensor_desc(mask))
        _check(self.lib.kvrt_gather_async(self._ctx, layer, n, arr, sp, ctypes.byref(kd), ctypes.byref(vd), md),
               "kvrt_gather_async")
        return out_k, out_v, mask

    def append_gather(self, layer: int, k: torch.Tensor, v: torch.Tensor, slots: Sequence[int],
                      out: tuple, start_pos: Sequence[int] | None = None) -> tuple:
        """``append(layer, k, v, slots)`` then ``gather(layer, slots, out=out,
        start_pos=start_pos)`` in one launch where the layer allows it (bf16
        CONTIG / RING, Q <= max_q, contiguous k / v). ``out`` is (K, V) or
        (K, V, mask) as for ``gather``; returns it."""
        require_cuda(k, "k")
        require_cuda(v, "v")
        out_k, out_v = out[0], out[1]
        require_cuda(out_k, "out_k")
        require_cuda(out_v, "out_v")
        mask = out[2] if len(out) > 2 else None
        if mask is not None:
            require_cuda(mask, "out mask")
        self._bind()
        arr, n = self._slots(slots)
        sp = None if start_pos is None else (ctypes.c_int32 * n)(*[int(x) for x in start_pos])
        kd, vd = tensor_desc(k), tensor_desc(v)
        okd, ovd = tensor_desc(out_k), tensor_desc(out_v)
        md = None if mask is None else ctypes.byref(tensor_desc(mask))
        _check(self.lib.kvrt_append_gather_async(self._ctx, layer, n, arr, ctypes.byref(kd), ctypes.byref(vd), sp,
                                                 ctypes.byref(okd), ctypes.byref(ovd), md),
               "kvrt_append_gather_async")
        return out_k, out_v, mask

    def truncate(self, slot: int, new_len: int, layer: int = -1, generation: int = L.KVRT_ANY_GENERATION,
                 expected_len: int = -1) -> None:
        """Rollback to new_len positions: a length edit, no KV bytes move.

        Refused (``KVRTError`` code -2, nothing changes) below the slot's prefix
        mask; with a nonzero ``generation``, when the slot has been replaced
        since; with ``expected_len`` >= 0, when a layer's length is not that
        position; after a graph capture until :meth:`sync_lengths`
        (rewind_session_async's identity and position checks,
        impl.inc:3588-3618); and when the next query's window would need a row
        the layer no longer stores (a RING row a later position overwrote, a
        page :meth:`evict` released). ``new_len`` 0 always succeeds (a
        release). A rollback the host accepted against lengths that
        graph replays have since advanced is dropped on the device and
        reported by :meth:`health` (code -6)."""
        self._bind()
        _check(self.lib.kvrt_truncate(self._ctx, slot, layer, int(new_len), int(generation), int(expected_len)),
               "kvrt_truncate")

    def reserve(self, slot: int, positions: int) -> None:
        """PAGED: map the pages of the slot's next ``positions`` positions now, so
        that a captured graph of fused appends replays across page boundaries."""
        self._bind()
        _check(self.lib.kvrt_reserve_async(self._ctx, int(slot), int(positions)), "kvrt_reserve_async")

    def evict(self, slot: int, keep_from: int) -> None:
        self._own()
        _check(self.lib.kvrt_evict(self._ctx, slot, int(keep_from)), "kvrt_evict")

    def copy_prefix(self, src_slot: int, dst_slot: int, n_tokens: int,
                    generation: int = L.KVRT_ANY_GENERATION) -> int:
        """Clone the first n_tokens positions of src_slot (and its prefix mask) into
        dst_slot (all layers, one launch); returns dst_slot's new generation.
        A nonzero ``generation`` must be src_slot's current one."""
        self._bind()
        _check(self.lib.kvrt_copy_prefix_async(self._ctx, src_slot, dst_slot, int(n_tokens), int(generation)),
               "kvrt_copy_prefix_async")
        return self.slot_generation(dst_slot)

    def copy_session(self, dst_slot: int, src: "KVRuntime", src_slot: int, n_tokens: int,
                     generation: int = L.KVRT_ANY_GENERATION) -> int:
        """Copy the first n_tokens positions of ``src``'s src_slot into dst_slot of this
        runtime (identical topology), on this runtime's current stream; returns
        dst_slot's new generation."""
        self._bind()
        _check(self.lib.kvrt_copy_session_async(self._ctx, int(dst_slot), src._ctx, int(src_slot), int(n_tokens),
                                                int(generation)),
               "kvrt_copy_session_async")
        return self.slot_generation(dst_slot)

    def set_layer_rope(self, layer: int, inv_freq: Sequence[float] | None, scaling: float = 1.0) -> None:
        """RoPE inverse frequencies (head_dim / 2 fp32 values) of a layer for rollover."""
        self._bind()
        if inv_freq is None:
            _check(self.lib.kvrt_set_layer_rope(self._ctx, layer, None, 0, float(scaling)), "kvrt_set_layer_rope")
            return
        vals = [float(x) for x in inv_freq]
        arr = (ctypes.c_float * max(1, len(vals)))(*vals)
        _check(self.lib.kvrt_set_layer_rope(self._ctx, layer, arr, len(vals), float(scaling)), "kvrt_set_layer_rope")

    def rollover(self, slot: int, prefix_len: int, retained_rows: int,
                 generation: int = L.KVRT_ANY_GENERATION) -> None:
        """Keep the prefix, move the newest retained_rows rows behind it and
        rotate their keys by the position shift (layers with a RoPE table)."""
        self._bind()
        _check(self.lib.kvrt_rollover_async(self._ctx, int(slot), int(prefix_len), int(retained_rows),
                                            int(generation)),
               "kvrt_rollover_async")

    # ---- state -----------------------------------------------------------------
    def slot_info(self, slot: int) -> dict[str, int]:
        """generation, prefix_len, min_len and max_len of a slot."""
        self._own()
        info = L.KvrtSlotInfo()
        _check(self.lib.kvrt_slot_info_get(self._ctx, int(slot), ctypes.byref(info)), "kvrt_slot_info_get")
        return {name: int(getattr(info, name)) for name, _ in L.KvrtSlotInfo._fields_ if name != "reserved"}

    def slot_generation(self, slot: int) -> int:
        return self.slot_info(slot)["generation"]

    def seq_length(self, slot: int, layer: int = 0) -> int:
        self._own()
        out = ctypes.c_int32()
        _check(self.lib.kvrt_session_state(self._ctx, slot, layer, ctypes.byref(out)), "kvrt_session_state")
        return int(out.value)

    def sync_lengths(self) -> None:
        """Synchronise the bound stream and reload host lengths from the device
        (after HIP graph replays)."""
        self._own()
        _check(self.lib.kvrt_sync_lengths(self._ctx), "kvrt_sync_lengths")

    def counters(self) -> dict[str, int]:
        c = L.KvrtCounters()
        _check(self.lib.kvrt_get_counters(self._ctx, ctypes.byref(c)), "kvrt_get_counters")
        return {name: int(getattr(c, name)) for name, _ in L.KvrtCounters._fields_}

    def health(self) -> int:
        """Synchronise the bound stream and return the kvrt status code (0 = healthy)."""
        self._own()
        return int(self.lib.kvrt_health(self._ctx))

    def synchronize(self) -> None:
        """Wait for the context's work; afterwards it may move to another stream."""
        _check(self.health(), "kvrt_health")

    def layer_view(self, slot: int, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """HF-shaped [1, kv_heads, L, D] views of a slot's logical K/V.

        CONTIG layers return zero-copy views of the storage; RING and PAGED
        layers return a gathered copy (bf16, or fp32 dequantised for INT8).
        """
        spec = self.layers[self._owner(layer)]
        n = self.seq_length(slot, layer)
        if spec.layout == "contig":
            k, v, _, _ = self.storage(layer)
            return k[slot:slot + 1, :, :n, :], v[slot:slot + 1, :, :n, :]
        k, v, _ = self.gather(layer, [slot], mask_dtype=None)
        return k, v

    def close(self) -> None:
        if self._ctx:
            self.lib.kvrt_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self) -> None:  # pragma: no cover - interpreter teardown order
        try:
            self.close()
        except Exception:
            pass


def attend_tensors(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lengths: torch.Tensor,
                   scale: float, window: int = 0, out: torch.Tensor | None = None,
                   prefix_attention: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention over caller-owned K/V [n, kv_heads, Lmax, D] with per-item lengths.

    q [n, Hq, Q, D] bf16; lengths int32 [n] on the device. Query row i of item
    b sits at position lengths[b] - Q + i. ``prefix_attention`` [n, P]
    (int64 / int32 / bool, P <= 512) hides key j < P of item b where it is 0.
    """
    lib = L.load()
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (lengths, "lengths")):
        require_cuda(t, name)
    q = q.contiguous()
    lengths = lengths.to(torch.int32).contiguous()
    out = torch.empty_like(q) if out is None else out
    qd, kd, vd, od = tensor_desc(q), tensor_desc(k), tensor_desc(v), tensor_desc(out)
    pd = None
    if prefix_attention is not None:
        require_cuda(prefix_attention, "prefix_attention")
        prefix_attention = prefix_attention.contiguous()
        pd = ctypes.byref(tensor_desc(prefix_attention))
    _check(lib.kvrt_attend_tensors_async(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd),
                                         ctypes.c_void_p(lengths.data_ptr()), pd, ctypes.byref(od), float(scale),
                                         int(window), ctypes.c_void_p(current_stream_handle(q.device))),
           "kvrt_attend_tensors_async")
    return out


def tensors_status(device: torch.device | str | None = None) -> int:
    """Synchronise the current stream; report and clear the error flag of its
    tensor-attention workspace (0, or -6 when a length was clamped)."""
    dev = torch.device(device if device is not None else "cuda")
    return int(L.load().kvrt_tensors_status(ctypes.c_void_p(current_stream_handle(dev))))


def copy_rows(src: torch.Tensor, dst: torch.Tensor, rows: int) -> None:
    """dst[:, :, :rows] = src[:, :, :rows] for 4-D tensors (2- or 4-byte elements)."""
    lib = L.load()
    require_cuda(src, "src")
    require_cuda(dst, "dst")
    sd, dd = tensor_desc(src), tensor_desc(dst)
    _check(lib.kvrt_copy_rows_async(ctypes.byref(sd), ctypes.byref(dd), int(rows),
                                    ctypes.c_void_p(current_stream_handle(src.device))),
           "kvrt_copy_rows_async")
