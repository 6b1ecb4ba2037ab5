"""CPU oracle for the KV append / gather / truncate / attend hot path.

TEST INFRASTRUCTURE ONLY. This module restates, in numpy, what the reference
computes on this path. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker;
the product (``gemma-4-omni_amd/kvrt``) never imports or calls it.

Semantics restated (reference paths relative to the andr-lab/gemma-4-omni
tree; HF = transformers.cache_utils, a third-party dependency pinned at
5.5.0 by the reference Dockerfile:49-51):

* append  — HF ``DynamicLayer.update`` = ``torch.cat([keys, k], dim=-2)``
  (cache_utils.py:127-146), reached via duplex_kernel/kv_cache.py:95-97;
  native: gemma4_cache_append_async (native/gemma4_listener_microbatch/
  gemma4_listener_cache.cu:182-215), write_audio_kv (native/qwen_talker/
  qwen_talker_kernels.cu:207-251).
* truncate — ``_slice_kv`` keep the first ``keep_len`` rows
  (duplex_kernel/kv_cache.py:205-216); native cursor edit
  gemma4_cache_truncate_async (gemma4_listener_cache.cu:409-421).
* gather  — ``_StaticPaddingWorkspace.padded/padded_mask``: zero buffer of the
  target length, valid prefix copied, mask tail ``False`` / ``finfo.min``
  (duplex_kernel/shape_stable_listener.py:28-69).
* attend  — ``F.scaled_dot_product_attention`` over ``repeat_kv``'d K/V with
  fp32 softmax (shape_stable_listener.py:241-251); visibility as
  kernel_build_explicit_sdpa_mask (gemma4_listener_kernels.cuh:500-525):
  key k visible to query position p iff prefix_valid (k >= P or
  prefix_attention[k] != 0, :517-518; P = 0 without a mask), k <= p and,
  for window W > 0, k >= p - W + 1; GQA q head h reads kv head
  h // (Hq / Hkv). The same prefix term gates every listener attention path
  (kernel_stream_sdpa_q4_bf16 :595-597, kernel_prefill_sdpa_bf16 :743-745,
  gemma4_listener_attention_ordered.cu:96-101,
  gemma4_listener_microbatch_impl.inc:2659-2660).
* canonical prefix mask — kernel_set_canonical_prefix_mask
  (gemma4_listener_kernels.cuh:111-118): position 0 (BOS) and the last
  position (BOA) visible, the 32 text slots between them not; 34 positions
  by default (GEMMA4_CANONICAL_PREFIX_LEN, generated_topology.h:22; the
  Python side asserts the same mask, duplex_kernel/listener.py:1983-1988).
* sliding retention — HF ``DynamicSlidingWindowLayer`` keeps the last W-1
  rows after an update (cache_utils.py:229-261); window start of the native
  cache ``base - W + 1`` (gemma4_listener_cache.cu:448-452).
* window range — gemma4_q4_range_from_position
  (gemma4_listener_kernels.cuh:23-49).
* RoPE rebase — kernel_rope_rebase_bf16 / kernel_rope_bf16
  (native/gemma4_listener_microbatch/gemma4_listener_kernels.cuh:294-360),
  rollover compaction gemma4_cache_rebase_async (gemma4_listener_cache.cu:
  303-351): ``rope_rebase``, ``OracleCache.rollover``.
* talker masks — build_joint_mask_kernel / build_audio_only_mask_kernel
  (native/qwen_talker/qwen_talker_kernels.cu:296-347, launchers :759-807):
  ``talker_mask`` and ``attend_masked``.
* int8 KV (no reference implementation; closed form): per (token, head)
  scale = amax / 127 (fp32), q = clamp(round_half_even(x / scale), -127, 127),
  dequant = q * scale (fp32); amax == 0 gives scale 0 and q = 0.

bf16 values are carried as float32 arrays holding exactly-representable
bf16 values (or as uint16 bit patterns where bitwise identity is asserted).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit pattern, round to nearest even (quiet NaN kept)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return (r & 0xFFFF).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 value (returned as float32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---------------------------------------------------------------------------
# window / position math
# ---------------------------------------------------------------------------


def q_range_from_position(base_position: int, q_len: int, capacity: int, sliding_window: int):
    """(total_k_len, start_offset, valid) of a Q-row step at base_position.

    Restates gemma4_q4_range_from_position (gemma4_listener_kernels.cuh:23-39).
    """
    total = base_position + q_len
    start = base_position - sliding_window + 1 if (sliding_window > 0 and base_position >= sliding_window) else 0
    valid = q_len > 0 and total <= capacity and start < total
    return min(total, 2**32 - 1), start, valid


def visible_range(query_position: int, window: int) -> tuple[int, int]:
    """Inclusive [lo, hi] of the keys visible to one query position."""
    lo = max(0, query_position - window + 1) if window > 0 else 0
    return lo, query_position


def ring_capacity(window: int, max_q: int, max_seq_len: int) -> int:
    """Rows a sliding layer must retain: W + q - 1, capped by max_seq_len.

    Restates derive_contract (native/gemma4_listener_microbatch/
    sliding_repeat_capacity.h:30-60).
    """
    return min(window + max_q - 1, max_seq_len)


# ---------------------------------------------------------------------------
# int8 quantisation
# ---------------------------------------------------------------------------


def quantize_int8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric int8 per row (last axis): returns (q int8 [..., D], scale fp32 [...])."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x), axis=-1).astype(np.float32)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(x / scale[..., None]).astype(np.float32)
    r = np.where(amax[..., None] > 0, np.clip(r, -127, 127), 0)
    return r.astype(np.int8), scale


def dequantize_int8(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    return (q.astype(np.float32) * scale[..., None].astype(np.float32)).astype(np.float32)


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

CANONICAL_PREFIX_LEN = 34  # GEMMA4_CANONICAL_PREFIX_LEN (generated_topology.h:22)


def canonical_prefix_mask(length: int = CANONICAL_PREFIX_LEN) -> np.ndarray:
    """int64 [length]: 1 at position 0 and length - 1, else 0
    (kernel_set_canonical_prefix_mask, gemma4_listener_kernels.cuh:111-118)."""
    idx = np.arange(length)
    return ((idx == 0) | (idx == length - 1)).astype(np.int64)


def prefix_valid(key_positions: np.ndarray, prefix_attention: np.ndarray | None) -> np.ndarray:
    """Boolean per key: k >= P or prefix_attention[k] != 0 (P = its length;
    no mask: all True), gemma4_listener_kernels.cuh:517-518."""
    kp = np.asarray(key_positions)
    if prefix_attention is None:
        return np.ones(kp.shape, dtype=bool)
    pm = np.asarray(prefix_attention).reshape(-1)
    inside = (kp >= 0) & (kp < pm.size)
    out = np.ones(kp.shape, dtype=bool)
    out[inside] = pm[kp[inside]] != 0
    return out


def attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, q_positions: np.ndarray, scale: float,
           window: int = 0, key_positions: np.ndarray | None = None,
           prefix_attention: np.ndarray | None = None) -> np.ndarray:
    """Masked GQA attention, float64 softmax.

    q [Hq, Q, D]; k, v [Hkv, L, D] (already dequantised, float32);
    q_positions [Q] absolute query positions; key_positions [L] absolute key
    positions (default 0..L-1); prefix_attention [P] (or None): key position
    k < P is visible only where prefix_attention[k] != 0. Returns float32
    [Hq, Q, D]; a row with no visible key is 0.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    hq, qn, d = q.shape
    hkv, n_keys, _ = k.shape
    if hq % hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    g = hq // hkv
    kp = np.arange(n_keys) if key_positions is None else np.asarray(key_positions)
    pv = prefix_valid(kp, prefix_attention)
    out = np.zeros((hq, qn, d), dtype=np.float64)
    for h in range(hq):
        kh = h // g  # HF repeat_kv: kv head j serves q heads j*g .. j*g+g-1
        s = (q[h] @ k[kh].T) * float(scale)  # [Q, L]
        for i in range(qn):
            lo, hi = visible_range(int(q_positions[i]), window)
            vis = (kp >= lo) & (kp <= hi) & pv
            if not vis.any():
                continue
            row = np.where(vis, s[i], -np.inf)
            row = row - row[vis].max()
            p = np.exp(row)
            p /= p.sum()
            out[h, i] = p @ v[kh]
    return out.astype(np.float32)


# ---------------------------------------------------------------------------
# talker masks (JOINT Q = 2 and audio-only Q = 1)
# ---------------------------------------------------------------------------

MASKED_BF16 = float(bf16_bits_to_f32(np.array([0xFF7F], dtype=np.uint16))[0])  # -3.3895313892515355e38


def talker_gate(mode: int, visible_prefix_count: int, prefix_log_gate: float) -> float:
    """Additive value of a gated prefix key: fp32 ``gate - logf(count)`` stored
    as bf16 (qwen_talker_kernels.cu:774-777 computes it, :318-320 / :344-346
    write it through ``__float2bfloat16``); 0 outside mode 2."""
    if mode != 2:
        return 0.0
    logc = np.float32(np.log(float(visible_prefix_count)))  # correctly rounded logf
    g = np.float32(np.float32(prefix_log_gate) - logc)
    return float(round_bf16(np.array([g], dtype=np.float32))[0])


def talker_mask(rows: int, key_len: int, prefix_start: int, audio_start: int, prefix_position: int,
                audio_position: int, mode: int, visible_prefix_count: int = 0,
                prefix_log_gate: float = -8.0) -> np.ndarray:
    """Additive mask [rows, key_len] (float32 holding bf16 values).

    rows = 2 restates build_joint_mask_kernel (native/qwen_talker/
    qwen_talker_kernels.cu:296-321: row 0 the prefix query, row 1 the audio
    query); rows = 1 restates build_audio_only_mask_kernel (:323-347, with
    prefix_position = visible_prefix_position). Per key position p:
    stable = p < prefix_start; visible_prefix = prefix_start <= p <=
    prefix_position; audio = audio_start <= p <= audio_position; allowed =
    stable or (visible_prefix and (prefix row or mode != 1)) or (audio row and
    audio); value 0 if allowed else bf16 finfo.min, replaced by the gate for
    an audio row on a visible-prefix key in mode 2.
    """
    if rows not in (1, 2):
        raise ValueError("talker masks have 1 (audio-only) or 2 (joint) query rows")
    p = np.arange(key_len)
    stable = p < prefix_start
    vis_prefix = (p >= prefix_start) & (p <= prefix_position)
    audio = (p >= audio_start) & (p <= audio_position)
    gate = talker_gate(mode, visible_prefix_count, prefix_log_gate)
    out = np.empty((rows, key_len), dtype=np.float32)
    for r in range(rows):
        audio_row = rows == 1 or r == 1
        allowed = stable | (vis_prefix & (not audio_row or mode != 1)) | (audio & audio_row)
        val = np.where(allowed, np.float32(0.0), np.float32(MASKED_BF16))
        if audio_row and mode == 2:
            val = np.where(vis_prefix, np.float32(gate), val)
        out[r] = val
    return out


def attend_masked(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray, scale: float) -> np.ndarray:
    """softmax(q.k * scale + mask) v per q head, float64; GQA by repeat_kv.

    q [Hq, Q, D]; k, v [Hkv, L, D]; mask [Q, L] additive (broadcast over
    heads), as the talker's masked SDPA (qwen_talker_aten_attention.cpp:150-160).
    Returns float32 [Hq, Q, D].
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    hq, qn, _ = q.shape
    g = hq // k.shape[0]
    out = np.zeros(q.shape, dtype=np.float64)
    for h in range(hq):
        s = (q[h] @ k[h // g].T) * float(scale) + np.asarray(mask, dtype=np.float64)
        s = s - s.max(axis=1, keepdims=True)
        w = np.exp(s)
        out[h] = (w / w.sum(axis=1, keepdims=True)) @ v[h // g]
    return out.astype(np.float32)


# ---------------------------------------------------------------------------
# RoPE (forward and rebase of cached keys)
# ---------------------------------------------------------------------------


def rope_cos_sin(delta_or_pos: float, inv_freq: np.ndarray, scaling: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """bf16 (cos, sin) per pair: f = fp32(p * inv_freq[i]); bf16(fp32(cos f) * scaling).

    Restates the angle step of kernel_rope_bf16 / kernel_rope_rebase_bf16
    (native/gemma4_listener_microbatch/gemma4_listener_kernels.cuh:294-360)
    with cos / sin of the fp32 argument correctly rounded to fp32.
    """
    f = (np.float32(delta_or_pos) * np.asarray(inv_freq, np.float32)).astype(np.float32)
    c = np.cos(f.astype(np.float64)).astype(np.float32) * np.float32(scaling)
    s = np.sin(f.astype(np.float64)).astype(np.float32) * np.float32(scaling)
    return round_bf16(c.astype(np.float32)), round_bf16(s.astype(np.float32))


def rope_rotate(x: np.ndarray, cos_b: np.ndarray, sin_b: np.ndarray) -> np.ndarray:
    """Rotate the (dim i, dim i + D/2) pairs of bf16 rows x [..., D] with bf16
    pointwise products and bf16 add / subtract:
    x1' = bf16(bf16(x1 c) - bf16(x2 s)), x2' = bf16(bf16(x2 c) + bf16(x1 s))
    (gemma4_listener_kernels.cuh:323-330, :350-359)."""
    x = np.asarray(x, np.float32)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    x1c, x2s = round_bf16(x1 * cos_b), round_bf16(x2 * sin_b)
    x2c, x1s = round_bf16(x2 * cos_b), round_bf16(x1 * sin_b)
    return np.concatenate([round_bf16((x1c - x2s).astype(np.float32)),
                           round_bf16((x2c + x1s).astype(np.float32))], axis=-1)


def rope_rebase(x: np.ndarray, inv_freq: np.ndarray, delta: int, scaling: float = 1.0) -> np.ndarray:
    """kernel_rope_rebase_bf16: rotate already-rotated keys by delta positions."""
    c, s = rope_cos_sin(delta, inv_freq, scaling)
    return rope_rotate(x, c, s)


def gemma_inv_freq(head_dim: int, base: float, rotary_pairs: int | None = None) -> np.ndarray:
    """fp32 inverse frequencies 1 / base^(2i / D), zero beyond rotary_pairs
    (gemma4_listener.cu:1840-1880: sliding D 256 all 128 pairs; full D 512
    proportional RoPE with 64 rotated pairs)."""
    half = head_dim // 2
    pairs = half if rotary_pairs is None else rotary_pairs
    i = np.arange(half)
    out = (1.0 / np.power(np.float64(base), (2.0 * i) / head_dim)).astype(np.float32)
    out[pairs:] = 0.0
    return out


def attend_bruteforce(q, k, v, q_positions, scale, window=0, prefix_attention=None):
    """Pure-Python-loop attention (tiny shapes only): golden-vector generator."""
    hq, qn, d = len(q), len(q[0]), len(q[0][0])
    hkv, n_keys = len(k), len(k[0])
    g = hq // hkv
    out = [[[0.0] * d for _ in range(qn)] for _ in range(hq)]
    pm = [] if prefix_attention is None else [int(x) for x in prefix_attention]
    import math
    for h in range(hq):
        kh = h // g
        for i in range(qn):
            p_pos = q_positions[i]
            vis = [j for j in range(n_keys) if j <= p_pos and (window <= 0 or j >= p_pos - window + 1)
                   and (j >= len(pm) or pm[j] != 0)]
            if not vis:
                continue
            scores = {j: sum(q[h][i][t] * k[kh][j][t] for t in range(d)) * scale for j in vis}
            m = max(scores.values())
            w = {j: math.exp(s - m) for j, s in scores.items()}
            z = sum(w.values())
            for t in range(d):
                out[h][i][t] = sum(w[j] * v[kh][j][t] for j in vis) / z
    return out


# ---------------------------------------------------------------------------
# logical cache model
# ---------------------------------------------------------------------------


@dataclass
class OracleLayer:
    kv_heads: int
    head_dim: int
    window: int = 0
    int8: bool = False


class _Rows:
    """Rows [H, n, ...] with amortised O(1) append (capacity doubling)."""

    def __init__(self, heads: int, tail: tuple, dtype) -> None:
        self.buf = np.zeros((heads, 16) + tail, dtype=dtype)
        self.n = 0

    def view(self) -> np.ndarray:
        return self.buf[:, :self.n]

    def append(self, x: np.ndarray) -> None:
        q = x.shape[1]
        if self.n + q > self.buf.shape[1]:
            grown = np.zeros((self.buf.shape[0], max(2 * self.buf.shape[1], self.n + q)) + self.buf.shape[2:],
                             dtype=self.buf.dtype)
            grown[:, :self.n] = self.buf[:, :self.n]
            self.buf = grown
        self.buf[:, self.n:self.n + q] = x
        self.n += q

    def truncate(self, n: int) -> None:
        self.n = min(self.n, int(n))


@dataclass
class OracleCache:
    """Logical KV of n_slots sessions: per (slot, layer) full-history rows.

    Keeps every appended row (float32 values; int8 layers keep the quantised
    ints and scales), which is the logical view all layouts must reproduce.
    """

    layers: list
    n_slots: int
    rows: dict = field(default_factory=dict)
    prefix: dict = field(default_factory=dict)  # slot -> prefix_attention [P] (per slot, all layers)

    def set_prefix_attention(self, slot: int, mask) -> None:
        """The slot's prefix-attention mask (None clears it), imported with the
        session (gemma4_listener_microbatch_impl.inc:2590-2621)."""
        if mask is None or np.asarray(mask).size == 0:
            self.prefix.pop(slot, None)
        else:
            self.prefix[slot] = np.asarray(mask).reshape(-1).astype(np.int64).copy()

    def copy_prefix_attention(self, src: int, dst: int) -> None:
        """Clones carry the source's mask (impl.inc:4100, :4162)."""
        self.set_prefix_attention(dst, self.prefix.get(src))

    def _get(self, slot, layer):
        key = (slot, layer)
        if key not in self.rows:
            spec = self.layers[layer]
            dt = np.int8 if spec.int8 else np.float32
            self.rows[key] = (_Rows(spec.kv_heads, (spec.head_dim,), dt), _Rows(spec.kv_heads, (spec.head_dim,), dt),
                              _Rows(spec.kv_heads, (), np.float32), _Rows(spec.kv_heads, (), np.float32))
        return self.rows[key]

    def length(self, slot: int, layer: int) -> int:
        return self._get(slot, layer)[0].n

    def append(self, slot: int, layer: int, k: np.ndarray, v: np.ndarray) -> None:
        """k, v [Hkv, Q, D] float32 (bf16 values): concatenate along positions."""
        kr, vr, ks, vs = self._get(slot, layer)
        if self.layers[layer].int8:
            kq, ksc = quantize_int8(k)
            vq, vsc = quantize_int8(v)
            kr.append(kq)
            vr.append(vq)
            ks.append(ksc)
            vs.append(vsc)
        else:
            kr.append(np.asarray(k, np.float32))
            vr.append(np.asarray(v, np.float32))

    def truncate(self, slot: int, layer: int, keep_len: int) -> None:
        for r in self._get(slot, layer):
            r.truncate(keep_len)

    def copy_prefix(self, src: int, dst: int, layer: int, n: int) -> None:
        """dst's rows of a layer become the first n rows of src's
        (gemma4_cache_copy_async, gemma4_listener_cache.cu:306-345)."""
        for a, b in zip(self._get(src, layer), self._get(dst, layer)):
            b.truncate(0)
            if n:
                b.append(a.view()[:, :n].copy())

    def rollover(self, slot: int, layer: int, prefix_len: int, retained: int,
                 inv_freq: np.ndarray | None = None, scaling: float = 1.0) -> None:
        """Keep [0, prefix_len), move the last `retained` rows behind it and
        rotate their keys by prefix_len - (L - retained) positions
        (gemma4_cache_rebase_async, gemma4_listener_cache.cu:303-351, then
        kernel_rope_rebase_bf16 per layer, impl.inc:3835-3895)."""
        if self.layers[layer].int8:
            raise ValueError("rollover rotates bf16 keys only")
        kr, vr, ks, vs = self._get(slot, layer)
        L = kr.n
        if not (0 < prefix_len and 0 < retained and L > prefix_len + retained):
            raise ValueError("rollover needs L > prefix_len + retained > 0")
        k, v = kr.view(), vr.view()
        moved_k = k[:, L - retained:].copy()
        if inv_freq is not None:
            moved_k = rope_rebase(moved_k, inv_freq, prefix_len - (L - retained), scaling)
        new_k = np.concatenate([k[:, :prefix_len], moved_k], axis=1)
        new_v = np.concatenate([v[:, :prefix_len], v[:, L - retained:]], axis=1)
        kr.truncate(0)
        vr.truncate(0)
        kr.append(new_k)
        vr.append(new_v)

    def values(self, slot: int, layer: int) -> tuple[np.ndarray, np.ndarray]:
        """Dequantised float32 K, V [Hkv, L, D]."""
        kr, vr, ks, vs = self._get(slot, layer)
        if self.layers[layer].int8:
            return dequantize_int8(kr.view(), ks.view()), dequantize_int8(vr.view(), vs.view())
        return kr.view(), vr.view()

    def gather(self, layer: int, slots: list[int], lmax: int, start: list[int] | None = None):
        """Padded [n, Hkv, lmax, D] float32 K, V and bool mask [n, lmax]."""
        spec = self.layers[layer]
        n = len(slots)
        ko = np.zeros((n, spec.kv_heads, lmax, spec.head_dim), np.float32)
        vo = np.zeros_like(ko)
        mask = np.zeros((n, lmax), bool)
        for i, s in enumerate(slots):
            kk, vv = self.values(s, layer)
            st = 0 if start is None else start[i]
            m = kk.shape[1] - st
            ko[i, :, :m] = kk[:, st:]
            vo[i, :, :m] = vv[:, st:]
            mask[i, :m] = True
        return ko, vo, mask

    def attend(self, slot: int, layer: int, q: np.ndarray, scale: float) -> np.ndarray:
        """q [Hq, Q, D] at the last Q positions of (slot, layer)."""
        kk, vv = self.values(slot, layer)
        n_keys = kk.shape[1]
        qn = q.shape[1]
        window = self.layers[layer].window
        lo = 0 if window <= 0 else max(0, n_keys - qn - window + 1)
        pos = np.arange(n_keys - qn, n_keys)
        # keys below the first query's window are never visible: skip them
        return attend(q, kk[:, lo:], vv[:, lo:], pos, scale, window, key_positions=np.arange(lo, n_keys),
                      prefix_attention=self.prefix.get(slot))


def sliding_retained(length: int, window: int) -> tuple[int, int]:
    """[start, length) rows an HF DynamicSlidingWindowLayer keeps after updates."""
    return max(0, length - (window - 1)), length
