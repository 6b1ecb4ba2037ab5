"""GPU parity of the talker attention (kvrt_attend_talker_async) against the
oracle's restatement of the reference talker masks (build_joint_mask_kernel /
build_audio_only_mask_kernel, native/qwen_talker/qwen_talker_kernels.cu:296-347)
followed by masked SDPA. Talker shape: 16 q heads over 8 kv heads, head_dim
128, bf16 CONTIG cache with rows written at explicit positions (stable text,
visible and not-yet-visible prefix frames, audio frames). Tolerance max-abs
1e-2 on bf16 outputs."""
from __future__ import annotations

import ctypes
import math
import random

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2
HQ, HKV, D = 16, 8, 128
SCALE = 1.0 / math.sqrt(D)


class _Talker:
    """A kvrt runtime and its host mirror, filled slot by slot."""

    def __init__(self, n, capacity, seed, hq=HQ, hkv=HKV, d=D, **kw):
        from kvrt import KVRuntime, LayerSpec

        self.hq, self.hkv, self.d, self.scale = hq, hkv, d, 1.0 / math.sqrt(d)
        self.rt = KVRuntime([LayerSpec(kv_heads=hkv, head_dim=d)], n, capacity, max_q=2, device="cuda", **kw)
        self.k = np.zeros((n, hkv, capacity, d), np.float32)
        self.v = np.zeros((n, hkv, capacity, d), np.float32)
        self.len = [0] * n
        self.gen = torch.Generator().manual_seed(seed)

    def write(self, slot, positions, scale=1.0):
        positions = list(positions)
        for c in range(0, len(positions), 128):
            pos = positions[c:c + 128]
            k = randn_bf16(self.gen, (1, self.hkv, len(pos), self.d), scale)
            v = randn_bf16(self.gen, (1, self.hkv, len(pos), self.d), scale)
            self.rt.write_positions(0, k.cuda(), v.cuda(), [slot], [pos])
            self.k[slot][:, pos] = to_np(k[0])
            self.v[slot][:, pos] = to_np(v[0])
            self.len[slot] = max(self.len[slot], max(pos) + 1)

    def fill(self, slot, m, q_rows, junk=True):
        """Stable text, visible prefix (minus the step's own prefix row),
        large-valued rows in the invisible part of the prefix region, audio
        frames before the step."""
        if m.prefix_start:
            self.write(slot, range(0, m.prefix_start))
        last_prefix = m.prefix_position - (1 if q_rows == 2 else 0)
        if last_prefix >= m.prefix_start:
            self.write(slot, range(m.prefix_start, last_prefix + 1))
        if junk and m.audio_start - m.prefix_position > 1:
            self.write(slot, range(m.prefix_position + 1, m.audio_start), scale=8.0)
        if m.audio_position > m.audio_start:
            self.write(slot, range(m.audio_start, m.audio_position))

    def step(self, slots, masks, q_rows):
        """Write the step's K/V rows, then attend; returns (out, reference)."""
        pos = [[m.prefix_position, m.audio_position] if q_rows == 2 else [m.audio_position] for m in masks]
        n = len(slots)
        k = randn_bf16(self.gen, (n, self.hkv, q_rows, self.d))
        v = randn_bf16(self.gen, (n, self.hkv, q_rows, self.d))
        self.rt.write_positions(0, k.cuda(), v.cuda(), slots, pos)
        for i, s in enumerate(slots):
            self.k[s][:, pos[i]] = to_np(k[i])
            self.v[s][:, pos[i]] = to_np(v[i])
            self.len[s] = max(self.len[s], max(pos[i]) + 1)
        q = randn_bf16(self.gen, (n, self.hq, q_rows, self.d), 0.5)
        out = self.rt.attend_talker(0, q.cuda(), slots, self.scale, masks)
        torch.cuda.synchronize()
        assert self.rt.health() == 0
        refs = []
        for i, (s, m) in enumerate(zip(slots, masks)):
            L = self.len[s]
            mask = O.talker_mask(q_rows, L, m.prefix_start, m.audio_start, m.prefix_position, m.audio_position,
                                 m.prefix_attention_mode, m.visible_prefix_count, m.prefix_log_gate)
            refs.append(O.attend_masked(to_np(q[i]), self.k[s][:, :L], self.v[s][:, :L], mask, self.scale))
        return out, refs


def _worst(out, refs):
    return max(float(np.abs(to_np(out[i]) - r).max()) for i, r in enumerate(refs))


@pytest.mark.parametrize("q_rows", [2, 1])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_talker_step_matches_oracle(q_rows, mode):
    from kvrt import TalkerMask

    t = _Talker(1, 512, seed=10 * mode + q_rows)
    m = TalkerMask(prefix_start=37, audio_start=60, prefix_position=45, audio_position=300,
                   prefix_attention_mode=mode, visible_prefix_count=9 if mode == 2 else 0, prefix_log_gate=-2.0)
    t.fill(0, m, q_rows)
    out, refs = t.step([0], [m], q_rows)
    assert _worst(out, refs) <= ATOL


def test_batched_slots_with_mixed_modes_and_lengths():
    """Three sessions in one launch: no stable text, a long audio tail
    (many key splits) and a gated prefix, each with its own ranges."""
    from kvrt import TalkerMask

    t = _Talker(3, 2048, seed=3)
    masks = [
        TalkerMask(0, 16, 7, 40, prefix_attention_mode=0),
        TalkerMask(120, 160, 155, 1900, prefix_attention_mode=1),
        TalkerMask(64, 96, 70, 500, prefix_attention_mode=2, visible_prefix_count=7, prefix_log_gate=-8.0),
    ]
    for s, m in enumerate(masks):
        t.fill(s, m, 2)
    out, refs = t.step([0, 1, 2], masks, 2)
    assert _worst(out, refs) <= ATOL
    # the same sessions' audio-only step at the next audio position
    nxt = [TalkerMask(m.prefix_start, m.audio_start, m.prefix_position, m.audio_position + 1,
                      m.prefix_attention_mode, m.visible_prefix_count, m.prefix_log_gate) for m in masks]
    out, refs = t.step([2, 0, 1], [nxt[2], nxt[0], nxt[1]], 1)
    assert _worst(out, refs) <= ATOL


@pytest.mark.parametrize("gate,count", [(6.0, 1), (-30.0, 4), (0.0, 1000)])
def test_gate_extremes(gate, count):
    from kvrt import TalkerMask

    t = _Talker(1, 256, seed=int(abs(gate)) + count)
    m = TalkerMask(10, 40, 30, 200, prefix_attention_mode=2, visible_prefix_count=count, prefix_log_gate=gate)
    t.fill(0, m, 2)
    out, refs = t.step([0], [m], 2)
    assert _worst(out, refs) <= ATOL


def test_last_capacity_row_and_single_stable_key():
    from kvrt import TalkerMask

    t = _Talker(1, 300, seed=21)
    m = TalkerMask(1, 3, 1, 299, prefix_attention_mode=1)
    t.fill(0, m, 2)
    out, refs = t.step([0], [m], 2)
    assert _worst(out, refs) <= ATOL


def test_q1_cursor_phase_is_the_causal_decode():
    """After every prefix frame is real, the reference's Q1 step uses the
    cursor mask k <= cursor (qwen_talker_kernels.cu:349-359): the plain causal
    decode over the slot's length, equal to the talker mask with the whole
    prefix visible in mode 0."""
    from kvrt import TalkerMask

    t = _Talker(1, 512, seed=33)
    m = TalkerMask(20, 50, 49, 333, prefix_attention_mode=0)
    t.fill(0, m, 1)
    out, refs = t.step([0], [m], 1)
    assert _worst(out, refs) <= ATOL
    q = randn_bf16(t.gen, (1, HQ, 1, D), 0.5)
    causal = t.rt.attend(0, q.cuda(), [0], SCALE)
    talker = t.rt.attend_talker(0, q.cuda(), [0], SCALE, [m])
    torch.cuda.synchronize()
    ref = O.attend(to_np(q[0]), t.k[0][:, :334], t.v[0][:, :334], np.array([333]), SCALE)
    assert float(np.abs(to_np(causal[0]) - ref).max()) <= ATOL
    assert float((causal.float() - talker.float()).abs().max()) <= ATOL


def _raw_call(rt, q, masks):
    from kvrt import _lib as L
    from kvrt.runtime import tensor_desc

    out = torch.empty_like(q)
    arr = (ctypes.c_int32 * len(masks))(*range(len(masks)))
    marr = (L.KvrtTalkerMask * len(masks))(*masks)
    qd, od = tensor_desc(q), tensor_desc(out)
    rt._bind()
    return rt.lib.kvrt_attend_talker_async(rt._ctx, 0, len(masks), arr, ctypes.byref(qd), ctypes.byref(od),
                                           SCALE, marr)


def _cmask(ps, as_, pp, ap, mode=0, count=0, gate=-8.0):
    from kvrt import _lib as L

    m = L.KvrtTalkerMask()
    m.prefix_start, m.audio_start, m.prefix_position, m.audio_position = ps, as_, pp, ap
    m.prefix_attention_mode, m.visible_prefix_count, m.prefix_log_gate = mode, count, gate
    return m


def test_invalid_talker_calls_are_refused_before_any_launch():
    from kvrt import KVRTError, KVRuntime, LayerSpec, TalkerMask
    from kvrt import _lib as L

    t = _Talker(1, 128, seed=1)
    t.write(0, range(0, 64))
    q = torch.zeros((1, HQ, 2, D), dtype=torch.bfloat16, device="cuda")
    before = t.rt.counters()["launches"]
    assert _raw_call(t.rt, q, [_cmask(2, 8, 4, 10, mode=3)]) == L.KVRT_EINVAL
    assert _raw_call(t.rt, q, [_cmask(2, 8, 4, 10, mode=2, count=0)]) == L.KVRT_EINVAL
    assert _raw_call(t.rt, q, [_cmask(2, 8, 4, 10, gate=float("nan"))]) == L.KVRT_EINVAL
    assert _raw_call(t.rt, q, [_cmask(2, 8, 8, 10)]) == L.KVRT_EINVAL      # prefix position in the audio region
    assert _raw_call(t.rt, q, [_cmask(5, 8, 4, 10)]) == L.KVRT_EINVAL      # prefix position before prefix start
    assert _raw_call(t.rt, q, [_cmask(2, 8, 4, 7)]) == L.KVRT_EINVAL       # audio position before audio start
    assert _raw_call(t.rt, q, [_cmask(2, 8, 4, 64)]) == L.KVRT_ESTATE      # audio row not written yet
    q3 = torch.zeros((1, HQ, 3, D), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(KVRTError):
        t.rt.attend_talker(0, q3, [0], SCALE, [TalkerMask(2, 8, 4, 10)])
    assert t.rt.counters()["launches"] == before
    ring = KVRuntime([LayerSpec(kv_heads=HKV, head_dim=D, layout="ring", window=16, ring_rows=17)], 1, 128,
                     max_q=2, device="cuda")
    x = torch.zeros((1, HKV, 20, D), dtype=torch.bfloat16, device="cuda")
    ring.import_(0, 0, x, x)
    with pytest.raises(KVRTError) as e:
        ring.attend_talker(0, q, [0], SCALE, [TalkerMask(2, 8, 4, 10)])
    assert e.value.code == L.KVRT_EINVAL
    assert t.rt.health() == 0 and ring.health() == 0


def _talker_cases(n_cases: int, seed: int) -> list[tuple]:
    r = random.Random(seed)
    out = []
    while len(out) < n_cases:
        d, hkv, g, q_rows = r.choice([64, 128, 256, 512]), r.choice([1, 2, 4, 8]), r.choice([1, 2, 4, 8]), r.choice([1, 2])
        if g * q_rows > 16:
            continue
        masks = []
        for _ in range(r.choice([1, 2, 3, 4])):
            ps = r.choice([0, r.randint(1, 200)])
            pp = ps + r.randint(0, 40)
            as_ = pp + 1 + r.choice([0, r.randint(1, 60)])
            ap = as_ + r.choice([0, r.randint(1, 60), r.randint(100, 3000)])
            mode = r.choice([0, 1, 2])
            count = r.randint(1, 50) if mode == 2 else 0
            masks.append((ps, as_, pp, ap, mode, count, r.choice([-8.0, -2.0, 0.5])))
        out.append((d, hkv, g, q_rows, tuple(masks), r.choice([0, 64, 512]), r.randrange(1 << 30)))
    return out


TALKER_CASES = _talker_cases(16, 2718)


@pytest.mark.parametrize("case", TALKER_CASES, ids=[
    f"d{c[0]}-h{c[1]}g{c[2]}-q{c[3]}-n{len(c[4])}-wg{c[5]}" for c in TALKER_CASES])
def test_random_talker_shapes_and_masks(case):
    """Seeded random talker steps: head_dim 64..512, 1..8 KV heads, GQA groups
    1..8, JOINT (Q 2) and audio-only (Q 1) rows, 1..4 sessions each with its
    own stable text, prefix, reserved and audio ranges (audio tails up to
    3000 positions), modes 0 / 1 / 2 with random counts and gates, and
    several workgroup budgets."""
    from kvrt import TalkerMask

    d, hkv, g, q_rows, ms, wgs, seed = case
    masks = [TalkerMask(ps, as_, pp, ap, prefix_attention_mode=mode, visible_prefix_count=count,
                        prefix_log_gate=gate) for ps, as_, pp, ap, mode, count, gate in ms]
    cap = max(m.audio_position for m in masks) + 8
    t = _Talker(len(masks), cap, seed, hq=hkv * g, hkv=hkv, d=d, decode_wgs=wgs)
    for s, m in enumerate(masks):
        t.fill(s, m, q_rows)
    slots = list(range(len(masks)))
    random.Random(seed).shuffle(slots)
    out, refs = t.step(slots, [masks[s] for s in slots], q_rows)
    assert _worst(out, refs) <= ATOL
