"""GPU parity of the slot lifecycle: clone (kvrt_copy_prefix_async), copy
between contexts (kvrt_copy_session_async) and rollover with RoPE rebase
(kvrt_rollover_async + kvrt_set_layer_rope) against the oracle, bit-exact on
the stored rows; then the real 35-layer Gemma-4 listener topology (15 owned
layers, layers 15-34 reading 13 / 14, D 256 sliding and D 512 full layers)
stepped, rolled over and cloned with attention checked on every layer
(max-abs 1e-2)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2


def _fill(rt, orc, slot, layer, n, gen, hkv, d, scale=1.0):
    k, v = randn_bf16(gen, (1, hkv, n, d), scale), randn_bf16(gen, (1, hkv, n, d), scale)
    rt.import_(slot, layer, k.cuda(), v.cuda())
    orc.append(slot, layer, to_np(k[0]), to_np(v[0]))


def _check_rows(rt, orc, slot, layer, start=0):
    """The slot's logical rows [start, L) equal the oracle's, bit for bit."""
    L = rt.seq_length(slot, layer)
    assert L == orc.length(slot, layer)
    k, v, _ = rt.gather(layer, [slot], start_pos=[start], mask_dtype=None)
    torch.cuda.synchronize()
    ok, ov = orc.values(slot, layer)
    if k.dtype == torch.bfloat16:
        assert np.array_equal(bits(k[0]), O.f32_to_bf16_bits(ok[:, start:]))
        assert np.array_equal(bits(v[0]), O.f32_to_bf16_bits(ov[:, start:]))
    else:
        assert np.array_equal(to_np(k[0]), ok[:, start:]) and np.array_equal(to_np(v[0]), ov[:, start:])


@pytest.mark.parametrize("layout", ["contig", "paged"])
@pytest.mark.parametrize("length,prefix,retained", [
    (2000, 300, 128),   # far apart (the usual rollover at a full cache)
    (140, 20, 116),     # source and destination ranges overlap
    (9, 2, 6),          # minimum shapes
])
def test_rollover_rows_match_oracle_bit_exact(layout, length, prefix, retained):
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(length + retained)
    kw = dict(block_size=16, pool_pages=600) if layout == "paged" else {}
    specs = [LayerSpec(kv_heads=1, head_dim=256, layout=layout, window=512),
             LayerSpec(kv_heads=1, head_dim=512, layout=layout),
             LayerSpec(kv_heads=2, head_dim=128, layout=layout),      # no RoPE table: moved unrotated
             LayerSpec(kv_heads=1, head_dim=256, layout=layout, shared_src=0)]
    rt = KVRuntime(specs, 2, 2048, max_q=2, device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(s.kv_heads, s.head_dim) for s in specs[:3]], 2)
    for slot, n in ((0, length), (1, 77)):
        for layer, s in enumerate(specs[:3]):
            _fill(rt, orc, slot, layer, n, gen, s.kv_heads, s.head_dim, 2.0)
    inv = {0: O.gemma_inv_freq(256, 1e4), 1: O.gemma_inv_freq(512, 1e6, 64)}
    rt.set_layer_rope(0, inv[0].tolist())
    rt.set_layer_rope(1, inv[1].tolist())
    rt.rollover(0, prefix, retained)
    for layer in range(3):
        orc.rollover(0, layer, prefix, retained, inv.get(layer))
    assert rt.health() == 0
    for layer in range(3):
        _check_rows(rt, orc, 0, layer)
        _check_rows(rt, orc, 1, layer)  # the other slot is untouched
    assert rt.seq_length(0, 3) == prefix + retained


def test_rollover_then_decode_continues_at_the_compacted_position():
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(9)
    rt = KVRuntime([LayerSpec(kv_heads=1, head_dim=256, window=64)], 1, 1024, max_q=2, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, 256, 64)], 1)
    _fill(rt, orc, 0, 0, 900, gen, 1, 256)
    inv = O.gemma_inv_freq(256, 1e4)
    rt.set_layer_rope(0, inv.tolist())
    rt.rollover(0, 40, 50)
    orc.rollover(0, 0, 40, 50, inv)
    for _ in range(3):
        q = randn_bf16(gen, (1, 8, 2, 256), 0.5)
        k, v = randn_bf16(gen, (1, 1, 2, 256)), randn_bf16(gen, (1, 1, 2, 256))
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), [0], 1 / 16)
        orc.append(0, 0, to_np(k[0]), to_np(v[0]))
        torch.cuda.synchronize()
        ref = orc.attend(0, 0, to_np(q[0]), 1 / 16)
        assert float(np.abs(to_np(out[0]) - ref).max()) <= ATOL
    assert rt.seq_length(0) == 96 and rt.health() == 0


def test_rollover_refusals():
    from kvrt import KVRTError, KVRuntime, LayerSpec

    ring = KVRuntime([LayerSpec(kv_heads=1, head_dim=128, layout="ring", window=8, ring_rows=9)], 1, 64,
                     max_q=2, device="cuda")
    x = torch.zeros((1, 1, 30, 128), dtype=torch.bfloat16, device="cuda")
    ring.import_(0, 0, x, x)
    with pytest.raises(KVRTError) as e:
        ring.rollover(0, 4, 8)
    assert e.value.code == -1
    rt = KVRuntime([LayerSpec(kv_heads=1, head_dim=128), LayerSpec(kv_heads=1, head_dim=128)], 1, 256,
                   max_q=2, device="cuda")
    rt.import_(0, 0, x, x)
    with pytest.raises(KVRTError) as e:  # layers at different lengths
        rt.rollover(0, 4, 8)
    assert e.value.code == -2
    rt.import_(0, 1, x, x)
    for prefix, kept, code in ((0, 8, -1), (4, 0, -1), (4, 130, -1), (22, 8, -2), (4, 26, -2)):
        with pytest.raises(KVRTError) as e:
            rt.rollover(0, prefix, kept)
        assert e.value.code == code, (prefix, kept)
    with pytest.raises(KVRTError):
        rt.set_layer_rope(0, [1.0] * 63)  # head_dim / 2 entries required
    assert rt.seq_length(0) == 30 and rt.health() == 0


@pytest.mark.parametrize("layout,dtype", [("contig", "bf16"), ("ring", "bf16"), ("paged", "bf16"), ("paged", "int8")])
def test_copy_prefix_every_layout(layout, dtype):
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(5)
    kw = dict(block_size=16, pool_pages=300) if layout == "paged" else {}
    win = 64 if layout == "ring" else 0
    spec = LayerSpec(kv_heads=2, head_dim=128, layout=layout, dtype=dtype, window=win,
                     ring_rows=(64 + 2 - 1) if layout == "ring" else 0)
    rt = KVRuntime([spec, LayerSpec(kv_heads=1, head_dim=64)], 3, 1024, max_q=2, device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(2, 128, win, int8=dtype == "int8"), O.OracleLayer(1, 64)], 3)
    for slot, n in ((0, 500), (2, 40)):
        for layer, (h, d) in enumerate(((2, 128), (1, 64))):
            k, v = randn_bf16(gen, (1, h, n, d)), randn_bf16(gen, (1, h, n, d))
            rt.import_(slot, layer, k.cuda(), v.cuda())
            orc.append(slot, layer, to_np(k[0]), to_np(v[0]))
    # clone into slot 1 (empty) and slot 2 (over its own rows); a ring keeps
    # positions [435, 500), so its clone must still see a whole window
    n = 499 if layout == "ring" else 450
    for dst in (1, 2):
        rt.copy_prefix(0, dst, n)
        for layer in range(2):
            orc.copy_prefix(0, dst, layer, n)
    assert rt.health() == 0
    for dst in (1, 2):
        start = n - 63 if layout == "ring" else 0
        _check_rows(rt, orc, dst, 0, start)
        _check_rows(rt, orc, dst, 1)
    # the clone then decodes like the source would
    q = randn_bf16(gen, (1, 4, 1, 128), 0.5)
    a = rt.attend(0, q.cuda(), [1], 0.1)
    torch.cuda.synchronize()
    ref = orc.attend(1, 0, to_np(q[0]), 0.1)
    assert float(np.abs(to_np(a[0]) - ref).max()) <= ATOL


def test_copy_prefix_refusals_leave_state_unchanged():
    from kvrt import KVRTError, KVRuntime, LayerSpec

    rt = KVRuntime([LayerSpec(kv_heads=1, head_dim=128, layout="ring", window=32, ring_rows=33)], 2, 512,
                   max_q=2, device="cuda")
    x = torch.ones((1, 1, 300, 128), dtype=torch.bfloat16, device="cuda")
    rt.import_(0, 0, x, x)
    with pytest.raises(KVRTError) as e:  # the window of position 100 left the ring long ago
        rt.copy_prefix(0, 1, 100)
    assert e.value.code == -2 and rt.seq_length(1) == 0
    paged = KVRuntime([LayerSpec(kv_heads=1, head_dim=128, layout="paged")], 2, 1024, max_q=2, device="cuda",
                      block_size=16, pool_pages=30)
    paged.import_(0, 0, x, x)          # 19 pages
    before = paged.counters()["pages_in_use"]
    with pytest.raises(KVRTError) as e:  # 19 more pages do not fit in the 11 left
        paged.copy_prefix(0, 1, 300)
    assert e.value.code == -5
    assert paged.counters()["pages_in_use"] == before and paged.seq_length(1) == 0
    paged.copy_prefix(0, 1, 160)       # 10 pages fit
    assert paged.seq_length(1) == 160 and paged.health() == 0


def _ring_step(rt, orc, gen, slot=0):
    """One fused Q1 step on the ring layer, checked against the oracle."""
    q = randn_bf16(gen, (1, 2, 1, 128), 0.5)
    k, v = randn_bf16(gen, (1, 1, 1, 128)), randn_bf16(gen, (1, 1, 1, 128))
    out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), [slot], 0.1)
    orc.append(slot, 0, to_np(k[0]), to_np(v[0]))
    torch.cuda.synchronize()
    return float(np.abs(to_np(out[0]) - orc.attend(slot, 0, to_np(q[0]), 0.1)).max())


def test_ring_rollbacks_stop_at_rows_later_positions_overwrote():
    """A ring of 70 rows under a 64-key window. After 500 positions it holds
    [430, 500); a rollback to 495 leaves those rows in place, so a second
    rollback (or one after a shorter re-append) may only go as far as the
    window of its next query still starts at 430 or later: position 427's row
    now holds position 497. Rollbacks to 0 (a release) always succeed."""
    from kvrt import KVRTError, KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(31)
    rt = KVRuntime([LayerSpec(kv_heads=1, head_dim=128, layout="ring", window=64, ring_rows=70)], 2, 1024,
                   max_q=2, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, 128, 64)], 2)
    _fill(rt, orc, 0, 0, 500, gen, 1, 128)
    rt.truncate(0, 495)
    orc.truncate(0, 0, 495)
    for bad in (490, 492):  # windows from 427 / 429: overwritten by 497 / 499
        with pytest.raises(KVRTError) as e:
            rt.truncate(0, bad)
        assert e.value.code == -2 and rt.seq_length(0) == 495
    assert _ring_step(rt, orc, gen) <= ATOL
    assert _ring_step(rt, orc, gen) <= ATOL       # 497: the ring still remembers 500
    with pytest.raises(KVRTError):
        rt.truncate(0, 492)
    with pytest.raises(KVRTError):                # a clone's next query needs [429, 492]
        rt.copy_prefix(0, 1, 492)
    rt.truncate(0, 493)                           # window [430, 493): all resident
    orc.truncate(0, 0, 493)
    assert _ring_step(rt, orc, gen) <= ATOL
    # a copy into another context of the same topology carries the floor too
    other = KVRuntime([LayerSpec(kv_heads=1, head_dim=128, layout="ring", window=64, ring_rows=70)], 1, 1024,
                      max_q=2, device="cuda")
    with pytest.raises(KVRTError):
        other.copy_session(0, rt, 0, 492)
    other.copy_session(0, rt, 0, 494)
    with pytest.raises(KVRTError):
        other.truncate(0, 492)
    orc_other = O.OracleCache([O.OracleLayer(1, 128, 64)], 1)
    orc_other.append(0, 0, *orc.values(0, 0))
    orc_other.truncate(0, 0, 494)
    assert _ring_step(other, orc_other, gen) <= ATOL
    assert other.health() == 0
    rt.copy_prefix(0, 1, 494)                     # the clone inherits the ring's floor
    orc.copy_prefix(0, 1, 0, 494)
    with pytest.raises(KVRTError):
        rt.truncate(1, 492)
    assert _ring_step(rt, orc, gen, slot=1) <= ATOL
    _check_rows(rt, orc, 1, 0, start=495 - 63)
    # an empty clone and releases of long slots
    rt.copy_prefix(0, 1, 0)
    assert rt.seq_length(1) == 0
    orc.copy_prefix(0, 1, 0, 0)
    rt.truncate(0, 0)
    orc.truncate(0, 0, 0)
    for slot in (0, 1):
        for _ in range(3):
            assert _ring_step(rt, orc, gen, slot) <= ATOL
    assert rt.health() == 0
    paged = KVRuntime([LayerSpec(kv_heads=1, head_dim=128, layout="paged", window=32)], 1, 1024, max_q=2,
                      device="cuda", block_size=16, pool_pages=40)
    x = torch.ones((1, 1, 300, 128), dtype=torch.bfloat16, device="cuda")
    slot = paged.acquire_slot()
    paged.import_(slot, 0, x, x)
    paged.evict(slot, 240)
    with pytest.raises(KVRTError):               # below the released pages
        paged.truncate(slot, 200)
    paged.release_slot(slot)
    assert paged.seq_length(slot) == 0 and paged.counters()["pages_in_use"] == 0 and paged.health() == 0


def test_copy_session_between_contexts():
    from kvrt import KVRTError, KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(8)
    specs = [LayerSpec(kv_heads=1, head_dim=256, window=512), LayerSpec(kv_heads=1, head_dim=512),
             LayerSpec(kv_heads=1, head_dim=256, shared_src=0)]
    a = KVRuntime(specs, 2, 1024, max_q=2, device="cuda")
    b = KVRuntime(specs, 3, 1024, max_q=2, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, 256, 512), O.OracleLayer(1, 512)], 4)
    for layer, d in ((0, 256), (1, 512)):
        _fill(a, orc, 1, layer, 700, gen, 1, d)
    b.copy_session(2, a, 1, 650)
    for layer in range(2):
        orc.copy_prefix(1, 3, layer, 650)
    assert b.health() == 0 and b.seq_length(2, 2) == 650
    for layer in range(2):
        kb, vb, _ = b.gather(layer, [2], mask_dtype=None)
        torch.cuda.synchronize()
        ok, ov = orc.values(3, layer)
        assert np.array_equal(bits(kb[0]), O.f32_to_bf16_bits(ok))
        assert np.array_equal(bits(vb[0]), O.f32_to_bf16_bits(ov))
    other = KVRuntime([LayerSpec(kv_heads=1, head_dim=256, window=256), specs[1], specs[2]], 2, 1024,
                      max_q=2, device="cuda")
    with pytest.raises(KVRTError) as e:
        other.copy_session(0, a, 1, 10)
    assert e.value.code == -1


def _gemma_specs(max_q):
    from kvrt import LayerSpec

    specs = []
    for i in range(35):
        full = i % 5 == 4
        src = -1 if i < 15 else (14 if full else 13)
        specs.append(LayerSpec(kv_heads=1, head_dim=512 if full else 256, window=0 if full else 512,
                               shared_src=src))
    return specs


def test_gemma_listener_topology_steps_rollover_and_clone():
    """35 layers, Hq 8 / Hkv 1: owned layers append + attend, shared layers
    attend over 13 / 14; rollover with the sliding (D 256, base 1e4) and
    proportional full (D 512, base 1e6, 64 pairs) RoPE tables; clone."""
    from kvrt import KVRuntime

    gen = torch.Generator().manual_seed(35)
    specs = _gemma_specs(2)
    rt = KVRuntime(specs, 3, 2048, max_q=2, device="cuda")
    owner = [i if s.shared_src < 0 else s.shared_src for i, s in enumerate(specs)]
    orc = O.OracleCache([O.OracleLayer(1, s.head_dim, s.window) for s in specs], 3)
    for slot, n in ((0, 700), (1, 300)):
        for layer in range(15):
            _fill(rt, orc, slot, layer, n, gen, 1, specs[layer].head_dim)
    inv_s, inv_f = O.gemma_inv_freq(256, 1e4), O.gemma_inv_freq(512, 1e6, 64)
    for layer in range(15):
        rt.set_layer_rope(layer, (inv_f if layer % 5 == 4 else inv_s).tolist())

    def step(slots):
        # Gemma-4 attends with scaling 1.0 over RMS-normed q / k; q of norm
        # ~0.5 keeps the softmax soft, so outputs stay below 4 where bf16
        # rounding (half an ulp: 0.0078) fits the 1e-2 bound
        n = len(slots)
        worst = 0.0
        for layer, s in enumerate(specs):
            q = randn_bf16(gen, (n, 8, 2, s.head_dim), 0.5 / s.head_dim ** 0.5)
            if owner[layer] == layer:
                k = randn_bf16(gen, (n, 1, 2, s.head_dim))
                v = randn_bf16(gen, (n, 1, 2, s.head_dim))
                out = rt.append_attend(layer, q.cuda(), k.cuda(), v.cuda(), slots, 1.0)
                for i, slot in enumerate(slots):
                    orc.append(slot, layer, to_np(k[i]), to_np(v[i]))
            else:
                out = rt.attend(layer, q.cuda(), slots, 1.0)
            torch.cuda.synchronize()
            for i, slot in enumerate(slots):
                ref = orc.attend(slot, owner[layer], to_np(q[i]), 1.0)
                worst = max(worst, float(np.abs(to_np(out[i]) - ref).max()))
        return worst

    for _ in range(2):
        assert step([0, 1]) <= ATOL
    rt.rollover(0, 96, 128)
    for layer in range(15):
        orc.rollover(0, layer, 96, 128, inv_f if layer % 5 == 4 else inv_s)
    assert rt.seq_length(0, 34) == 224
    for layer in (0, 4, 13, 14):
        _check_rows(rt, orc, 0, layer)
    assert step([1, 0]) <= ATOL
    rt.copy_prefix(0, 2, rt.seq_length(0))
    for layer in range(15):
        orc.copy_prefix(0, 2, layer, orc.length(0, layer))
    assert step([0, 2]) <= ATOL
    assert rt.health() == 0
