"""Confinement and identity of a kvrt context on the GPU: one bound stream
(a second stream is refused while the context's work may still run, as the
reference's batch API refuses it with -6: gemma4_listener_microbatch_impl.inc:
445-473), one owner thread (native_listener_microbatch.py:1128-1131), and slot
generations that make lifecycle calls from a stale owner fail with nothing
changed (rewind_session_async's identity check, impl.inc:3588-3618). Also the
contracts fixed around them: positional updates return the whole slot storage
(_SlotKVCache.update, future_prefix.py:544-565) and a full-attention PAGED
decode refuses to read evicted pages."""
from __future__ import annotations

import ctypes
import threading

import numpy as np
import pytest
import torch

from tests.helpers import bits, randn_bf16

pytestmark = pytest.mark.gpu


def _rt(**kw):
    from kvrt import KVRuntime, LayerSpec

    return KVRuntime([LayerSpec(kv_heads=2, head_dim=128), LayerSpec(kv_heads=1, head_dim=256)], 3, 512,
                     max_q=2, device="cuda", **kw)


def _fill(rt, slot, n, gen):
    for layer, (h, d) in enumerate(((2, 128), (1, 256))):
        rt.import_(slot, layer, randn_bf16(gen, (1, h, n, d)).cuda(), randn_bf16(gen, (1, h, n, d)).cuda())


def test_second_stream_is_refused_while_work_is_in_flight():
    from kvrt import KVRTError
    from kvrt import _lib as L

    gen = torch.Generator().manual_seed(1)
    rt = _rt()
    _fill(rt, 0, 100, gen)  # enqueued on the default stream
    before = rt.counters()
    side = torch.cuda.Stream()
    k = randn_bf16(gen, (1, 2, 1, 128)).cuda()
    with torch.cuda.stream(side):
        with pytest.raises(KVRTError) as e:
            rt.append(0, k, k, [0])
    assert e.value.code == L.KVRT_ESTATE
    assert rt.counters() == before and rt.seq_length(0, 0) == 100
    # the C entry point itself refuses, and binding the bound stream again is a no-op
    assert rt.lib.kvrt_bind_stream(rt._ctx, ctypes.c_void_p(side.cuda_stream)) == L.KVRT_ESTATE
    assert rt.lib.kvrt_bind_stream(rt._ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    # after a synchronisation the context may move
    rt.synchronize()
    with torch.cuda.stream(side):
        rt.append(0, k, k, [0])
        assert rt.health() == 0
    assert rt.seq_length(0, 0) == 101
    rt.append(0, k, k, [0])  # back on the default stream: legal, the side stream was synchronised
    assert rt.seq_length(0, 0) == 102 and rt.health() == 0


def test_calls_from_another_thread_are_refused():
    gen = torch.Generator().manual_seed(2)
    rt = _rt()
    _fill(rt, 0, 10, gen)
    rt.synchronize()
    before = rt.counters()
    errors = []

    def other():
        for call in (lambda: rt.seq_length(0), lambda: rt.truncate(0, 5), lambda: rt.health()):
            try:
                call()
                errors.append(None)
            except RuntimeError as e:
                errors.append(str(e))

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert len(errors) == 3 and all(e and "thread" in e for e in errors)
    assert rt.counters() == before and rt.seq_length(0) == 10


def test_stale_generations_are_refused_and_change_nothing():
    from kvrt import KVRTError

    gen = torch.Generator().manual_seed(3)
    rt = _rt()
    g0 = rt.reset_slot(0)
    _fill(rt, 0, 300, gen)
    g1 = rt.slot_generation(0)  # the imports renewed it
    rt.synchronize()
    rt.reset_slot(0)  # a new session in slot 0: holders of g1 are stale
    _fill(rt, 0, 300, gen)
    g2 = rt.slot_generation(0)
    assert len({g0, g1, g2}) == 3 and 0 not in (g0, g1, g2)
    k0, v0, _ = rt.gather(0, [0])
    torch.cuda.synchronize()
    before = rt.counters()
    for call in (lambda: rt.truncate(0, 100, generation=g1), lambda: rt.copy_prefix(0, 1, 300, generation=g1),
                 lambda: rt.rollover(0, 10, 64, generation=g1)):
        with pytest.raises(KVRTError) as e:
            call()
        assert e.value.code == -2
    assert rt.counters() == before and rt.seq_length(0, 0) == rt.seq_length(0, 1) == 300
    assert rt.seq_length(1, 0) == 0
    g3 = rt.copy_prefix(0, 1, 300, generation=g2)
    assert g3 not in (g1, g2) and rt.slot_generation(0) == g2
    rt.truncate(0, 100, generation=g2)
    with pytest.raises(KVRTError):
        rt.truncate(1, 100, generation=g2)  # slot 1's generation is g3
    rt.truncate(1, 100, generation=g3)
    k1, v1, _ = rt.gather(0, [1], lmax=300)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(k1[0, :, :100]), bits(k0[0, :, :100]))
    assert rt.health() == 0


def test_positional_update_returns_the_whole_slot_storage():
    from kvrt import KVRTCache, KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(4)
    rt = KVRuntime([LayerSpec(kv_heads=8, head_dim=128)], 2, 64, max_q=2, device="cuda")
    cache = KVRTCache(rt)
    k, v = randn_bf16(gen, (1, 8, 2, 128)).cuda(), randn_bf16(gen, (1, 8, 2, 128)).cuda()
    keys, values = cache.update(k, v, 0, {"cache_position": torch.tensor([3, 9])})
    assert keys.shape == values.shape == (1, 8, 64, 128)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(keys[0, :, 9]), bits(k[0, :, 1]))
    assert float(keys[0, :, 4].abs().max()) == 0.0  # never written: zeros, as _SlotKVCache's
    assert cache.get_seq_length(0) == 10 and cache.get_mask_sizes(1, 0) == (64, 0)


def test_full_attention_paged_decode_refuses_evicted_pages():
    from kvrt import KVRTError, KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(5)
    rt = KVRuntime([LayerSpec(kv_heads=1, head_dim=128, layout="paged")], 1, 256, max_q=1, block_size=16,
                   pool_pages=16, device="cuda")
    rt.import_(0, 0, randn_bf16(gen, (1, 1, 100, 128)).cuda(), randn_bf16(gen, (1, 1, 100, 128)).cuda())
    q = randn_bf16(gen, (1, 2, 1, 128)).cuda()
    rt.attend(0, q, [0], 0.1)
    rt.evict(0, 40)  # pages 0 and 1 released; a window-0 query still sees key 0
    before = rt.counters()
    with pytest.raises(KVRTError) as e:
        rt.attend(0, q, [0], 0.1)
    assert e.value.code == -2 and rt.counters() == before
    k = randn_bf16(gen, (1, 1, 1, 128)).cuda()
    with pytest.raises(KVRTError):
        rt.append_attend(0, q, k, k, [0], 0.1)
    assert rt.seq_length(0) == 100 and rt.health() == 0


def test_slot_growth_keeps_every_slot_and_adds_empty_ones():
    """ensure_capacity / kvrt_grow_slots (gemma4_listener_batch_ensure_capacity,
    native_listener_microbatch.py:1217-1268): rows, lengths, masks, pages and
    generations of the existing slots survive; the new slots are empty with
    new generations and take sessions like the others."""
    from kvrt import KVRuntime, LayerSpec
    from oracle import kv_oracle as O
    from tests.helpers import to_np

    gen = torch.Generator().manual_seed(6)
    specs = [LayerSpec(kv_heads=2, head_dim=128), LayerSpec(kv_heads=1, head_dim=256, layout="ring", window=64,
                                                             ring_rows=65),
             LayerSpec(kv_heads=2, head_dim=128, layout="paged"), LayerSpec(kv_heads=2, head_dim=128, shared_src=0)]
    rt = KVRuntime(specs, 2, 400, max_q=2, block_size=16, pool_pages=100, device="cuda")
    orc = O.OracleCache([O.OracleLayer(2, 128), O.OracleLayer(1, 256, 64), O.OracleLayer(2, 128)], 6)
    mask = O.canonical_prefix_mask()
    for slot, n in ((0, 300), (1, 90)):
        for layer, s in enumerate(specs[:3]):
            k, v = randn_bf16(gen, (1, s.kv_heads, n, s.head_dim)), randn_bf16(gen, (1, s.kv_heads, n, s.head_dim))
            rt.import_(slot, layer, k.cuda(), v.cuda())
            orc.append(slot, layer, to_np(k[0]), to_np(v[0]))
    rt.set_prefix_attention(1, torch.from_numpy(mask).cuda())
    orc.set_prefix_attention(1, mask)
    before = {s: rt.slot_info(s) for s in (0, 1)}
    rows = {(s, l): rt.gather(l, [s], mask_dtype=None)[:2] for s in (0, 1) for l in range(3)}
    torch.cuda.synchronize()
    assert rt.ensure_capacity(5) == 5 and rt.ensure_capacity(3) == 5
    assert {s: rt.slot_info(s) for s in (0, 1)} == before
    for (s, l), (k, v) in rows.items():
        k2, v2, _ = rt.gather(l, [s], mask_dtype=None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(k2), bits(k))
        np.testing.assert_array_equal(bits(v2), bits(v))
    gens = {rt.slot_generation(s) for s in range(5)}
    assert len(gens) == 5
    for s in (2, 3, 4):
        assert rt.slot_info(s)["max_len"] == 0 and rt.slot_info(s)["prefix_len"] == 0
        assert float(rt.storage(0)[0][s].abs().max()) == 0.0
    for layer, s in enumerate(specs[:3]):
        k, v = randn_bf16(gen, (1, s.kv_heads, 150, s.head_dim)), randn_bf16(gen, (1, s.kv_heads, 150, s.head_dim))
        rt.import_(4, layer, k.cuda(), v.cuda())
        orc.append(4, layer, to_np(k[0]), to_np(v[0]))
    worst = 0.0
    for layer, s in enumerate(specs):
        hq = 4 if s.head_dim == 128 else 8
        q = randn_bf16(gen, (3, hq, 2, s.head_dim), 1.0 / s.head_dim ** 0.5)
        out = rt.attend(layer, q.cuda(), [0, 1, 4], 1.0)
        torch.cuda.synchronize()
        for i, slot in enumerate((0, 1, 4)):
            ref = orc.attend(slot, min(layer, 2) if layer < 3 else 0, to_np(q[i]), 1.0)
            worst = max(worst, float(np.abs(to_np(out[i]) - ref).max()))
    assert worst <= 1e-2
    assert rt.health() == 0


def test_library_owned_context_grows_through_the_c_abi():
    from kvrt import _lib as L
    from kvrt.runtime import current_stream_handle, tensor_desc

    lib = L.load()
    gen = torch.Generator().manual_seed(8)
    cfg = L.KvrtConfig()
    cfg.struct_size = ctypes.sizeof(L.KvrtConfig)
    cfg.n_layers, cfg.n_slots, cfg.capacity, cfg.block_size, cfg.pool_pages, cfg.max_q = 1, 2, 256, 16, 0, 1
    spec = L.KvrtLayerSpec(L.LAYOUT_CONTIG, L.DT_BF16, 2, 128, 0, 0, -1, 0)
    ctx = ctypes.c_void_p()
    assert lib.kvrt_create(ctypes.byref(cfg), ctypes.byref(spec), ctypes.byref(ctx)) == 0
    try:
        assert lib.kvrt_bind_stream(ctx, ctypes.c_void_p(current_stream_handle(torch.device("cuda")))) == 0
        k = randn_bf16(gen, (1, 2, 200, 128)).cuda()
        kd = tensor_desc(k)
        assert lib.kvrt_import_async(ctx, 1, 0, ctypes.byref(kd), ctypes.byref(kd), 0) == 0
        st = (L.KvrtStorage * 1)()
        assert lib.kvrt_grow_slots(ctx, 4, st) == L.KVRT_EINVAL  # the context owns its storage
        assert lib.kvrt_grow_slots(ctx, 4, None) == 0
        out = torch.empty((1, 2, 200, 128), dtype=torch.bfloat16, device="cuda")
        od = tensor_desc(out)
        slots = (ctypes.c_int32 * 1)(1)
        assert lib.kvrt_gather_async(ctx, 0, 1, slots, None, ctypes.byref(od), ctypes.byref(od), None) == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(out), bits(k))
        length = ctypes.c_int32()
        assert lib.kvrt_session_state(ctx, 3, 0, ctypes.byref(length)) == 0 and length.value == 0
        assert lib.kvrt_health(ctx) == 0
    finally:
        lib.kvrt_destroy(ctx)
