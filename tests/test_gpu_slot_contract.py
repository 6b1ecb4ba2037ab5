"""The slot contract of rollback and import, through the C ABI on the GPU.

A rollback carries the caller's view of the slot: its generation and its
current position (gemma4_listener_batch_rewind_session_async refuses a stale
identity, a sequence position that is not the slot's and current_position !=
valid_kv_len with -2: gemma4_listener_microbatch_impl.inc:3601-3610). An import
starts a session and never lands on a live one
(gemma4_listener_batch_import_cache_async refuses a primed slot,
impl.inc:2595, and takes the row's identity, :2629-2637). Host lengths go
stale when a captured graph replays; the runtime refuses to roll back against
them, and the device refuses an edit validated against lengths it no longer
holds. Every refusal leaves counters, lengths and stored rows as they were."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import bits, randn_bf16

pytestmark = pytest.mark.gpu


def _rt(n_slots=3, capacity=640):
    from kvrt import KVRuntime, LayerSpec

    return KVRuntime([LayerSpec(kv_heads=8, head_dim=128), LayerSpec(kv_heads=1, head_dim=256)], n_slots, capacity,
                     max_q=2, device="cuda")


def _layers(gen, n):
    return [(randn_bf16(gen, (1, h, n, d)).cuda(), randn_bf16(gen, (1, h, n, d)).cuda())
            for h, d in ((8, 128), (1, 256))]


def _stored(rt, slot, lmax):
    out = []
    for layer in range(2):
        k, v, _ = rt.gather(layer, [slot], lmax=lmax)
        torch.cuda.synchronize()
        out.append((bits(k).tobytes(), bits(v).tobytes()))
    return out


def _refused(call, code=-2):
    from kvrt import KVRTError

    with pytest.raises(KVRTError) as e:
        call()
    assert e.value.code == code


def test_truncate_refuses_a_position_that_is_not_the_slots():
    gen = torch.Generator().manual_seed(21)
    rt = _rt()
    g = rt.import_session(0, _layers(gen, 300))
    rt.synchronize()
    stored = _stored(rt, 0, 300)
    before = rt.counters()
    for exp in (299, 301, 0):
        _refused(lambda: rt.truncate(0, 100, generation=g, expected_len=exp))
        _refused(lambda: rt.truncate(0, 100, layer=1, expected_len=exp))
    _refused(lambda: rt.truncate(0, 100, generation=g, expected_len=-2), code=-1)
    assert rt.counters() == before and [rt.seq_length(0, l) for l in range(2)] == [300, 300]
    assert _stored(rt, 0, 300) == stored
    rt.truncate(0, 100, generation=g, expected_len=300)
    rt.truncate(0, 60, layer=1, expected_len=100)
    assert [rt.seq_length(0, l) for l in range(2)] == [100, 60]
    _refused(lambda: rt.truncate(0, 50, expected_len=100))  # layer 1 is at 60
    rt.truncate(0, 50, layer=0, expected_len=100)
    rt.synchronize()
    rt.sync_lengths()  # the device holds what the host does
    assert [rt.seq_length(0, l) for l in range(2)] == [50, 60]
    assert rt.health() == 0


def test_import_refuses_a_live_slot_and_renews_the_generation():
    gen = torch.Generator().manual_seed(22)
    rt = _rt()
    g0 = rt.reset_slot(0)
    layers = _layers(gen, 120)
    rt.import_(0, 0, *layers[0])
    g1 = rt.slot_generation(0)
    assert g1 not in (0, g0)
    rt.synchronize()
    stored = _stored(rt, 0, 120)
    before = rt.counters()
    other = _layers(gen, 40)
    _refused(lambda: rt.import_(0, 0, *other[0]))  # layer 0 holds rows
    assert rt.counters() == before and rt.seq_length(0, 0) == 120 and rt.slot_generation(0) == g1
    assert _stored(rt, 0, 120)[0] == stored[0]
    _refused(lambda: rt.truncate(0, 10, generation=g0))  # the import made g0 stale
    rt.import_(0, 1, *layers[1])  # the empty layer of the same slot
    g2 = rt.slot_generation(0)
    assert g2 not in (g0, g1)
    # a masked session: every layer is live, and the mask keeps it so
    rt.set_prefix_attention(0, torch.ones(34, dtype=torch.int64, device="cuda"))
    for layer in range(2):
        _refused(lambda: rt.import_(0, layer, *other[layer]))
    _refused(lambda: rt.truncate(0, 0, generation=g2))  # below the mask: the rewind floor
    # release (mask cleared, rows dropped) takes a new session; holders of g2 are then stale
    rt.set_prefix_attention(0, None)
    rt.truncate(0, 0, generation=g2, expected_len=120)
    rt.import_(0, 0, *other[0])
    rt.import_(0, 1, *other[1])
    g3 = rt.slot_generation(0)
    assert g3 not in (g0, g1, g2)
    _refused(lambda: rt.truncate(0, 10, generation=g2))
    rt.truncate(0, 10, generation=g3, expected_len=40)
    k, _, _ = rt.gather(0, [0], lmax=10)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(k[0]), bits(other[0][0][0, :, :10]))
    assert rt.health() == 0


def test_rollback_against_graph_replayed_lengths_is_refused():
    """Capture one fused append + attend over 2 slots, then: before a length
    read-back, import and truncate are refused; after it, 3 replays advance
    the device lengths behind the host's back, and a truncate naming the true
    position is refused on the host; one that names no position is dropped
    by the device (health -6), which keeps its lengths and rows."""
    gen = torch.Generator().manual_seed(23)
    rt = _rt()
    for s in (0, 1):
        rt.import_session(s, _layers(gen, 500))
    q = randn_bf16(gen, (2, 16, 1, 128)).cuda()
    kn, vn = randn_bf16(gen, (2, 8, 1, 128)).cuda(), randn_bf16(gen, (2, 8, 1, 128)).cuda()
    out = torch.empty((2, 16, 1, 128), dtype=torch.bfloat16, device="cuda")
    rt.append_attend(0, q, kn, vn, [0, 1], 0.088, out=out)  # eager first: workspace sized
    rt.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            rt.append_attend(0, q, kn, vn, [0, 1], 0.088, out=out)
        # the capture advanced the host lengths only: nothing rolls back or
        # imports against them until they are read back
        before = rt.counters()
        _refused(lambda: rt.truncate(0, 400))
        _refused(lambda: rt.truncate(0, 400, expected_len=502))
        _refused(lambda: rt.import_(2, 0, *_layers(gen, 8)[0]))
        assert rt.counters() == before
        rt.sync_lengths()
        assert rt.seq_length(0, 0) == 501
        for _ in range(3):
            g.replay()
        side.synchronize()
        stored = _stored(rt, 0, 504)
        before = rt.counters()
        _refused(lambda: rt.truncate(0, 400, layer=0, expected_len=504))  # the host still says 501
        assert rt.counters() == before and rt.seq_length(0, 0) == 501
        rt.truncate(0, 400)  # accepted against the stale 501: the device must drop it
        assert rt.health() == -6
        rt.sync_lengths()
        assert rt.seq_length(0, 0) == 504 and rt.seq_length(1, 0) == 504 and rt.seq_length(0, 1) == 500
        assert _stored(rt, 0, 504) == stored
        rt.truncate(0, 400, layer=0, expected_len=504)
        rt.sync_lengths()
        assert rt.seq_length(0, 0) == 400


def test_a_refused_call_does_not_hold_the_stream():
    """A call refused by its argument checks enqueues nothing, so the context
    may still move to another stream afterwards."""
    gen = torch.Generator().manual_seed(24)
    rt = _rt()
    rt.import_session(0, _layers(gen, 64))
    rt.synchronize()
    bad = randn_bf16(gen, (1, 3, 1, 128)).cuda()  # 3 kv heads: the layer has 8
    _refused(lambda: rt.append(0, bad, bad, [0]), code=-1)
    _refused(lambda: rt.truncate(0, 70), code=-2)
    side = torch.cuda.Stream()
    k = randn_bf16(gen, (1, 8, 1, 128)).cuda()
    with torch.cuda.stream(side):
        rt.append(0, k, k, [0])  # no KVRT_ESTATE: nothing was in flight
        assert rt.health() == 0
    assert rt.seq_length(0, 0) == 65
