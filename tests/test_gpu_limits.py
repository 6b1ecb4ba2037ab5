"""Edge cases of the decode path at the boundaries of the ABI: the most slots a
batched call takes (KVRT_MAX_ITEMS), a fused append into an empty slot, an
append that fills the capacity exactly and the one that would overflow it,
and empty imports. Refused calls must leave lengths and counters unchanged.
Attention against the fp64 oracle at max-abs 1e-2; cache contents bit-exact."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, np_bf16_bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2


def test_max_items_in_one_call_and_one_more_refused():
    """64 ragged slots (1 to 700 positions) in one fused append + attend
    launch, then a 65-slot call that must be refused before any launch."""
    from kvrt import KVRTError, KVRuntime, LayerSpec

    n = 64
    gen = torch.Generator().manual_seed(64)
    spec = LayerSpec(kv_heads=2, head_dim=64)
    rt = KVRuntime([spec], n + 1, 720, max_q=1, device="cuda")
    orc = O.OracleCache([O.OracleLayer(2, 64)], n + 1)
    lens = [1 + (i * 37) % 700 for i in range(n)]
    for s, ln in enumerate(lens):
        k, v = randn_bf16(gen, (1, 2, ln, 64)), randn_bf16(gen, (1, 2, ln, 64))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    slots = list(range(n))
    q = randn_bf16(gen, (n, 4, 1, 64), 0.5)
    k, v = randn_bf16(gen, (n, 2, 1, 64)), randn_bf16(gen, (n, 2, 1, 64))
    out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), slots, 0.125)
    torch.cuda.synchronize()
    worst = 0.0
    for i in slots:
        orc.append(i, 0, to_np(k[i]), to_np(v[i]))
        worst = max(worst, float(np.abs(to_np(out[i]) - orc.attend(i, 0, to_np(q[i]), 0.125)).max()))
    assert worst <= ATOL, worst
    kg, vg, _ = rt.gather(0, slots)
    ko, vo, _ = orc.gather(0, slots, kg.shape[2])
    np.testing.assert_array_equal(bits(kg), np_bf16_bits(ko))
    np.testing.assert_array_equal(bits(vg), np_bf16_bits(vo))

    before = rt.counters()
    lens_before = [rt.seq_length(s, 0) for s in range(n + 1)]
    q65 = randn_bf16(gen, (n + 1, 4, 1, 64)).cuda()
    k65 = randn_bf16(gen, (n + 1, 2, 1, 64)).cuda()
    with pytest.raises(KVRTError):
        rt.append_attend(0, q65, k65, k65, list(range(n + 1)), 0.125)
    assert rt.counters() == before
    assert [rt.seq_length(s, 0) for s in range(n + 1)] == lens_before
    assert rt.health() == 0


@pytest.mark.parametrize("d,hq,layout", [(128, 16, "contig"), (256, 8, "ring"), (512, 8, "contig")])
def test_fused_append_into_an_empty_slot_returns_v(d, hq, layout):
    """One visible key: the softmax weight is exactly 1, so every q head's
    output is the appended v row bit for bit (both decode kernels' shapes)."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(d + hq)
    hkv = 8 if hq == 16 else 1
    ring = dict(window=64, ring_rows=64) if layout == "ring" else {}
    rt = KVRuntime([LayerSpec(kv_heads=hkv, head_dim=d, layout=layout, **ring)], 3, 128, max_q=1, device="cuda")
    q = randn_bf16(gen, (2, hq, 1, d))
    k, v = randn_bf16(gen, (2, hkv, 1, d)), randn_bf16(gen, (2, hkv, 1, d))
    out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), [2, 0], 1.0 / math.sqrt(d))
    torch.cuda.synchronize()
    g = hq // hkv
    want = v.repeat_interleave(g, dim=1)  # q head h reads kv head h // g
    np.testing.assert_array_equal(bits(out.cpu()), bits(want))
    assert rt.seq_length(2, 0) == 1 and rt.seq_length(0, 0) == 1 and rt.seq_length(1, 0) == 0
    assert rt.health() == 0


def test_append_fills_capacity_then_refuses_without_changes():
    from kvrt import KVRTError, KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(9)
    cap = 100
    rt = KVRuntime([LayerSpec(kv_heads=1, head_dim=128)], 2, cap, max_q=2, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, 128)], 2)
    k, v = randn_bf16(gen, (1, 1, cap - 2, 128)), randn_bf16(gen, (1, 1, cap - 2, 128))
    rt.import_(0, 0, k.cuda(), v.cuda())
    orc.append(0, 0, to_np(k[0]), to_np(v[0]))
    q = randn_bf16(gen, (1, 2, 2, 128), 0.5)
    k, v = randn_bf16(gen, (1, 1, 2, 128)), randn_bf16(gen, (1, 1, 2, 128))
    out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), [0], 0.09)  # ends exactly at capacity
    torch.cuda.synchronize()
    orc.append(0, 0, to_np(k[0]), to_np(v[0]))
    assert float(np.abs(to_np(out[0]) - orc.attend(0, 0, to_np(q[0]), 0.09)).max()) <= ATOL
    assert rt.seq_length(0, 0) == cap
    before = rt.counters()
    one = randn_bf16(gen, (1, 1, 1, 128)).cuda()
    with pytest.raises(KVRTError):
        rt.append(0, one, one, [0])
    with pytest.raises(KVRTError):
        rt.append_attend(0, randn_bf16(gen, (1, 2, 1, 128)).cuda(), one, one, [0], 0.09)
    assert rt.counters() == before and rt.seq_length(0, 0) == cap
    kg, _, _ = rt.gather(0, [0])
    ko, _, _ = orc.gather(0, [0], cap)
    np.testing.assert_array_equal(bits(kg), np_bf16_bits(ko))
    assert rt.health() == 0


def test_empty_import_leaves_an_empty_layer():
    """An import fills an empty layer with its S rows, so S = 0 (an empty
    torch tensor, whose data pointer is null) leaves it empty; an import over
    a layer that holds rows is refused (code -2, nothing changes) until the
    slot is emptied. The next fused step then sees only its own key."""
    from kvrt import KVRTError, KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(1)
    rt = KVRuntime([LayerSpec(kv_heads=2, head_dim=64)], 2, 32, max_q=1, device="cuda")
    k = randn_bf16(gen, (1, 2, 5, 64)).cuda()
    rt.import_(1, 0, k, k)
    e = torch.empty((1, 2, 0, 64), dtype=torch.bfloat16, device="cuda")
    before = rt.counters()
    with pytest.raises(KVRTError) as err:
        rt.import_(1, 0, e, e)
    assert err.value.code == -2 and rt.counters() == before and rt.seq_length(1, 0) == 5
    rt.truncate(1, 0)
    rt.import_(1, 0, e, e)
    rt.import_(0, 0, e, e)
    torch.cuda.synchronize()
    assert rt.seq_length(1, 0) == 0 and rt.seq_length(0, 0) == 0
    q = randn_bf16(gen, (1, 2, 1, 64)).cuda()
    kn, vn = randn_bf16(gen, (1, 2, 1, 64)).cuda(), randn_bf16(gen, (1, 2, 1, 64)).cuda()
    out = rt.append_attend(0, q, kn, vn, [1], 0.125)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(out), bits(vn))
    assert rt.seq_length(1, 0) == 1
    assert rt.health() == 0
