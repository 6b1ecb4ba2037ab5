"""GPU parity of the core kvrt operations against the CPU oracle.

Cache operations (append, import, gather, truncate, copy) must be bit-exact;
attention within max-abs 1e-2 of the oracle's fp64-softmax result, computed
on the same seeded bf16 inputs.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, np_bf16_bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2  # attention tolerance (bf16 output vs fp64 softmax oracle)


def _rt(layers, n_slots, capacity, **kw):
    from kvrt import KVRuntime

    return KVRuntime(layers, n_slots, capacity, device="cuda", **kw)


def _oracle_layers(specs):
    return [O.OracleLayer(s.kv_heads, s.head_dim, s.window, s.dtype == "int8") for s in specs]


def _assert_gather_equal(rt, orc, layer, slots, ring_window=0):
    k, v, mask = rt.gather(layer, slots)
    lmax = k.shape[2]
    if ring_window:
        starts = [O.sliding_retained(orc.length(s, layer), ring_window)[0] for s in slots]
    else:
        starts = None
    ko, vo, mo = orc.gather(layer, slots, lmax, starts)
    if k.dtype == torch.bfloat16:
        np.testing.assert_array_equal(bits(k), np_bf16_bits(ko))
        np.testing.assert_array_equal(bits(v), np_bf16_bits(vo))
    else:  # int8 layers gather dequantised fp32
        np.testing.assert_array_equal(to_np(k).view(np.uint32), ko.view(np.uint32))
        np.testing.assert_array_equal(to_np(v).view(np.uint32), vo.view(np.uint32))
    np.testing.assert_array_equal(mask.cpu().numpy(), mo)


@pytest.mark.parametrize("layout", ["contig", "ring", "paged"])
@pytest.mark.parametrize("qn", [1, 2])
def test_append_then_gather_is_bitexact(layout, qn):
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(11 + qn)
    W = 24
    kw = {}
    if layout == "ring":
        spec = LayerSpec(kv_heads=2, head_dim=128, layout="ring", window=W, ring_rows=W + qn - 1 + 4)
    elif layout == "paged":
        spec = LayerSpec(kv_heads=2, head_dim=128, layout="paged")
        kw = dict(block_size=16, pool_pages=64)
    else:
        spec = LayerSpec(kv_heads=2, head_dim=128)
    rt = _rt([spec], n_slots=3, capacity=256, max_q=2, **kw)
    orc = O.OracleCache(_oracle_layers([spec]), 3)
    slots = [2, 0]
    for step in range(40):
        k = randn_bf16(gen, (len(slots), 2, qn, 128))
        v = randn_bf16(gen, (len(slots), 2, qn, 128))
        rt.append(0, k.cuda(), v.cuda(), slots)
        for i, s in enumerate(slots):
            orc.append(s, 0, to_np(k[i]), to_np(v[i]))
    torch.cuda.synchronize()
    assert rt.health() == 0
    assert rt.seq_length(2, 0) == 40 * qn
    _assert_gather_equal(rt, orc, 0, slots, ring_window=W if layout == "ring" else 0)


def test_import_and_truncate_move_no_bytes():
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(3)
    spec = LayerSpec(kv_heads=8, head_dim=128)
    rt = _rt([spec, spec], n_slots=2, capacity=512, max_q=2)
    orc = O.OracleCache(_oracle_layers([spec, spec]), 2)
    for layer in range(2):
        k = randn_bf16(gen, (1, 8, 300, 128))
        v = randn_bf16(gen, (1, 8, 300, 128))
        rt.import_(1, layer, k.cuda(), v.cuda())
        orc.append(1, layer, to_np(k[0]), to_np(v[0]))
    torch.cuda.synchronize()
    before = [bits(rt.storage(l)[0]).copy() for l in range(2)]
    rt.truncate(1, 257)
    for layer in range(2):
        orc.truncate(1, layer, 257)
    torch.cuda.synchronize()
    after = [bits(rt.storage(l)[0]) for l in range(2)]
    for b, a in zip(before, after):
        np.testing.assert_array_equal(a, b)  # rollback is a length edit only
    assert rt.seq_length(1, 0) == 257 and rt.seq_length(1, 1) == 257
    for layer in range(2):
        _assert_gather_equal(rt, orc, layer, [1])
    # re-append after rollback lands at the truncated length
    k = randn_bf16(gen, (1, 8, 2, 128))
    rt.append(0, k.cuda(), k.cuda(), [1])
    orc.append(1, 0, to_np(k[0]), to_np(k[0]))
    _assert_gather_equal(rt, orc, 0, [1])
    assert rt.counters()["truncations"] == 1


_DECODE_SHAPES = [
    (16, 8, 128, 1, 0, "contig"),   # talker shape
    (16, 8, 128, 2, 0, "contig"),
    (8, 1, 256, 1, 0, "contig"),    # thinker global shape
    (8, 1, 256, 2, 64, "ring"),     # thinker sliding shape, Q=2
    (8, 1, 256, 1, 64, "ring"),
    (8, 8, 128, 2, 0, "contig"),    # listener micro-batch shape (g=1)
    (8, 1, 512, 2, 0, "contig"),    # real Gemma full layers (D=512)
    (8, 1, 512, 1, 0, "contig"),
    (16, 8, 128, 1, 0, "paged"),
    (4, 2, 64, 3, 0, "contig"),     # odd Q: rows tile padding
    # LDS-DMA ring decodes (bf16 CONTIG / RING, <= 4 rows per kv head) at each head_dim
    (2, 1, 256, 1, 64, "ring"),
    (4, 1, 64, 1, 32, "ring"),
    (1, 1, 128, 1, 0, "contig"),
    (2, 1, 512, 1, 0, "contig"),    # q staged over 2 KiB of the ring
    (4, 1, 512, 1, 0, "contig"),    # q staged over 4 KiB of the ring (64 KiB of LDS)
]
# g * Q of 8 or 16 rows per kv head has two kernels (decode_kernel="auto"
# picks one by shape): run those shapes on each, forced.
_DECODE_CASES = [s + ("auto",) for s in _DECODE_SHAPES] + [
    s + (kern,) for s in _DECODE_SHAPES if (s[0] // s[1]) * s[3] in (8, 16) for kern in ("valu", "mfma")]


@pytest.mark.parametrize("hq,hkv,d,qn,window,layout,kernel", _DECODE_CASES)
def test_decode_attention_matches_oracle(hq, hkv, d, qn, window, layout, kernel):
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(hq * 131 + d + qn)
    kw = {}
    if layout == "ring":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="ring", window=window, ring_rows=window + 4 - 1)
    elif layout == "paged":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="paged")
        kw = dict(block_size=16, pool_pages=256)
    else:
        spec = LayerSpec(kv_heads=hkv, head_dim=d, window=window)
    rt = _rt([spec], n_slots=4, capacity=1024, max_q=4, decode_kernel=kernel, **kw)
    orc = O.OracleCache(_oracle_layers([spec]), 4)
    slots = [3, 1, 0]
    lens = [517, 33, 200]
    for s, n in zip(slots, lens):
        k = randn_bf16(gen, (1, hkv, n, d))
        v = randn_bf16(gen, (1, hkv, n, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    scale = 1.0 / math.sqrt(d)
    for step in range(3):
        q = randn_bf16(gen, (len(slots), hq, qn, d), 0.5)
        k = randn_bf16(gen, (len(slots), hkv, qn, d), 0.5)
        v = randn_bf16(gen, (len(slots), hkv, qn, d), 0.5)
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), slots, scale)
        for i, s in enumerate(slots):
            orc.append(s, 0, to_np(k[i]), to_np(v[i]))
            ref = orc.attend(s, 0, to_np(q[i]), scale)
            got = to_np(out[i])
            err = np.abs(got - ref).max()
            assert err <= ATOL, (step, s, err)
    assert rt.health() == 0
    _assert_gather_equal(rt, orc, 0, slots, ring_window=window if layout == "ring" else 0)


def test_fused_equals_append_then_attend_bitwise():
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(5)
    spec = LayerSpec(kv_heads=8, head_dim=128)
    rt_a = _rt([spec], n_slots=2, capacity=2048, max_q=2)
    rt_b = _rt([spec], n_slots=2, capacity=2048, max_q=2)
    for s in range(2):
        k = randn_bf16(gen, (1, 8, 1500, 128))
        v = randn_bf16(gen, (1, 8, 1500, 128))
        rt_a.import_(s, 0, k.cuda(), v.cuda())
        rt_b.import_(s, 0, k.cuda(), v.cuda())
    for _ in range(4):
        q = randn_bf16(gen, (2, 16, 1, 128)).cuda()
        k = randn_bf16(gen, (2, 8, 1, 128)).cuda()
        v = randn_bf16(gen, (2, 8, 1, 128)).cuda()
        oa = rt_a.append_attend(0, q, k, v, [0, 1], 0.088)
        rt_b.append(0, k, v, [0, 1])
        ob = rt_b.attend(0, q, [0, 1], 0.088)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(oa), bits(ob))
    np.testing.assert_array_equal(bits(rt_a.storage(0)[0]), bits(rt_b.storage(0)[0]))


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_paged_int8_quantise_dequantise_attend_and_evict(kernel):
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(4)
    spec = LayerSpec(kv_heads=8, head_dim=128, layout="paged", dtype="int8", window=96)
    rt = _rt([spec], n_slots=3, capacity=1024, max_q=1, block_size=16, pool_pages=128, decode_kernel=kernel)
    orc = O.OracleCache(_oracle_layers([spec]), 3)
    lens = {0: 300, 2: 130}
    for s, n in lens.items():
        k = randn_bf16(gen, (1, 8, n, 128))
        v = randn_bf16(gen, (1, 8, n, 128))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    _assert_gather_equal(rt, orc, 0, [0, 2])
    slots = [0, 2]
    for step in range(40):
        q = randn_bf16(gen, (2, 16, 1, 128), 0.5)
        k = randn_bf16(gen, (2, 8, 1, 128), 0.5)
        v = randn_bf16(gen, (2, 8, 1, 128), 0.5)
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), slots, 1 / math.sqrt(128))
        for i, s in enumerate(slots):
            orc.append(s, 0, to_np(k[i]), to_np(v[i]))
            ref = orc.attend(s, 0, to_np(q[i]), 1 / math.sqrt(128))
            assert np.abs(to_np(out[i]) - ref).max() <= ATOL
            # evict pages wholly older than the next step's window start
            L = rt.seq_length(s, 0)
            rt.evict(s, L + 1 - 96 + 1 - 1)
    assert rt.health() == 0
    c = rt.counters()
    assert c["pages_evicted"] > 0
    # evicted pages were recycled to the free list: pool usage stays bounded
    assert c["pages_in_use"] <= 2 * (96 // 16 + 2) + 2


@pytest.mark.parametrize("dtype,kernel", [("bf16", "auto"), ("int8", "valu"), ("int8", "mfma")])
def test_paged_decode_past_the_preloaded_page_window(dtype, kernel):
    """A wave preloads the page-table entries of its first 64 pages and looks
    further pages up directly: with one workgroup per (session, kv head)
    (decode_wgs 1) a 5000-key session gives each wave ~78 pages of 16 keys,
    so both lookups are exercised; pages come from a shuffled pool."""
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(17)
    spec = LayerSpec(kv_heads=8, head_dim=128, layout="paged", dtype=dtype)
    rt = _rt([spec], n_slots=2, capacity=5200, max_q=1, block_size=16, pool_pages=700, pool_seed=9,
             decode_wgs=1, decode_kernel=kernel)
    orc = O.OracleCache(_oracle_layers([spec]), 2)
    for s, n in ((0, 5000), (1, 777)):
        k = randn_bf16(gen, (1, 8, n, 128))
        v = randn_bf16(gen, (1, 8, n, 128))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    for step in range(2):
        q = randn_bf16(gen, (2, 16, 1, 128), 0.5)
        out = rt.attend(0, q.cuda(), [0, 1], 1 / math.sqrt(128))
        for i in range(2):
            ref = orc.attend(i, 0, to_np(q[i]), 1 / math.sqrt(128))
            assert np.abs(to_np(out[i]) - ref).max() <= ATOL
        k = randn_bf16(gen, (2, 8, 1, 128), 0.5)
        rt.append(0, k.cuda(), k.cuda(), [0, 1])
        for i in range(2):
            orc.append(i, 0, to_np(k[i]), to_np(k[i]))
    assert rt.health() == 0


@pytest.mark.parametrize("d,hq,hkv,qn", [(128, 16, 8, 1), (64, 4, 1, 2), (256, 8, 2, 2), (512, 8, 1, 1),
                                         (128, 8, 8, 1), (128, 4, 1, 1)])
@pytest.mark.parametrize("kernel", ["valu", "mfma"])
def test_int8_paged_decode_matches_oracle(d, hq, hkv, qn, kernel):
    """INT8 PAGED decode on both kernels (the MFMA kernel converts the int8
    rows to bf16 operands and applies the K scale to the scores and the V
    scale to the probabilities), head dims 64..512, 1..8 rows per kv head,
    ragged lengths over a shuffled pool."""
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(d + hq + qn)
    spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="paged", dtype="int8")
    rt = _rt([spec], n_slots=3, capacity=1100, max_q=2, block_size=16, pool_pages=3 * 72, pool_seed=3,
             decode_kernel=kernel)
    orc = O.OracleCache(_oracle_layers([spec]), 3)
    slots = [2, 0, 1]
    for s, n in zip(slots, (1000, 37, 431)):
        k = randn_bf16(gen, (1, hkv, n, d))
        v = randn_bf16(gen, (1, hkv, n, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    scale = 1 / math.sqrt(d)
    for step in range(2):
        q = randn_bf16(gen, (3, hq, qn, d), 0.5)
        k = randn_bf16(gen, (3, hkv, qn, d), 0.5)
        v = randn_bf16(gen, (3, hkv, qn, d), 0.5)
        rt.append(0, k.cuda(), v.cuda(), slots)
        out = rt.attend(0, q.cuda(), slots, scale)
        for i, s in enumerate(slots):
            orc.append(s, 0, to_np(k[i]), to_np(v[i]))
            err = np.abs(to_np(out[i]) - orc.attend(s, 0, to_np(q[i]), scale)).max()
            assert err <= ATOL, (step, s, err)
    assert rt.health() == 0


def test_gather_then_attend_tensors_matches_oracle():
    """Listener micro-batch path: ragged gather -> padded batch -> attend."""
    from kvrt import LayerSpec, attend_tensors

    gen = torch.Generator().manual_seed(2)
    spec = LayerSpec(kv_heads=8, head_dim=128)
    rt = _rt([spec], n_slots=4, capacity=1200, max_q=2)
    orc = O.OracleCache(_oracle_layers([spec]), 4)
    lens = [64, 1024, 377, 512]
    for s, n in enumerate(lens):
        k = randn_bf16(gen, (1, 8, n, 128))
        v = randn_bf16(gen, (1, 8, n, 128))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    slots = [0, 1, 2, 3]
    kpad, vpad, mask = rt.gather(0, slots)
    lengths = mask.sum(dim=1).to(torch.int32)
    assert lengths.tolist() == lens
    q = randn_bf16(gen, (4, 8, 2, 128), 0.5)
    out = attend_tensors(q.cuda(), kpad, vpad, lengths, 1 / math.sqrt(128))
    for i, s in enumerate(slots):
        ref = orc.attend(s, 0, to_np(q[i]), 1 / math.sqrt(128))
        assert np.abs(to_np(out[i]) - ref).max() <= ATOL

    # the same gather into caller-owned strided views of larger buffers (a
    # static padding workspace), mask included: bit-identical, and returned
    kbuf = torch.full((4, 8, 1100, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    vbuf = torch.full_like(kbuf, -3.0)
    mbuf = torch.ones((4, 1100), dtype=torch.bool, device="cuda")
    lm = kpad.shape[2]
    out3 = (kbuf[:, :, :lm], vbuf[:, :, :lm], mbuf[:, :lm])
    k2, v2, m2 = rt.gather(0, slots, out=out3)
    assert m2.data_ptr() == mbuf.data_ptr()
    np.testing.assert_array_equal(bits(k2), bits(kpad))
    np.testing.assert_array_equal(bits(v2), bits(vpad))
    assert torch.equal(m2, mask)
    assert bool(mbuf[:, lm:].all())  # nothing written past Lmax
    with pytest.raises(ValueError):
        rt.gather(0, slots, out=(kbuf[:, :, :lm], vbuf[:, :, :lm], mbuf[:, :lm + 1]))
    with pytest.raises(ValueError):
        rt.gather(0, slots, out=(kbuf[:, :, :lm], vbuf[:, :, :lm], mbuf[:, :lm].float()))


def test_copy_prefix_and_copy_rows_bitexact():
    from kvrt import LayerSpec, copy_rows

    gen = torch.Generator().manual_seed(7)
    spec = LayerSpec(kv_heads=1, head_dim=256)
    rt = _rt([spec, spec], n_slots=2, capacity=300, max_q=2)
    orc = O.OracleCache(_oracle_layers([spec, spec]), 2)
    for layer in range(2):
        k = randn_bf16(gen, (1, 1, 250, 256))
        rt.import_(0, layer, k.cuda(), k.cuda())
        orc.append(0, layer, to_np(k[0]), to_np(k[0]))
        orc.append(1, layer, to_np(k[0]), to_np(k[0]))
        orc.truncate(1, layer, 97)
    rt.copy_prefix(0, 1, 97)
    for layer in range(2):
        assert rt.seq_length(1, layer) == 97
        _assert_gather_equal(rt, orc, layer, [1])
    src = randn_bf16(gen, (1, 2, 40, 64)).cuda()
    dst = torch.zeros((1, 2, 64, 64), dtype=torch.bfloat16, device="cuda")
    copy_rows(src, dst, 33)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(dst[:, :, :33]), bits(src[:, :, :33]))
    assert int(torch.count_nonzero(dst[:, :, 33:])) == 0


def test_single_key_and_uniform_score_invariants():
    """Closed forms: one visible key -> o = v; equal scores -> mean of V."""
    from kvrt import LayerSpec

    spec = LayerSpec(kv_heads=1, head_dim=256, layout="ring", window=1, ring_rows=1)
    rt = _rt([spec], n_slots=1, capacity=4096, max_q=1)
    gen = torch.Generator().manual_seed(9)
    for _ in range(5):
        q = randn_bf16(gen, (1, 8, 1, 256)).cuda()
        k = randn_bf16(gen, (1, 1, 1, 256)).cuda()
        v = randn_bf16(gen, (1, 1, 1, 256)).cuda()
        out = rt.append_attend(0, q, k, v, [0], 0.0625)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(out), bits(v.expand(1, 8, 1, 256)))
    spec = LayerSpec(kv_heads=2, head_dim=128)
    rt = _rt([spec], n_slots=1, capacity=2048, max_q=1)
    key = randn_bf16(gen, (1, 2, 1, 128))
    vals = randn_bf16(gen, (1, 2, 1500, 128))
    rt.import_(0, 0, key.expand(1, 2, 1500, 128).contiguous().cuda(), vals.cuda())
    q = randn_bf16(gen, (1, 4, 1, 128)).cuda()
    out = rt.attend(0, q, [0], 0.1)
    mean = to_np(vals[0]).astype(np.float64).mean(axis=1)  # [2, 128]
    got = to_np(out[0, :, 0])  # [4, 128]
    assert np.abs(got - np.repeat(mean, 2, axis=0)).max() <= 4e-3


def test_error_paths_fail_closed_and_poison():
    from kvrt import KVRTError, LayerSpec

    spec = LayerSpec(kv_heads=2, head_dim=128)
    rt = _rt([spec], n_slots=2, capacity=8, max_q=2)
    k = torch.zeros((1, 2, 2, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(KVRTError) as e:
        rt.append(0, k, k, [5])  # bad slot
    assert e.value.code == -1
    with pytest.raises(KVRTError):
        rt.append(0, k, k, [0, 0])  # duplicate slots
    for _ in range(4):
        rt.append(0, k[:1], k[:1], [0])
    with pytest.raises(KVRTError) as e:
        rt.append(0, k[:1], k[:1], [0])  # capacity 8 reached
    assert e.value.code == -2
    with pytest.raises(KVRTError) as e:
        rt.truncate(0, 9)  # beyond current length
    assert e.value.code == -2
    assert rt.health() == 0  # argument errors do not poison
    rt.lib.kvrt_debug_inject_failure(rt._ctx)
    with pytest.raises(KVRTError) as e:
        rt.truncate(0, 4)
    assert e.value.code == -3
    with pytest.raises(KVRTError) as e:
        rt.append(0, k[:1], k[:1], [1])
    assert e.value.code == -4
    assert rt.health() == -4


@pytest.mark.parametrize("hq,hkv,d,length,kernel", [(16, 1, 512, 16000, "auto"), (16, 8, 128, 16000, "auto"),
                                                   (8, 1, 256, 9000, "valu"), (8, 1, 256, 9000, "mfma")])
def test_many_splits_long_context(hq, hkv, d, length, kernel):
    """One stream, long context: the split count hits its cap (64 workgroups
    per kv head; 256 wave partials when the workgroup merge is off)."""
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(length + d)
    spec = LayerSpec(kv_heads=hkv, head_dim=d)
    rt = _rt([spec], n_slots=1, capacity=length + 4, max_q=1, decode_kernel=kernel)
    orc = O.OracleCache(_oracle_layers([spec]), 1)
    k = randn_bf16(gen, (1, hkv, length, d))
    v = randn_bf16(gen, (1, hkv, length, d))
    rt.import_(0, 0, k.cuda(), v.cuda())
    orc.append(0, 0, to_np(k[0]), to_np(v[0]))
    q = randn_bf16(gen, (1, hq, 1, d), 0.5)
    kn = randn_bf16(gen, (1, hkv, 1, d), 0.5)
    vn = randn_bf16(gen, (1, hkv, 1, d), 0.5)
    out = rt.append_attend(0, q.cuda(), kn.cuda(), vn.cuda(), [0], 1 / math.sqrt(d))
    orc.append(0, 0, to_np(kn[0]), to_np(vn[0]))
    ref = orc.attend(0, 0, to_np(q[0]), 1 / math.sqrt(d))
    assert np.abs(to_np(out[0]) - ref).max() <= ATOL
    assert rt.health() == 0
