"""The two ways a split-K decode combines its workgroup partials
(kvrt_config.decode_merge): a second merge kernel (SEPARATE) or the last
workgroup of each (slot, kv head) inside the decode launch (LAST_WG). With at
most 16 partial workgroups per (slot, kv head) both merge in the same order,
so their outputs must agree bit for bit; fresh q/k/v on every step make a
partial left over from an earlier launch show up as a mismatch. Lengths and
appended rows must agree too, and LAST_WG must issue one launch per call."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu

# (hq, hkv, d, qn, layout, window, dtype, decode_wgs): decode_wgs keeps the
# partial workgroups per (slot, kv head) at or below 16.
_CASES = [
    (16, 8, 128, 1, "contig", 0, "bf16", 96),    # talker shape, DMA ring kernel
    (16, 8, 128, 2, "contig", 0, "bf16", 96),
    (8, 1, 256, 1, "ring", 64, "bf16", 24),      # thinker sliding, 8 rows per kv head (VALU)
    (8, 1, 256, 1, "contig", 0, "bf16", 48),     # thinker global
    (2, 1, 512, 1, "contig", 0, "bf16", 48),     # D 512, DMA ring
    (8, 1, 256, 2, "contig", 0, "bf16", 48),     # 16 rows per kv head: MFMA kernel
    (8, 1, 512, 1, "contig", 0, "bf16", 48),     # 8 rows at D 512: MFMA kernel
    (16, 8, 128, 1, "paged", 0, "int8", 96),     # paged int8
    (16, 8, 128, 1, "paged", 0, "bf16", 96),
]


def _runtime(spec, n, capacity, merge, wgs, **kw):
    from kvrt import KVRuntime

    return KVRuntime([spec], n, capacity, max_q=2, decode_wgs=wgs, decode_merge=merge, device="cuda", **kw)


@pytest.mark.parametrize("hq,hkv,d,qn,layout,window,dtype,wgs", _CASES)
def test_last_workgroup_merge_equals_the_merge_kernel(hq, hkv, d, qn, layout, window, dtype, wgs):
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(hq * 7 + d + qn)
    kw = {}
    if layout == "ring":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="ring", window=window, ring_rows=window + 1)
    elif layout == "paged":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="paged", dtype=dtype)
        kw = dict(block_size=16, pool_pages=512)
    else:
        spec = LayerSpec(kv_heads=hkv, head_dim=d, window=window)
    slots = [2, 0, 3]
    lens = [700, 45, 1300]
    rts = {m: _runtime(spec, 4, 1500, m, wgs, **kw) for m in ("separate", "last_wg")}
    for s, n in zip(slots, lens):
        k = randn_bf16(gen, (1, hkv, n, d)).cuda()
        v = randn_bf16(gen, (1, hkv, n, d)).cuda()
        for rt in rts.values():
            rt.import_(s, 0, k, v)
    scale = 1.0 / math.sqrt(d)
    for step in range(10):
        q = randn_bf16(gen, (len(slots), hq, qn, d), 0.5).cuda()
        k = randn_bf16(gen, (len(slots), hkv, qn, d), 0.5).cuda()
        v = randn_bf16(gen, (len(slots), hkv, qn, d), 0.5).cuda()
        outs, launches = {}, {}
        for m, rt in rts.items():
            before = rt.counters()["launches"]
            if dtype == "int8":  # int8 layers quantise on append, then attend
                rt.append(0, k, v, slots)
                mid = rt.counters()["launches"]
                outs[m] = rt.attend(0, q, slots, scale)
                launches[m] = rt.counters()["launches"] - mid
            else:  # (PAGED: plus a page-table update when a page is mapped)
                outs[m] = rt.append_attend(0, q, k, v, slots, scale)
                launches[m] = rt.counters()["launches"] - before
        assert launches["separate"] == launches["last_wg"] + 1, launches
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(outs["separate"]), bits(outs["last_wg"]), err_msg=f"step {step}")
    for rt in rts.values():
        assert rt.health() == 0
    for s, n in zip(slots, lens):
        assert rts["separate"].seq_length(s, 0) == rts["last_wg"].seq_length(s, 0) == n + 10 * qn
    ka, va, _ = rts["separate"].gather(0, slots)
    kb, vb, _ = rts["last_wg"].gather(0, slots)
    np.testing.assert_array_equal(bits(ka), bits(kb))
    np.testing.assert_array_equal(bits(va), bits(vb))


def test_last_workgroup_merge_with_many_partials_matches_oracle():
    """More than 16 partial workgroups per (slot, kv head): LAST_WG merges them
    in one pass of its own order, so it is held to the oracle tolerance."""
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(17)
    spec = LayerSpec(kv_heads=1, head_dim=256)
    rt = _runtime(spec, 2, 6000, "last_wg", 0, decode_kernel="valu")  # AUTO runs this shape on MFMA
    orc = O.OracleCache([O.OracleLayer(1, 256, 0, False)], 2)
    for s, n in ((0, 5000), (1, 3100)):
        k = randn_bf16(gen, (1, 1, n, 256))
        v = randn_bf16(gen, (1, 1, n, 256))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    for step in range(3):
        q = randn_bf16(gen, (2, 8, 1, 256), 0.5)
        k = randn_bf16(gen, (2, 1, 1, 256), 0.5)
        v = randn_bf16(gen, (2, 1, 1, 256), 0.5)
        before = rt.counters()["launches"]
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), [0, 1], 1 / 16)
        assert rt.counters()["launches"] - before == 1
        for i in range(2):
            orc.append(i, 0, to_np(k[i]), to_np(v[i]))
            err = np.abs(to_np(out[i]) - orc.attend(i, 0, to_np(q[i]), 1 / 16)).max()
            assert err <= 1e-2, (step, i, err)
    assert rt.health() == 0


def test_talker_masks_last_workgroup_merge_equals_the_merge_kernel():
    from kvrt import KVRuntime, LayerSpec, TalkerMask

    gen = torch.Generator().manual_seed(29)
    rts = {m: KVRuntime([LayerSpec(kv_heads=8, head_dim=128)], 2, 1024, max_q=2, decode_wgs=64, decode_merge=m,
                        device="cuda") for m in ("separate", "last_wg")}
    k = randn_bf16(gen, (1, 8, 900, 128)).cuda()
    v = randn_bf16(gen, (1, 8, 900, 128)).cuda()
    for rt in rts.values():
        for s in range(2):
            rt.import_(s, 0, k, v)
    masks = [TalkerMask(prefix_start=300, audio_start=620, prefix_position=450, audio_position=899,
                        prefix_attention_mode=mode, visible_prefix_count=151, prefix_log_gate=-0.7)
             for mode in (0, 2)]
    for step in range(4):
        q = randn_bf16(gen, (2, 16, 2, 128), 0.5).cuda()
        outs = {m: rt.attend_talker(0, q, [0, 1], 0.088, masks) for m, rt in rts.items()}
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(outs["separate"]), bits(outs["last_wg"]), err_msg=f"step {step}")
    for rt in rts.values():
        assert rt.health() == 0


def test_last_workgroup_merge_many_layers_and_steps():
    """The talker topology of the north-star step (28 layers, 4 streams,
    16 / 8 heads, D 128, fused append) for 8 steps, fresh q/k/v per layer and
    step: 224 single-launch decodes, each compared bit for bit with the merge
    kernel's result, so that a partial read before it landed, or a counter
    left non-zero by an earlier launch, shows up."""
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(41)
    specs = [LayerSpec(kv_heads=8, head_dim=128)] * 28
    rts = {m: _runtime_layers(specs, 4, 700, m) for m in ("separate", "last_wg")}
    for layer in range(28):
        k = randn_bf16(gen, (1, 8, 600, 128)).cuda()
        v = randn_bf16(gen, (1, 8, 600, 128)).cuda()
        for rt in rts.values():
            for s in range(4):
                rt.import_(s, layer, k, v)
    slots = [0, 1, 2, 3]
    for step in range(8):
        for layer in range(28):
            q = randn_bf16(gen, (4, 16, 1, 128), 0.5).cuda()
            k = randn_bf16(gen, (4, 8, 1, 128), 0.5).cuda()
            v = randn_bf16(gen, (4, 8, 1, 128), 0.5).cuda()
            outs = {m: rt.append_attend(layer, q, k, v, slots, 0.088) for m, rt in rts.items()}
            np.testing.assert_array_equal(bits(outs["separate"]), bits(outs["last_wg"]),
                                          err_msg=f"step {step} layer {layer}")
    for rt in rts.values():
        assert rt.health() == 0
        assert rt.seq_length(3, 27) == 608


def _runtime_layers(specs, n, capacity, merge):
    from kvrt import KVRuntime

    return KVRuntime(specs, n, capacity, max_q=1, decode_wgs=192, decode_merge=merge, device="cuda")
