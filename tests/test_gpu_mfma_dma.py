"""GPU parity of the MFMA decode's LDS DMA ring (bf16 CONTIG / RING, D 128 and
256, 1, 2, 4 or 8 query rows per KV head over >= 2048 keys, the shapes AUTO sends
to it) against the oracle at max-abs 1e-2, beside the same launches forced
onto the VALU kernel: wave ranges of many tiles, of one or two tiles and
empty ones (decode_wgs 8 / 64 / 512), partial last tiles, fused appends and a
canonical prefix mask on one slot. The forced "mfma" kernel choice is also
checked on short caches and on the PAGED layout, which AUTO leaves to VALU."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2


@pytest.mark.parametrize("wgs", [8, 64, 512])
@pytest.mark.parametrize("layout", ["contig", "ring"])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
@pytest.mark.parametrize("d", [128, 256])
def test_mfma_dma_decode_parity(d, group, layout, wgs):
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(100 * group + wgs + len(layout) + d)
    hkv = 2
    window = 2304 if layout == "ring" else 0
    ring = dict(ring_rows=window) if layout == "ring" else {}
    spec = LayerSpec(kv_heads=hkv, head_dim=d, layout=layout, window=window, **ring)
    rts = {kern: KVRuntime([spec], 3, 4200, max_q=1, decode_wgs=wgs, decode_kernel=kern, device="cuda")
           for kern in ("auto", "valu")}
    orc = O.OracleCache([O.OracleLayer(hkv, d, window)], 3)
    lens = [2100, 4097, 3001]
    for s, n in enumerate(lens):
        k, v = randn_bf16(gen, (1, hkv, n, d)), randn_bf16(gen, (1, hkv, n, d))
        for rt in rts.values():
            rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    mask = O.canonical_prefix_mask(34)
    for rt in rts.values():
        rt.set_prefix_attention(1, torch.from_numpy(mask).cuda())
    orc.set_prefix_attention(1, mask)
    slots = [0, 1, 2]
    before = {name: rt.counters()["mfma_decodes"] for name, rt in rts.items()}
    worst = {name: 0.0 for name in rts}
    for _ in range(3):
        q = randn_bf16(gen, (3, hkv * group, 1, d), 1.0 / math.sqrt(d))
        k, v = randn_bf16(gen, (3, hkv, 1, d)), randn_bf16(gen, (3, hkv, 1, d))
        outs = {name: rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), slots, 1.0) for name, rt in rts.items()}
        torch.cuda.synchronize()
        for i, s in enumerate(slots):
            orc.append(s, 0, to_np(k[i]), to_np(v[i]))
            ref = orc.attend(s, 0, to_np(q[i]), 1.0)
            for name, out in outs.items():
                worst[name] = max(worst[name], float(np.abs(to_np(out[i]) - ref).max()))
    assert max(worst.values()) <= ATOL, worst
    # AUTO ran every launch on the MFMA kernel, the forced VALU runtime none
    assert rts["auto"].counters()["mfma_decodes"] - before["auto"] == 3
    assert rts["valu"].counters()["mfma_decodes"] - before["valu"] == 0
    for rt in rts.values():
        assert rt.health() == 0
        assert [rt.seq_length(s, 0) for s in slots] == [n + 3 for n in lens]


@pytest.mark.parametrize("lmax", [2304, 1024])
def test_tensor_path_clamps_a_length_beyond_the_view(lmax):
    """attend_tensors over caller-owned K/V [3, 8, Lmax, 128] with 16 q heads
    (2 rows per KV head: the MFMA DMA decode at Lmax 2304, the VALU kernel at
    1024): the item whose length exceeds Lmax attends over the Lmax rows it
    has (its query at position Lmax - 1) and raises the tensor path's device
    flag; the other items match the oracle."""
    from kvrt.runtime import attend_tensors, tensors_status

    gen = torch.Generator().manual_seed(lmax)
    n, hkv, hq, d = 3, 8, 16, 128
    k, v = randn_bf16(gen, (n, hkv, lmax, d)), randn_bf16(gen, (n, hkv, lmax, d))
    q = randn_bf16(gen, (n, hq, 1, d), 1.0 / math.sqrt(d))
    lens = [lmax - 4, lmax + 100, lmax // 2 + 3]
    out = attend_tensors(q.cuda(), k.cuda(), v.cuda(), torch.tensor(lens, dtype=torch.int32).cuda(), 1.0)
    assert tensors_status() == -6
    for i, ln in enumerate(lens):
        seen = min(ln, lmax)
        ref = O.attend(to_np(q[i]), to_np(k[i, :, :seen]), to_np(v[i, :, :seen]), np.array([seen - 1]), 1.0)
        assert float(np.abs(to_np(out[i]) - ref).max()) <= ATOL, (lmax, i)
    assert tensors_status() == 0  # the flag was cleared


@pytest.mark.parametrize("merge", ["separate", "last_wg"])
@pytest.mark.parametrize("kernel", ["auto", "valu", "mfma"])
@pytest.mark.parametrize("d,hkv,hq", [(128, 8, 16), (256, 1, 8)])
def test_ragged_batch_matches_the_oracle(d, hkv, hq, kernel, merge):
    """A ragged batch (4038 / 925 / 1269 / 130 / 2600 positions) in one
    launch: the split count follows the longest item, so the short items'
    waves hold a few keys or none, and every item's partials still merge to
    the oracle's attention, with the merge kernel or in the decode's last
    workgroup, over fused append steps."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(d + hkv + len(kernel) + len(merge))
    lens = [4038, 925, 1269, 130, 2600]
    n = len(lens)
    rt = KVRuntime([LayerSpec(kv_heads=hkv, head_dim=d)], n, 4200, max_q=1, decode_kernel=kernel,
                   decode_merge=merge, device="cuda")
    orc = O.OracleCache([O.OracleLayer(hkv, d)], n)
    for s, ln in enumerate(lens):
        k, v = randn_bf16(gen, (1, hkv, ln, d)), randn_bf16(gen, (1, hkv, ln, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    slots = list(range(n))
    worst = 0.0
    for _ in range(4):
        q = randn_bf16(gen, (n, hq, 1, d), 1.0 / math.sqrt(d))
        k, v = randn_bf16(gen, (n, hkv, 1, d)), randn_bf16(gen, (n, hkv, 1, d))
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), slots, 1.0)
        torch.cuda.synchronize()
        for i, s in enumerate(slots):
            orc.append(s, 0, to_np(k[i]), to_np(v[i]))
            worst = max(worst, float(np.abs(to_np(out[i]) - orc.attend(s, 0, to_np(q[i]), 1.0)).max()))
    assert worst <= ATOL, worst
    assert rt.health() == 0
    assert [rt.seq_length(s, 0) for s in slots] == [ln + 4 for ln in lens]


@pytest.mark.parametrize("layout", ["contig", "paged"])
def test_forced_mfma_small_rows_short_and_paged(layout):
    """decode_kernel="mfma" sends 2-row decodes to the MFMA kernel at any key
    count and layout: CONTIG at a few hundred keys (the DMA ring), PAGED
    (register-staged 8-row tiles over a shuffled page pool)."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(7 + len(layout))
    hkv, hq, d = 8, 16, 128
    lens = [300, 45, 1000]
    kw = dict(block_size=16, pool_pages=3 * (1100 // 16 + 4), pool_seed=3) if layout == "paged" else {}
    rt = KVRuntime([LayerSpec(kv_heads=hkv, head_dim=d, layout=layout)], 3, 1100, max_q=1, decode_kernel="mfma",
                   device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(hkv, d)], 3)
    for s, ln in enumerate(lens):
        k, v = randn_bf16(gen, (1, hkv, ln, d)), randn_bf16(gen, (1, hkv, ln, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    slots = [0, 1, 2]
    before = rt.counters()["mfma_decodes"]
    worst = 0.0
    for _ in range(3):
        q = randn_bf16(gen, (3, hq, 1, d), 1.0 / math.sqrt(d))
        k, v = randn_bf16(gen, (3, hkv, 1, d)), randn_bf16(gen, (3, hkv, 1, d))
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), slots, 1.0)
        torch.cuda.synchronize()
        for i, s in enumerate(slots):
            orc.append(s, 0, to_np(k[i]), to_np(v[i]))
            worst = max(worst, float(np.abs(to_np(out[i]) - orc.attend(s, 0, to_np(q[i]), 1.0)).max()))
    assert worst <= ATOL, worst
    assert rt.counters()["mfma_decodes"] - before == 3
    assert rt.health() == 0
