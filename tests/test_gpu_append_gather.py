"""kvrt_append_gather_async against kvrt_append_async + kvrt_gather_async:
two runtimes with the same imported caches take the same steps, one through
the fused call, one through the two calls. The padded K/V batches, masks,
lengths and, at the end, the whole caches must agree bit for bit (the
two-call path is held to the oracle by the gather and append tests); the
appended rows of the batch must equal the k / v given. CONTIG and RING
layers take one launch, PAGED layers the two-launch route inside the call.
A captured graph of the fused call replays at advancing device lengths."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import bits, randn_bf16

pytestmark = pytest.mark.gpu


def _pair(spec, n, capacity, **kw):
    from kvrt import KVRuntime

    return [KVRuntime([spec], n, capacity, max_q=2, device="cuda", **kw) for _ in range(2)]


def _specs():
    from kvrt import LayerSpec

    return {
        "contig": (LayerSpec(kv_heads=8, head_dim=128), {}),
        "ring": (LayerSpec(kv_heads=1, head_dim=256, layout="ring", window=64, ring_rows=64 + 2 - 1), {}),
        "paged": (LayerSpec(kv_heads=2, head_dim=128, layout="paged"), dict(block_size=16, pool_pages=256)),
    }


@pytest.mark.parametrize("qn", [1, 2])
@pytest.mark.parametrize("layout", ["contig", "ring", "paged"])
def test_fused_append_gather_equals_append_then_gather(layout, qn):
    spec, kw = _specs()[layout]
    gen = torch.Generator().manual_seed(len(layout) * 10 + qn)
    n, hkv, d = 3, spec.kv_heads, spec.head_dim
    lens = [300, 17, 129]
    two, fused = _pair(spec, 4, 600, **kw)
    slots = [2, 0, 3]
    for s, ln in zip(slots, lens):
        k, v = randn_bf16(gen, (1, hkv, ln, d)).cuda(), randn_bf16(gen, (1, hkv, ln, d)).cuda()
        two.import_(s, 0, k, v)
        fused.import_(s, 0, k, v)
    lmax = 340 if layout != "ring" else 64
    for step in range(6):
        k = randn_bf16(gen, (n, hkv, qn, d)).cuda()
        v = randn_bf16(gen, (n, hkv, qn, d)).cuda()
        outs = []
        for rt, is_fused in ((two, False), (fused, True)):
            ok = torch.full((n, hkv, lmax, d), float("nan"), dtype=torch.bfloat16, device="cuda")
            ov = torch.full_like(ok, float("nan"))
            mk = torch.empty((n, lmax), dtype=torch.bool, device="cuda")
            before = rt.counters()["launches"]
            if is_fused:
                rt.append_gather(0, k, v, slots, out=(ok, ov, mk))
            else:
                rt.append(0, k, v, slots)
                rt.gather(0, slots, out=(ok, ov, mk))
            launches = rt.counters()["launches"] - before
            outs.append((ok, ov, mk, launches))
        torch.cuda.synchronize()
        (ka, va, ma, la), (kb, vb, mb, lb) = outs
        np.testing.assert_array_equal(bits(ka), bits(kb), err_msg=f"step {step}")
        np.testing.assert_array_equal(bits(va), bits(vb), err_msg=f"step {step}")
        np.testing.assert_array_equal(ma.cpu().numpy(), mb.cpu().numpy())
        assert lb == (1 if layout != "paged" else la), (la, lb)
        # the appended rows sit at the end of each item's valid range
        for i, s in enumerate(slots):
            length = fused.seq_length(s, 0)
            start = max(0, length - (spec.window - 1)) if layout == "ring" else 0
            row = length - start - qn
            assert torch.equal(kb[i, :, row:row + qn], k[i]) and torch.equal(vb[i, :, row:row + qn], v[i])
    for s in slots:
        assert two.seq_length(s, 0) == fused.seq_length(s, 0)
    assert two.health() == 0 and fused.health() == 0
    ka, va, _ = two.gather(0, slots)
    kb, vb, _ = fused.gather(0, slots)
    np.testing.assert_array_equal(bits(ka), bits(kb))
    np.testing.assert_array_equal(bits(va), bits(vb))


@pytest.mark.parametrize("layout", ["contig", "ring"])
def test_fused_append_gather_graph_replays_at_advancing_lengths(layout):
    """One captured fused call (4 slots, Q 2; CONTIG 8 x D 128, or RING
    window 64 / 65 rows, 1 x D 256) replayed 8 times with fresh rows copied
    in: every replay's batch and mask equal the two eager calls of a second
    runtime bit for bit (on RING the window start moves with the device
    length), and the device lengths advance by 2."""
    spec, _ = _specs()[layout]
    gen = torch.Generator().manual_seed(11)
    n, hkv, d, qn = 4, spec.kv_heads, spec.head_dim, 2
    lmax = 700 if layout == "contig" else 64
    two, fused = _pair(spec, n, 720)
    lens = [454, 610, 334, 542]
    slots = list(range(n))
    for s, ln in zip(slots, lens):
        k, v = randn_bf16(gen, (1, hkv, ln, d)).cuda(), randn_bf16(gen, (1, hkv, ln, d)).cuda()
        two.import_(s, 0, k, v)
        fused.import_(s, 0, k, v)
    kin = torch.empty((n, hkv, qn, d), dtype=torch.bfloat16, device="cuda")
    vin = torch.empty_like(kin)
    okb = torch.empty((n, hkv, lmax, d), dtype=torch.bfloat16, device="cuda")
    ovb = torch.empty_like(okb)
    mkb = torch.empty((n, lmax), dtype=torch.bool, device="cuda")
    fused.append_gather(0, kin.zero_(), vin.zero_(), slots, out=(okb, ovb, mkb))  # eager call first
    two.append(0, kin, vin, slots)
    torch.cuda.synchronize()
    fused.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fused.append_gather(0, kin, vin, slots, out=(okb, ovb, mkb))
    fused.sync_lengths()
    for r in range(8):
        k, v = randn_bf16(gen, (n, hkv, qn, d)).cuda(), randn_bf16(gen, (n, hkv, qn, d)).cuda()
        kin.copy_(k)
        vin.copy_(v)
        g.replay()
        two.append(0, k, v, slots)
        ka, va, ma = two.gather(0, slots, lmax=lmax)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(okb), bits(ka), err_msg=f"replay {r}")
        np.testing.assert_array_equal(bits(ovb), bits(va), err_msg=f"replay {r}")
        np.testing.assert_array_equal(mkb.cpu().numpy(), ma.cpu().numpy())
    fused.sync_lengths()
    assert [fused.seq_length(s, 0) for s in slots] == [ln + 2 * 9 for ln in lens]
    assert fused.health() == 0 and two.health() == 0


def test_fused_append_gather_refusals_change_nothing():
    """Past capacity: KVRT_ESTATE, no row written, no length moved; a
    strided k / v takes the two-launch route with the same result."""
    from kvrt import KVRTError

    spec, _ = _specs()["contig"]
    gen = torch.Generator().manual_seed(5)
    hkv, d = 8, 128
    two, fused = _pair(spec, 2, 100)
    for rt in (two, fused):
        rt.import_(0, 0, torch.zeros((1, hkv, 99, d), dtype=torch.bfloat16, device="cuda"),
                   torch.zeros((1, hkv, 99, d), dtype=torch.bfloat16, device="cuda"))
    ok = torch.empty((1, hkv, 100, d), dtype=torch.bfloat16, device="cuda")
    ov = torch.empty_like(ok)
    k = randn_bf16(gen, (1, hkv, 2, d)).cuda()
    with pytest.raises(KVRTError):
        fused.append_gather(0, k, k, [0], out=(ok, ov))
    assert fused.seq_length(0, 0) == 99
    # strided k / v ([n, Q, hkv, D] storage seen as [n, hkv, Q, D])
    ks = randn_bf16(gen, (1, 2, hkv, d)).cuda().permute(0, 2, 1, 3)
    vs = randn_bf16(gen, (1, 2, hkv, d)).cuda().permute(0, 2, 1, 3)
    assert not ks.is_contiguous()
    for rt in (two, fused):
        rt.import_(1, 0, torch.ones((1, hkv, 5, d), dtype=torch.bfloat16, device="cuda"),
                   torch.ones((1, hkv, 5, d), dtype=torch.bfloat16, device="cuda"))
    two.append(0, ks, vs, [1])
    ka, va, _ = two.gather(0, [1], lmax=100)
    ob = torch.empty((1, hkv, 100, d), dtype=torch.bfloat16, device="cuda")
    before = fused.counters()["launches"]
    kb, vb, _ = fused.append_gather(0, ks, vs, [1], out=(ob, torch.empty_like(ob)))
    assert fused.counters()["launches"] - before == 2  # the append, then the gather
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(ka), bits(kb))
    np.testing.assert_array_equal(bits(va), bits(vb))
    assert fused.health() == 0


def test_fused_append_gather_at_the_item_and_head_limits():
    """64 slots x 64 kv heads in one call (every per-(item, head) and
    per-item arrival counter in use), three steps: bit for bit the two calls,
    lengths advanced on every slot."""
    from kvrt import LayerSpec

    spec = LayerSpec(kv_heads=64, head_dim=64)
    gen = torch.Generator().manual_seed(64)
    n, hkv, d = 64, 64, 64
    two, fused = _pair(spec, n, 64)
    lens = [int(x) for x in torch.randint(0, 40, (n,), generator=gen)]
    slots = list(range(n))[::-1]
    for s, ln in zip(slots, lens):
        if ln:
            k, v = randn_bf16(gen, (1, hkv, ln, d)).cuda(), randn_bf16(gen, (1, hkv, ln, d)).cuda()
            two.import_(s, 0, k, v)
            fused.import_(s, 0, k, v)
    for step in range(3):
        k, v = randn_bf16(gen, (n, hkv, 2, d)).cuda(), randn_bf16(gen, (n, hkv, 2, d)).cuda()
        lm = max(lens) + 2 * (step + 1)
        two.append(0, k, v, slots)
        ka, va, ma = two.gather(0, slots, lmax=lm)
        kb = torch.empty((n, hkv, lm, d), dtype=torch.bfloat16, device="cuda")
        vb, mb = torch.empty_like(kb), torch.empty((n, lm), dtype=torch.bool, device="cuda")
        fused.append_gather(0, k, v, slots, out=(kb, vb, mb))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(ka), bits(kb), err_msg=f"step {step}")
        np.testing.assert_array_equal(bits(va), bits(vb), err_msg=f"step {step}")
        np.testing.assert_array_equal(ma.cpu().numpy(), mb.cpu().numpy())
    fused.sync_lengths()
    assert [fused.seq_length(s, 0) for s in slots] == [ln + 6 for ln in lens]
    assert fused.health() == 0 and two.health() == 0
