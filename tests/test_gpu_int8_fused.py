"""The fused int8 append + decode (one launch per layer: the decode quantises
the new rows in-kernel, stores them with their scales and maps their pages
through page-table edits carried in its launch arguments) against the append
kernel followed by the decode: two runtimes with the same pool order take the
same steps, and the stored int8 rows, scales, lengths and outputs must agree
bit for bit, over appends that cross into new pages. Both paths are held to
the CPU oracle by the config 5 test (tests/test_gpu_configs.py)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from tests.helpers import bits, randn_bf16

pytestmark = pytest.mark.gpu


def _rt(max_q, kernel="auto"):
    from kvrt import KVRuntime, LayerSpec

    spec = LayerSpec(kv_heads=8, head_dim=128, layout="paged", dtype="int8")
    return KVRuntime([spec], 4, 640, max_q=max_q, device="cuda", block_size=16, pool_pages=160, pool_seed=4,
                     decode_kernel=kernel)


def _raw(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


@pytest.mark.parametrize("kernel", ["auto", "mfma"])
@pytest.mark.parametrize("qn", [1, 2])
def test_fused_int8_append_attend_equals_append_then_attend(qn, kernel):
    """AUTO runs the VALU decode; a forced MFMA decode at this shape runs the
    int8 ring kernel, which quantises the new rows in its own launch too."""
    gen = torch.Generator().manual_seed(60 + qn)
    fused, two = _rt(qn, kernel), _rt(qn, kernel)
    slots = [3, 0, 1]
    lens = [37, 130, 79]  # the appends cross block boundaries on different steps
    for s, n in zip(slots, lens):
        k, v = randn_bf16(gen, (1, 8, n, 128)).cuda(), randn_bf16(gen, (1, 8, n, 128)).cuda()
        fused.import_(s, 0, k, v)
        two.import_(s, 0, k, v)
    scale = 1.0 / math.sqrt(128)
    for step in range(24):
        q = randn_bf16(gen, (3, 16, qn, 128), 0.5).cuda()
        k = randn_bf16(gen, (3, 8, qn, 128)).cuda()
        v = randn_bf16(gen, (3, 8, qn, 128)).cuda()
        before = fused.counters()["launches"]
        a = fused.append_attend(0, q, k, v, slots, scale)
        assert fused.counters()["launches"] - before == 1, step  # page edits included
        two.append(0, k, v, slots)
        b = two.attend(0, q, slots, scale)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(a), bits(b), err_msg=f"step {step}")
    for s, n in zip(slots, lens):
        assert fused.seq_length(s, 0) == two.seq_length(s, 0) == n + 24 * qn
    fused.sync_lengths()
    assert [fused.seq_length(s, 0) for s in slots] == [n + 24 * qn for n in lens]
    for x, y in zip(fused.storage(0), two.storage(0)):
        np.testing.assert_array_equal(_raw(x), _raw(y))
    assert fused.counters()["pages_in_use"] == two.counters()["pages_in_use"]
    assert fused.health() == 0 and two.health() == 0


def test_paged_int8_graph_replays_across_page_boundaries():
    """A captured fused int8 step over 3 PAGED slots replays 20 times across
    page boundaries once the pages are reserved (kvrt_reserve_async): every
    replay's output equals an eager runtime's bit for bit, the logical rows
    agree afterwards, and a replay past the reservation raises the device
    flag (the writer finds no page and stores nothing) instead of writing."""
    gen = torch.Generator().manual_seed(64)
    eager, graphed = _rt(1), _rt(1)
    slots = [3, 0, 1]
    lens = [37, 130, 79]
    for s, n in zip(slots, lens):
        k, v = randn_bf16(gen, (1, 8, n, 128)).cuda(), randn_bf16(gen, (1, 8, n, 128)).cuda()
        eager.import_(s, 0, k, v)
        graphed.import_(s, 0, k, v)
    scale = 1.0 / math.sqrt(128)
    qb = torch.zeros((3, 16, 1, 128), dtype=torch.bfloat16, device="cuda")
    kb, vb = torch.zeros((3, 8, 1, 128), dtype=torch.bfloat16, device="cuda"), torch.zeros(
        (3, 8, 1, 128), dtype=torch.bfloat16, device="cuda")
    ob = torch.empty_like(qb)
    for s in slots:
        graphed.reserve(s, 21)  # the eager step below and 20 replays
    graphed.append_attend(0, qb, kb, vb, slots, scale, out=ob)  # eager: workspace sized, context bound
    eager.append_attend(0, qb, kb, vb, slots, scale)
    graphed.synchronize()
    eager.synchronize()  # both move to the capture stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            graphed.append_attend(0, qb, kb, vb, slots, scale, out=ob)
        graphed.sync_lengths()
        pages = graphed.counters()["pages_in_use"]
        for r in range(20):
            q = randn_bf16(gen, (3, 16, 1, 128), 0.5).cuda()
            k, v = randn_bf16(gen, (3, 8, 1, 128)).cuda(), randn_bf16(gen, (3, 8, 1, 128)).cuda()
            qb.copy_(q)
            kb.copy_(k)
            vb.copy_(v)
            g.replay()
            ref = eager.append_attend(0, q, k, v, slots, scale)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(bits(ob), bits(ref), err_msg=f"replay {r}")
        graphed.sync_lengths()
        assert [graphed.seq_length(s, 0) for s in slots] == [n + 21 for n in lens]
        assert graphed.counters()["pages_in_use"] == pages  # every page came from the reservation
        for s in slots:
            ka, va, _ = graphed.gather(0, [s])
            kr, vr, _ = eager.gather(0, [s])
            torch.cuda.synchronize()
            np.testing.assert_array_equal(_raw(ka), _raw(kr))
            np.testing.assert_array_equal(_raw(va), _raw(vr))
        assert graphed.health() == 0
        # past the reservation (whole pages: slot 3 is at 58 with pages to
        # position 64, slot 0 at 151 with pages to 160): 10 more replays land
        # rows on unmapped pages
        for _ in range(10):
            g.replay()
        assert graphed.health() == -6
    assert eager.health() == 0
