"""GPU parity of the chunked-prefill MFMA attention (kvrt_attend_prefill_async)
against the fp64 oracle: Gemma sliding layers at the reference's canonical
prefill length (Q = 291 with a 512 window, ring of 802 rows), Gemma full
layers (D = 512), talker prefill (16 q / 8 kv heads), Q3..Q8 text appends, paged
storage and ragged streams. Tolerance max-abs 1e-2 on bf16 outputs."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2


def _setup(hq, hkv, d, window, layout, prefix_lens, qn, seed):
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(seed)
    kw = {}
    if layout == "ring":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="ring", window=window, ring_rows=window + qn - 1)
    elif layout == "paged":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="paged", window=window)
        kw = dict(block_size=16, pool_pages=512)
    else:
        spec = LayerSpec(kv_heads=hkv, head_dim=d, window=window)
    n = len(prefix_lens)
    rt = KVRuntime([spec], n, max(prefix_lens) + qn + 8, max_q=qn, device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(hkv, d, window)], n)
    for s, p in enumerate(prefix_lens):
        if p:
            k, v = randn_bf16(gen, (1, hkv, p, d)), randn_bf16(gen, (1, hkv, p, d))
            rt.import_(s, 0, k.cuda(), v.cuda())
            orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    # the chunk's own K/V rows go in first (prefill-length append), then attention
    k, v = randn_bf16(gen, (n, hkv, qn, d)), randn_bf16(gen, (n, hkv, qn, d))
    rt.append(0, k.cuda(), v.cuda(), list(range(n)))
    for s in range(n):
        orc.append(s, 0, to_np(k[s]), to_np(v[s]))
    q = randn_bf16(gen, (n, hq, qn, d), 0.5)
    return rt, orc, q


def _check(rt, orc, q, scale, prefill=True):
    n = q.shape[0]
    fn = rt.attend_prefill if prefill else rt.attend
    out = fn(0, q.cuda(), list(range(n)), scale)
    torch.cuda.synchronize()
    assert rt.health() == 0
    worst = 0.0
    for s in range(n):
        ref = orc.attend(s, 0, to_np(q[s]), scale)
        worst = max(worst, float(np.abs(to_np(out[s]) - ref).max()))
    assert worst <= ATOL, worst
    return out


@pytest.mark.parametrize(
    "hq,hkv,d,window,layout,prefix,qn",
    [
        (8, 1, 256, 512, "ring", [0], 291),          # Gemma sliding, canonical prefill target
        (8, 1, 256, 512, "ring", [700], 291),        # ... over a ring that has wrapped
        (8, 1, 512, 0, "contig", [0, 130], 291),     # Gemma full layers, D = 512
        (16, 8, 128, 0, "contig", [37, 0, 400], 100),  # talker prefill, ragged prefixes
        (8, 1, 256, 512, "ring", [1500, 20], 8),     # Q8 text append (64 rows per kv head)
        (8, 1, 256, 0, "contig", [300], 3),          # Q3 text append
        (4, 4, 64, 0, "paged", [45, 300], 37),       # paged pool
        (4, 2, 128, 24, "paged", [200], 50),         # paged + window
        # few query blocks over many keys: the keys of a block are split over
        # workgroups and the partials merged (8 and 2 key ranges)
        (8, 1, 512, 0, "contig", [2000, 900], 64),
        (4, 2, 128, 600, "paged", [1500], 40),
        # the talker's whole-response prefill: a grid of 1024 workgroups, one
        # wave per head (LDS DMA ring, two waves per workgroup)
        (16, 8, 128, 0, "contig", [0, 0, 0, 0], 512),
        # LDS DMA ring over a wrapped ring layout, two waves per head
        (8, 2, 128, 200, "ring", [900, 64], 77),
        # talker-sized grids (>= 512 workgroups, DMA ring): an odd block count
        # over ragged prefixes, and a windowed ring layout
        (16, 8, 128, 0, "contig", [0, 37, 300, 5], 481),
        (16, 8, 128, 200, "ring", [0, 900, 64, 10], 300),
        # GQA groups of 6 and 3 (3 q heads per workgroup: the index splits
        # by a divisor that is not a power of two)
        (6, 1, 128, 0, "contig", [100, 37], 50),
        (12, 2, 256, 512, "ring", [300], 40),
        (3, 1, 64, 0, "paged", [70], 33),
        # a key split (one long stream) leaves the short streams' later key
        # ranges empty: their clamped fetches must stay on mapped pages (the
        # health check below would report the device flag otherwise)
        (12, 4, 128, 0, "paged", [31, 839, 241], 1),
        (8, 2, 64, 0, "paged", [5, 1500], 3),
    ],
)
def test_prefill_matches_oracle(hq, hkv, d, window, layout, prefix, qn):
    rt, orc, q = _setup(hq, hkv, d, window, layout, prefix, qn, seed=hq * 7 + d + qn)
    _check(rt, orc, q, 1.0 / math.sqrt(d))


def test_prefill_single_query_and_decode_dispatch():
    """Q = 1 through the MFMA kernel; g * Q above 16 rows dispatches to it from attend()."""
    rt, orc, q = _setup(2, 1, 128, 0, "contig", [77], 1, seed=5)
    _check(rt, orc, q, 0.1)
    rt, orc, q = _setup(8, 1, 256, 512, "ring", [900], 4, seed=6)  # 32 rows per kv head
    _check(rt, orc, q, 1.0 / 16, prefill=False)


def test_prefill_and_decode_agree_where_both_apply():
    rt, orc, q = _setup(4, 2, 128, 0, "contig", [500, 123], 4, seed=7)
    a = rt.attend_prefill(0, q.cuda(), [0, 1], 0.09)
    b = rt.attend(0, q.cuda(), [0, 1], 0.09)  # 8 rows per kv head: decode kernel
    torch.cuda.synchronize()
    assert float((a.float() - b.float()).abs().max()) <= ATOL


def test_prefill_rejects_what_it_cannot_see():
    from kvrt import KVRTError, KVRuntime, LayerSpec

    rt = KVRuntime([LayerSpec(kv_heads=1, head_dim=256, layout="ring", window=64, ring_rows=64 + 8 - 1)], 1, 4096,
                   max_q=8, device="cuda")
    x = torch.zeros((1, 1, 1000, 256), dtype=torch.bfloat16, device="cuda")
    rt.import_(0, 0, x, x)
    q = torch.zeros((1, 8, 16, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(KVRTError) as e:  # 16 queries need 16 + 63 resident rows, the ring keeps 71
        rt.attend_prefill(0, q, [0], 0.1)
    assert e.value.code == -2
    q = torch.zeros((1, 8, 1001, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(KVRTError):  # more queries than positions
        rt.attend_prefill(0, q, [0], 0.1)
    assert rt.health() == 0


@pytest.mark.parametrize("logical_q", [3, 5, 7])
def test_even_physical_q_with_pad_row_truncation_equals_the_logical_q(logical_q):
    """The reference's variable-Q text step runs an even physical Q (logical
    + 1 pad row for odd logical Q), then truncates the cursor to the logical
    end (gemma4_listener_microbatch_impl.inc:3476-3586,
    native_listener_microbatch.py:1640-1655). kvrt takes any Q directly; both
    routes must give the same logical rows, cache and next decode."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(logical_q)
    hq, hkv, d = 8, 1, 256
    prefix = randn_bf16(gen, (1, hkv, 300, d))
    k = randn_bf16(gen, (1, hkv, logical_q + 1, d))
    v = randn_bf16(gen, (1, hkv, logical_q + 1, d))
    q = randn_bf16(gen, (1, hq, logical_q + 1, d), 0.5)
    outs, rts = [], []
    for physical in (logical_q, logical_q + 1):
        rt = KVRuntime([LayerSpec(kv_heads=hkv, head_dim=d, window=512)], 1, 512, max_q=8, device="cuda")
        rt.import_(0, 0, prefix.cuda(), prefix.cuda())
        rt.append(0, k[:, :, :physical].contiguous().cuda(), v[:, :, :physical].contiguous().cuda(), [0])
        outs.append(rt.attend_prefill(0, q[:, :, :physical].contiguous().cuda(), [0], 1 / 16))
        rt.truncate(0, 300 + logical_q)
        rts.append(rt)
    torch.cuda.synchronize()
    direct, padded = outs
    assert float((direct.float() - padded[:, :, :logical_q].float()).abs().max()) <= 1e-6
    assert rts[0].seq_length(0) == rts[1].seq_length(0) == 300 + logical_q
    qd = randn_bf16(gen, (1, hq, 1, d), 0.5).cuda()
    kd = randn_bf16(gen, (1, hkv, 1, d)).cuda()
    a = rts[0].append_attend(0, qd, kd, kd, [0], 1 / 16)
    b = rts[1].append_attend(0, qd, kd, kd, [0], 1 / 16)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert rts[0].health() == 0 and rts[1].health() == 0


# the prefill benchmark's cases: name, streams, Hq, Hkv, D, Q, prefix, window
BENCH_SHAPES = [
    ("thinker_sliding_q291", 4, 8, 1, 256, 291, 2048, 512),
    ("thinker_full_d512_q291", 4, 8, 1, 512, 291, 2048, 0),
    ("talker_prefill_q512", 4, 16, 8, 128, 512, 0, 0),
    ("thinker_prefill_q2048", 1, 8, 1, 256, 2048, 0, 0),
    ("thinker_full_d512_q2048", 4, 8, 1, 512, 2048, 2048, 0),
]


@pytest.mark.parametrize("name,n,hq,hkv,d,qn,prefix,window", BENCH_SHAPES, ids=[c[0] for c in BENCH_SHAPES])
def test_prefill_at_the_benchmark_shapes_on_sampled_rows(name, n, hq, hkv, d, qn, prefix, window):
    """The full-size chunks the prefill benchmark times (key-split grids,
    query-block pairs, the D 512 path, a wrapped ring): every q head of 12
    query rows per stream (the first, the last and 10 seeded others) against
    the oracle, which attends those rows only."""
    import random

    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(qn + d + prefix)
    layout = "ring" if window else "contig"
    spec = LayerSpec(kv_heads=hkv, head_dim=d, layout=layout, window=window,
                     ring_rows=window + qn - 1 if window else 0)
    L = prefix + qn
    rt = KVRuntime([spec], n, L + 8, max_q=qn, device="cuda")
    ks, vs = [], []
    for s in range(n):
        k, v = randn_bf16(gen, (1, hkv, L, d)), randn_bf16(gen, (1, hkv, L, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        ks.append(to_np(k[0]))
        vs.append(to_np(v[0]))
    q = randn_bf16(gen, (n, hq, qn, d), 0.5)
    scale = 1.0 / math.sqrt(d)
    out = rt.attend_prefill(0, q.cuda(), list(range(n)), scale)
    torch.cuda.synchronize()
    assert rt.health() == 0
    r = random.Random(qn * 7 + d)
    worst = 0.0
    for s in range(n):
        rows = sorted({0, qn - 1, *r.sample(range(qn), min(qn, 10))})
        ref = O.attend(to_np(q[s])[:, rows], ks[s], vs[s], np.array([L - qn + i for i in rows]), scale, window)
        worst = max(worst, float(np.abs(to_np(out[s])[:, rows] - ref).max()))
    assert worst <= ATOL, worst
