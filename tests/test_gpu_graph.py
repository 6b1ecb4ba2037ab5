"""HIP graph capture of fused append+attend steps: every replay must equal the
eager path bit for bit, and replays must advance the device lengths."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu


def _pair(specs, n_slots, capacity, gen, prefill, merge="auto"):
    from kvrt import KVRuntime

    a = KVRuntime(specs, n_slots, capacity, max_q=1, decode_merge=merge, device="cuda")
    b = KVRuntime(specs, n_slots, capacity, max_q=1, decode_merge=merge, device="cuda")
    for layer, spec in enumerate(specs):
        for s in range(n_slots):
            k = randn_bf16(gen, (1, spec.kv_heads, prefill, spec.head_dim)).cuda()
            v = randn_bf16(gen, (1, spec.kv_heads, prefill, spec.head_dim)).cuda()
            a.import_(s, layer, k, v)
            b.import_(s, layer, k, v)
    torch.cuda.synchronize()
    return a, b


@pytest.mark.parametrize("prefill", [1100, 2500])
@pytest.mark.parametrize("merge", ["auto", "separate", "last_wg"])
def test_graph_replays_match_eager_bitwise(merge, prefill):
    """At 1100 positions the talker- and thinker-global-shaped layers run on
    the VALU decode, at 2500 on the MFMA decode's LDS DMA ring."""
    from kvrt import LayerSpec

    gen = torch.Generator().manual_seed(21)
    specs = [
        LayerSpec(kv_heads=8, head_dim=128),                                    # talker-shaped
        LayerSpec(kv_heads=1, head_dim=256, layout="ring", window=64, ring_rows=64),  # thinker sliding
        LayerSpec(kv_heads=1, head_dim=256),                                    # thinker global
    ]
    hq = [16, 8, 8]
    n = 3
    steps = 6
    a, b = _pair(specs, n, prefill + 400, gen, prefill=prefill, merge=merge)
    inputs = [[(randn_bf16(gen, (n, hq[l], 1, s.head_dim), 0.5).cuda(),
                randn_bf16(gen, (n, s.kv_heads, 1, s.head_dim), 0.5).cuda(),
                randn_bf16(gen, (n, s.kv_heads, 1, s.head_dim), 0.5).cuda()) for l, s in enumerate(specs)]
              for _ in range(steps)]
    slots = [0, 1, 2]
    eager = []
    for t in range(steps):
        eager.append([a.append_attend(l, *inputs[t][l], slots, 0.07) for l in range(len(specs))])
    torch.cuda.synchronize()

    static_in = [tuple(x.clone() for x in inputs[0][l]) for l in range(len(specs))]
    static_out = [torch.empty_like(static_in[l][0]) for l in range(len(specs))]

    def step():
        for l in range(len(specs)):
            b.append_attend(l, *static_in[l], slots, 0.07, out=static_out[l])

    step()  # eager step 0: sizes the workspace
    b.synchronize()  # the capture runs on another stream: nothing of b's may be in flight
    for l in range(len(specs)):
        np.testing.assert_array_equal(bits(static_out[l]), bits(eager[0][l]))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    b.sync_lengths()
    assert b.seq_length(0, 0) == prefill + 1
    for t in range(1, steps):
        for l in range(len(specs)):
            for dst, src in zip(static_in[l], inputs[t][l]):
                dst.copy_(src)
        b.gather(0, [0])  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for l in range(len(specs)):
            np.testing.assert_array_equal(bits(static_out[l]), bits(eager[t][l]), err_msg=f"replay {t} layer {l}")
    b.sync_lengths()
    for l in range(len(specs)):
        for s in slots:
            assert b.seq_length(s, l) == a.seq_length(s, l) == prefill + steps
        ka, va, _ = a.gather(l, slots)
        kb, vb, _ = b.gather(l, slots)
        np.testing.assert_array_equal(bits(ka), bits(kb))
        np.testing.assert_array_equal(bits(va), bits(vb))
    assert a.health() == 0 and b.health() == 0
    mfma = b.counters()["mfma_decodes"]
    assert (mfma > 0) == (prefill >= 2048), mfma


def test_graph_replays_of_a_key_split_prefill_match_eager():
    """A prefill whose query blocks are few over many keys runs as key ranges
    plus a merge kernel. Captured after an eager call has sized the workspace,
    its replays equal the eager result bit for bit; captured on a fresh context
    it splits only if the workspace sized at create holds the ranges' partials
    (nothing is allocated inside a capture), and either way stays within the
    attention tolerance of the eager result."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(31)
    spec = LayerSpec(kv_heads=1, head_dim=512)
    rts = [KVRuntime([spec], 2, 2200, max_q=64, device="cuda") for _ in range(2)]
    for s, p in enumerate((2000, 1200)):
        k = randn_bf16(gen, (1, 1, p, 512)).cuda()
        v = randn_bf16(gen, (1, 1, p, 512)).cuda()
        for rt in rts:
            rt.import_(s, 0, k, v)
    q = randn_bf16(gen, (2, 8, 64, 512), 0.5).cuda()
    k = randn_bf16(gen, (2, 1, 64, 512)).cuda()
    for rt in rts:
        rt.append(0, k, k, [0, 1])
    torch.cuda.synchronize()
    a, b = rts
    eager = a.attend_prefill(0, q, [0, 1], 1 / 22.627)
    # captures run on a stream of their own: each context is synchronised
    # before it moves there and after it leaves
    a.synchronize()
    b.synchronize()
    out_a = torch.empty_like(q)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        a.attend_prefill(0, q, [0, 1], 1 / 22.627, out=out_a)
    out_b = torch.empty_like(q)
    gb = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gb):
        b.attend_prefill(0, q, [0, 1], 1 / 22.627, out=out_b)
    a.synchronize()
    b.synchronize()
    for _ in range(3):
        a.gather(0, [0])  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        gb.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(out_a), bits(eager))
        assert float((out_b.float() - eager.float()).abs().max()) <= 1e-2
    assert a.health() == 0 and b.health() == 0


def test_graph_replays_over_a_whole_talker_response():
    """The reference replays its talker Q1 graph across a whole response
    (native_qwen_talker.py:1103-1151). Here a step of the 28-layer talker
    (4 sessions, Hq 16 / Hkv 8, D 128), a thinker-global-shaped layer (Hq 8 /
    Hkv 1, D 256) and a one-head D 128 layer is captured once at 1900 keys
    and replayed 300 times with fresh inputs copied in before each replay.
    The replays cross three 128-key split buckets, the 2048-key point where
    AUTO would move the 8-row layer to the MFMA kernel, and the one where the
    one-head layer's partials outgrow the single-launch merge; the captured
    split count, kernel and merge stay, and every 25th replay is checked
    against the oracle at 1e-2 (the reduction order differs from an eager
    call at the new length, so the check is not bitwise)."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(300)
    n, start, steps = 4, 1900, 300
    talker = KVRuntime([LayerSpec(kv_heads=8, head_dim=128)] * 28, n, start + steps + 8, max_q=1, decode_wgs=192,
                       device="cuda")
    other_specs = [LayerSpec(kv_heads=1, head_dim=256), LayerSpec(kv_heads=1, head_dim=128)]
    other = KVRuntime(other_specs, n, start + steps + 8, max_q=1, decode_wgs=192, device="cuda")
    models = [(talker, [(16, 8, 128)] * 28), (other, [(8, 1, 256), (2, 1, 128)])]
    orcs = []
    for rt, shapes in models:
        orc = O.OracleCache([O.OracleLayer(hkv, d) for _, hkv, d in shapes], n)
        for layer, (_, hkv, d) in enumerate(shapes):
            for s in range(n):
                k, v = randn_bf16(gen, (1, hkv, start, d)), randn_bf16(gen, (1, hkv, start, d))
                rt.import_(s, layer, k.cuda(), v.cuda())
                orc.append(s, layer, to_np(k[0]), to_np(v[0]))
        orcs.append(orc)
    slots = list(range(n))
    bufs = [[(torch.empty((n, hq, 1, d), dtype=torch.bfloat16, device="cuda"),
              torch.empty((n, hkv, 1, d), dtype=torch.bfloat16, device="cuda"),
              torch.empty((n, hkv, 1, d), dtype=torch.bfloat16, device="cuda"),
              torch.empty((n, hq, 1, d), dtype=torch.bfloat16, device="cuda")) for hq, hkv, d in shapes]
            for _, shapes in models]

    def draw():
        host = [[(randn_bf16(gen, (n, hq, 1, d), 0.3), randn_bf16(gen, (n, hkv, 1, d)), randn_bf16(gen, (n, hkv, 1, d)))
                 for hq, hkv, d in shapes] for _, shapes in models]
        for m, layers in enumerate(host):
            for layer, (q, k, v) in enumerate(layers):
                for dst, src in zip(bufs[m][layer][:3], (q, k, v)):
                    dst.copy_(src)
        return host

    def step():
        for m, (rt, shapes) in enumerate(models):
            for layer in range(len(shapes)):
                q, k, v, o = bufs[m][layer]
                rt.append_attend(layer, q, k, v, slots, 0.09, out=o)

    def check(host):
        worst = 0.0
        for m, (rt, shapes) in enumerate(models):
            for layer in range(len(shapes)):
                out = to_np(bufs[m][layer][3])
                q = host[m][layer][0]
                for i in slots:
                    worst = max(worst, float(np.abs(out[i] - orcs[m].attend(i, layer, to_np(q[i]), 0.09)).max()))
        return worst

    def record(host):
        for m, (rt, shapes) in enumerate(models):
            for layer in range(len(shapes)):
                _, k, v = host[m][layer]
                for i in slots:
                    orcs[m].append(i, layer, to_np(k[i]), to_np(v[i]))

    host = draw()
    step()  # eager step: sizes the workspaces
    record(host)
    torch.cuda.synchronize()
    assert check(host) <= 1e-2
    for rt, _ in models:
        rt.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for rt, _ in models:
        rt.sync_lengths()
    checked = 0
    for t in range(1, steps):
        host = draw()
        g.replay()
        record(host)
        if t % 25 == 0 or t == steps - 1:
            torch.cuda.synchronize()
            worst = check(host)
            assert worst <= 1e-2, f"replay {t} at {start + t + 1} keys: max-abs {worst:.3g}"
            checked += 1
    torch.cuda.synchronize()
    for rt, shapes in models:
        rt.sync_lengths()
        for layer in range(len(shapes)):
            assert rt.seq_length(0, layer) == start + steps
        assert rt.health() == 0
    assert checked >= 12
