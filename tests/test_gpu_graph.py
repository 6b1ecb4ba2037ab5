"""HIP graph capture of fused append+attend steps: every replay must equal the
eager path bit for bit, and replays must advance the device lengths."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import bits, randn_bf16

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


@pytest.mark.parametrize("merge", ["auto", "separate", "last_wg"])
def test_graph_replays_match_eager_bitwise(merge):
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
    a, b = _pair(specs, n, 1500, gen, prefill=1100, merge=merge)
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
    torch.cuda.synchronize()
    for l in range(len(specs)):
        np.testing.assert_array_equal(bits(static_out[l]), bits(eager[0][l]))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    b.sync_lengths()
    assert b.seq_length(0, 0) == 1101
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
            assert b.seq_length(s, l) == a.seq_length(s, l) == 1100 + steps
        ka, va, _ = a.gather(l, slots)
        kb, vb, _ = b.gather(l, slots)
        np.testing.assert_array_equal(bits(ka), bits(kb))
        np.testing.assert_array_equal(bits(va), bits(vb))
    assert a.health() == 0 and b.health() == 0


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
    out_a = torch.empty_like(q)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        a.attend_prefill(0, q, [0, 1], 1 / 22.627, out=out_a)
    out_b = torch.empty_like(q)
    gb = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gb):
        b.attend_prefill(0, q, [0, 1], 1 / 22.627, out=out_b)
    for _ in range(3):
        a.gather(0, [0])  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        gb.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(out_a), bits(eager))
        assert float((out_b.float() - eager.float()).abs().max()) <= 1e-2
    assert a.health() == 0 and b.health() == 0
