"""HIP graph replays of fused append + decode steps over seeded random layer
stacks (CONTIG / RING / PAGED bf16 and int8 layers, head_dim 64 / 128 / 256,
GQA groups 1..8, Q 1 / 2, 1..4 ragged streams, every decode kernel and merge
mode), with rollbacks between replays: one step is captured, replayed with
fresh inputs copied in, and after every few replays the host reads the
device lengths back (kvrt_sync_lengths), rolls a stream back by 0..2
positions (kvrt_truncate, PAGED slots reserving their pages again) and
replays on. Every replay's outputs are checked against the oracle (max-abs
1e-2), the device lengths against the replay count, and the stored rows bit
for bit at the end."""
from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2


def _cases(n_cases: int, seed: int) -> list[tuple]:
    r = random.Random(seed)
    out = []
    while len(out) < n_cases:
        qn = r.choice([1, 2])
        layers = []
        for _ in range(r.choice([1, 2, 3])):
            d = r.choice([64, 128, 256])
            layout = r.choice(["contig", "ring", "paged"])
            dtype = "int8" if layout == "paged" and r.random() < 0.4 else "bf16"
            hkv, g = r.choice([1, 2, 8]), r.choice([1, 2, 4, 8])
            if g * qn > (8 if dtype == "int8" else 16):
                g = 1
            window = r.choice([64, 200]) if layout == "ring" else r.choice([0, 0, 300])
            layers.append((d, layout, dtype, hkv, g, window))
        lens = tuple(r.randint(1, 3000) for _ in range(r.choice([1, 2, 3, 4])))
        kernel, merge = r.choice(["auto", "valu", "mfma"]), r.choice(["auto", "separate", "last_wg"])
        out.append((qn, tuple(layers), lens, kernel, merge, r.randrange(1 << 30)))
    return out


CASES = _cases(16, 4242)


@pytest.mark.parametrize("case", CASES, ids=[
    f"q{c[0]}-" + "+".join(f"{l[1]}{l[0]}{'i8' if l[2] == 'int8' else ''}h{l[3]}g{l[4]}" for l in c[1])
    + f"-n{len(c[2])}-{c[3]}-{c[4]}" for c in CASES])
def test_random_graph_replays_with_rollbacks_match_oracle(case):
    from kvrt import KVRuntime, LayerSpec

    qn, layers, lens, kernel, merge, seed = case
    r = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    n, replays, slack = len(lens), 12, 2
    cap = max(lens) + (replays + 2) * qn + 8
    specs = []
    for d, layout, dtype, hkv, g, window in layers:
        rows = window + qn - 1 + slack if layout == "ring" else 0
        specs.append(LayerSpec(kv_heads=hkv, head_dim=d, layout=layout, dtype=dtype, window=window, ring_rows=rows))
    paged = any(s.layout == "paged" for s in specs)
    kw = dict(block_size=16, pool_pages=len(specs) * n * (cap // 16 + 2) + 8, pool_seed=7) if paged else {}
    rt = KVRuntime(specs, n, cap, max_q=qn, decode_kernel=kernel, decode_merge=merge, device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(s.kv_heads, s.head_dim, s.window, s.dtype == "int8") for s in specs], n)
    for layer, s in enumerate(specs):
        for i, length in enumerate(lens):
            k, v = randn_bf16(gen, (1, s.kv_heads, length, s.head_dim)), randn_bf16(gen, (1, s.kv_heads, length, s.head_dim))
            rt.import_(i, layer, k.cuda(), v.cuda())
            orc.append(i, layer, to_np(k[0]), to_np(v[0]))
    slots = list(range(n))
    hq = [s.kv_heads * l[4] for s, l in zip(specs, layers)]
    scale = [1.0 / math.sqrt(s.head_dim) for s in specs]
    bufs = [(torch.empty((n, hq[l], qn, s.head_dim), dtype=torch.bfloat16, device="cuda"),
             torch.empty((n, s.kv_heads, qn, s.head_dim), dtype=torch.bfloat16, device="cuda"),
             torch.empty((n, s.kv_heads, qn, s.head_dim), dtype=torch.bfloat16, device="cuda"),
             torch.empty((n, hq[l], qn, s.head_dim), dtype=torch.bfloat16, device="cuda")) for l, s in enumerate(specs)]

    def draw():
        host = []
        for l, s in enumerate(specs):
            q = randn_bf16(gen, (n, hq[l], qn, s.head_dim), 0.5)
            k, v = randn_bf16(gen, (n, s.kv_heads, qn, s.head_dim)), randn_bf16(gen, (n, s.kv_heads, qn, s.head_dim))
            for dst, src in zip(bufs[l][:3], (q, k, v)):
                dst.copy_(src)
            host.append((q, k, v))
        return host

    def step():
        for l in range(len(specs)):
            q, k, v, o = bufs[l]
            rt.append_attend(l, q, k, v, slots, scale[l], out=o)

    def check(host, where):
        torch.cuda.synchronize()
        for l in range(len(specs)):
            q, k, v = host[l]
            out = to_np(bufs[l][3])
            for i in slots:
                orc.append(i, l, to_np(k[i]), to_np(v[i]))
                err = float(np.abs(out[i] - orc.attend(i, l, to_np(q[i]), scale[l])).max())
                assert err <= ATOL, (where, l, i, err)

    def reserve():
        if paged:
            for i in slots:
                rt.reserve(i, cap - rt.seq_length(i, 0))

    check_host = draw()
    step()  # eager step: sizes the workspace
    check(check_host, "eager")
    reserve()  # the captured step then maps no page itself
    rt.synchronize()  # the capture runs on another stream: nothing of the context's may be in flight
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    rt.sync_lengths()
    for t in range(replays):
        host = draw()
        g.replay()
        check(host, f"replay {t}")
        if t % 4 == 3:
            rt.sync_lengths()
            for l in range(len(specs)):
                for i in slots:
                    assert rt.seq_length(i, l) == orc.length(i, l), (t, l, i)
            i = r.randrange(n)
            back = r.randint(0, 2)
            new_len = orc.length(i, 0) - back
            rt.truncate(i, new_len)
            for l in range(len(specs)):
                orc.truncate(i, l, new_len)
            reserve()
    assert rt.health() == 0
    rt.sync_lengths()
    for l, s in enumerate(specs):
        for i in slots:
            L = orc.length(i, l)
            assert rt.seq_length(i, l) == L
            start = max(0, L - s.window + 1) if s.window > 0 else 0
            k, v, _ = rt.gather(l, [i], start_pos=[start], mask_dtype=None)
            torch.cuda.synchronize()
            ok_, ov = orc.values(i, l)
            if k.dtype == torch.bfloat16:
                assert np.array_equal(bits(k[0]), O.f32_to_bf16_bits(ok_[:, start:])), (l, i)
                assert np.array_equal(bits(v[0]), O.f32_to_bf16_bits(ov[:, start:])), (l, i)
            else:
                assert np.array_equal(to_np(k[0]), ok_[:, start:]) and np.array_equal(to_np(v[0]), ov[:, start:])
