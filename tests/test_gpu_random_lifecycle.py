"""GPU parity of seeded random slot lifecycles against the oracle: fused
decode steps (Q 1 / 2) on a CONTIG or PAGED (bf16 / int8) layer and a RING
layer, rollbacks (kvrt_truncate), clones (kvrt_copy_prefix_async), releases
and re-imports, in random order over three slots. Every accepted operation
must leave attention equal to the oracle's (max-abs 1e-2) and stored rows
equal bit for bit; a rollback or clone is refused exactly when the RING
layer no longer holds a key the next query sees (a row that a later
position overwrote since the slot was last empty)."""
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
    for _ in range(n_cases):
        d = r.choice([64, 128])
        hkv, g = r.choice([1, 2]), r.choice([1, 2, 4])
        first = r.choice(["contig", "paged", "paged"])
        dtype = "int8" if first == "paged" and r.random() < 0.5 else "bf16"
        window = r.choice([16, 48])
        slack = r.choice([0, 3, 20])
        out.append((d, hkv, g, first, dtype, window, slack, r.randrange(1 << 30)))
    return out


CASES = _cases(12, 97)


@pytest.mark.parametrize("case", CASES, ids=[f"d{c[0]}-h{c[1]}g{c[2]}-{c[3]}-{c[4]}-w{c[5]}s{c[6]}" for c in CASES])
def test_random_lifecycle_matches_oracle(case):
    from kvrt import KVRTError, KVRuntime, LayerSpec

    d, hkv, g, first, dtype, window, slack, seed = case
    r = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    n_slots, cap, max_q = 3, 400, 2
    rows = window + max_q - 1 + slack
    specs = [LayerSpec(kv_heads=hkv, head_dim=d, layout=first, dtype=dtype, window=r.choice([0, 64])),
             LayerSpec(kv_heads=hkv, head_dim=d, layout="ring", window=window, ring_rows=rows)]
    kw = dict(block_size=16, pool_pages=4 * n_slots * (cap // 16 + 2), pool_seed=3) if first == "paged" else {}
    rt = KVRuntime(specs, n_slots, cap, max_q=max_q, device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(hkv, d, specs[0].window, dtype == "int8"), O.OracleLayer(hkv, d, window)],
                        n_slots)
    scale = 1.0 / math.sqrt(d)
    # per slot: the longest the RING layer has been since the slot was last
    # empty; rows below high - rows have been overwritten
    high = [0] * n_slots

    def length(s):
        return orc.length(s, 0)

    def visible_floor(t):
        return max(0, t - window + 1)

    def import_fresh(s, n):
        for layer in range(2):
            k, v = randn_bf16(gen, (1, hkv, n, d)), randn_bf16(gen, (1, hkv, n, d))
            rt.import_(s, layer, k.cuda(), v.cuda())
            orc.append(s, layer, to_np(k[0]), to_np(v[0]))
        high[s] = n

    for s in range(n_slots):
        import_fresh(s, r.randint(1, 150))
    accepted = refused = steps = 0
    for op_i in range(36):
        op = r.choice(["step", "step", "step", "rollback", "rollback", "clone", "renew"])
        where = (op_i, op)
        if op == "step":
            qn = r.choice([1, 2])
            slots = sorted(r.sample(range(n_slots), r.randint(1, n_slots)))
            slots = [s for s in slots if length(s) + qn <= cap]
            if not slots:
                continue
            n = len(slots)
            q = randn_bf16(gen, (n, hkv * g, qn, d), 0.5)
            for layer in range(2):
                k, v = randn_bf16(gen, (n, hkv, qn, d)), randn_bf16(gen, (n, hkv, qn, d))
                out = rt.append_attend(layer, q.cuda(), k.cuda(), v.cuda(), slots, scale)
                torch.cuda.synchronize()
                for i, s in enumerate(slots):
                    orc.append(s, layer, to_np(k[i]), to_np(v[i]))
                    ref = orc.attend(s, layer, to_np(q[i]), scale)
                    err = float(np.abs(to_np(out[i]) - ref).max())
                    assert err <= ATOL, (where, layer, s, err)
            for s in slots:
                high[s] = max(high[s], length(s))
            steps += 1
        elif op == "rollback":
            s = r.randrange(n_slots)
            L = length(s)
            t = r.choice([0, max(0, L - r.randint(0, 3)), max(0, L - r.randint(0, rows + 4))])
            ok = t == 0 or visible_floor(t) >= max(0, high[s] - rows)
            if ok:
                rt.truncate(s, t)
                for layer in range(2):
                    orc.truncate(s, layer, t)
                if t == 0:
                    high[s] = 0
                accepted += 1
            else:
                with pytest.raises(KVRTError) as e:
                    rt.truncate(s, t)
                assert e.value.code == -2, where
                refused += 1
            assert rt.seq_length(s, 0) == rt.seq_length(s, 1) == length(s), where
        elif op == "clone":
            src, dst = r.sample(range(n_slots), 2)
            L = length(src)
            n = r.choice([0, L, max(0, L - r.randint(0, rows + 4)), r.randint(0, L)])
            ok = n == 0 or max(0, n - rows, high[src] - rows) <= visible_floor(n)
            if ok:
                rt.copy_prefix(src, dst, n)
                for layer in range(2):
                    orc.copy_prefix(src, dst, layer, n)
                high[dst] = max(n, high[src]) if n else 0
                accepted += 1
            else:
                with pytest.raises(KVRTError) as e:
                    rt.copy_prefix(src, dst, n)
                assert e.value.code == -2, where
                refused += 1
            assert rt.seq_length(dst, 1) == length(dst), where
        else:  # release, then a new session in the slot
            s = r.randrange(n_slots)
            rt.truncate(s, 0)
            for layer in range(2):
                orc.truncate(s, layer, 0)
            import_fresh(s, r.randint(0, 200))
        assert rt.health() == 0, where
    assert steps and accepted, (steps, accepted, refused)
    # stored rows, bit for bit: all of layer 0, the ring's next window
    torch.cuda.synchronize()
    for s in range(n_slots):
        L = length(s)
        if L == 0:
            continue
        for layer, start in ((0, 0), (1, visible_floor(L))):
            k, v, _ = rt.gather(layer, [s], start_pos=[start], mask_dtype=None)
            torch.cuda.synchronize()
            ok_, ov = orc.values(s, layer)
            if k.dtype == torch.bfloat16:
                assert np.array_equal(bits(k[0]), O.f32_to_bf16_bits(ok_[:, start:])), (s, layer)
                assert np.array_equal(bits(v[0]), O.f32_to_bf16_bits(ov[:, start:])), (s, layer)
            else:
                assert np.array_equal(to_np(k[0]), ok_[:, start:]) and np.array_equal(to_np(v[0]), ov[:, start:])
