"""GPU parity of seeded random slot lifecycles against the oracle: fused
decode steps (Q 1 / 2) on a CONTIG or PAGED (bf16 / int8) layer, a RING
layer and a layer sharing the first one's rows, with rollbacks
(kvrt_truncate), clones (kvrt_copy_prefix_async), page evictions
(kvrt_evict), prefix-attention masks, releases and re-imports in random order
over three slots. Every accepted operation must leave attention equal to the
oracle's (max-abs 1e-2) and stored rows equal bit for bit. A rollback or
clone must be refused (KVRT_ESTATE, nothing changed) exactly when it would
end inside the slot's prefix mask or when a key the next query sees is no
longer stored: a RING row that a later position overwrote since the slot was
last empty, or a PAGED row on a page kvrt_evict released."""
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
BS = 16  # page size


def _cases(n_cases: int, seed: int) -> list[tuple]:
    r = random.Random(seed)
    out = []
    for _ in range(n_cases):
        d = r.choice([64, 128])
        hkv, g = r.choice([1, 2]), r.choice([1, 2, 4])
        first = r.choice(["contig", "paged", "paged"])
        dtype = "int8" if first == "paged" and r.random() < 0.5 else "bf16"
        w0 = r.choice([0, 40, 64])
        window = r.choice([16, 48])
        slack = r.choice([0, 3, 20])
        out.append((d, hkv, g, first, dtype, w0, window, slack, r.randrange(1 << 30)))
    return out


CASES = _cases(16, 97)


@pytest.mark.parametrize("case", CASES, ids=[
    f"d{c[0]}-h{c[1]}g{c[2]}-{c[3]}-{c[4]}-w{c[5]}-ring{c[6]}s{c[7]}" for c in CASES])
def test_random_lifecycle_matches_oracle(case):
    from kvrt import KVRTError, KVRuntime, LayerSpec

    d, hkv, g, first, dtype, w0, window, slack, seed = case
    r = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    n_slots, cap, max_q = 3, 400, 2
    rows = window + max_q - 1 + slack
    specs = [LayerSpec(kv_heads=hkv, head_dim=d, layout=first, dtype=dtype, window=w0),
             LayerSpec(kv_heads=hkv, head_dim=d, layout="ring", window=window, ring_rows=rows),
             LayerSpec(kv_heads=hkv, head_dim=d, shared_src=0)]
    paged = first == "paged"
    kw = dict(block_size=BS, pool_pages=4 * n_slots * (cap // BS + 2), pool_seed=3) if paged else {}
    rt = KVRuntime(specs, n_slots, cap, max_q=max_q, device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(hkv, d, w0, dtype == "int8"), O.OracleLayer(hkv, d, window)], n_slots)
    owner = [0, 1, 0]
    scale = 1.0 / math.sqrt(d)
    # per slot: the longest the RING layer has been since the slot was last
    # empty (rows below high - rows are overwritten), the first live page and
    # the prefix mask's length
    high, live, plen = [0] * n_slots, [0] * n_slots, [0] * n_slots

    def length(s):
        return orc.length(s, 0)

    def need(t, w):
        """The first key position the query at position t sees."""
        return max(0, t - w + 1) if w > 0 else 0

    def import_fresh(s, n):
        for layer in range(2):
            k, v = randn_bf16(gen, (1, hkv, n, d)), randn_bf16(gen, (1, hkv, n, d))
            rt.import_(s, layer, k.cuda(), v.cuda())
            orc.append(s, layer, to_np(k[0]), to_np(v[0]))
        high[s] = n

    def rollback_ok(s, t):
        L = length(s)
        if t < plen[s]:
            return False
        if t in (0, L):
            return True
        if need(t, window) < max(0, high[s] - rows):
            return False
        return not (paged and (need(t, w0) if w0 > 0 else t) < live[s] * BS)

    def clone_ok(src, n):
        if n < plen[src]:
            return False
        if n == 0:
            return True
        if max(0, n - rows, high[src] - rows) > need(n, window):
            return False
        return not (paged and min(n, live[src] * BS) > need(n, w0))

    for s in range(n_slots):
        import_fresh(s, r.randint(1, 150))
    accepted = refused = steps = 0
    ops = ["step"] * 4 + ["rollback"] * 2 + ["clone", "renew", "mask"] + (["evict"] if paged and w0 else [])
    for op_i in range(40):
        op = r.choice(ops)
        where = (op_i, op)
        if op == "step":
            qn = r.choice([1, 2])
            slots = sorted(r.sample(range(n_slots), r.randint(1, n_slots)))
            slots = [s for s in slots if length(s) + qn <= cap]
            if not slots:
                continue
            n = len(slots)
            for layer in range(3):
                q = randn_bf16(gen, (n, hkv * g, qn, d), 0.5)
                if owner[layer] == layer:
                    k, v = randn_bf16(gen, (n, hkv, qn, d)), randn_bf16(gen, (n, hkv, qn, d))
                    out = rt.append_attend(layer, q.cuda(), k.cuda(), v.cuda(), slots, scale)
                    for i, s in enumerate(slots):
                        orc.append(s, layer, to_np(k[i]), to_np(v[i]))
                else:
                    out = rt.attend(layer, q.cuda(), slots, scale)
                torch.cuda.synchronize()
                for i, s in enumerate(slots):
                    ref = orc.attend(s, owner[layer], to_np(q[i]), scale)
                    err = float(np.abs(to_np(out[i]) - ref).max())
                    assert err <= ATOL, (where, layer, s, err)
            for s in slots:
                high[s] = max(high[s], length(s))
            steps += 1
        elif op == "rollback":
            s = r.randrange(n_slots)
            L = length(s)
            t = r.choice([0, max(0, L - r.randint(0, 3)), max(0, L - r.randint(0, rows + 4)), r.randint(0, L)])
            if rollback_ok(s, t):
                rt.truncate(s, t)
                for layer in range(2):
                    orc.truncate(s, layer, t)
                if t == 0:
                    high[s] = live[s] = 0
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
            if clone_ok(src, n):
                rt.copy_prefix(src, dst, n)
                for layer in range(2):
                    orc.copy_prefix(src, dst, layer, n)
                orc.copy_prefix_attention(src, dst)
                high[dst] = max(n, high[src]) if n else 0
                live[dst] = min(n, live[src] * BS) // BS if paged else 0
                plen[dst] = plen[src]
                accepted += 1
            else:
                with pytest.raises(KVRTError) as e:
                    rt.copy_prefix(src, dst, n)
                assert e.value.code == -2, where
                refused += 1
            assert rt.seq_length(dst, 1) == length(dst), where
        elif op == "evict":  # pages wholly older than the next query's window
            s = r.randrange(n_slots)
            keep = r.randint(0, need(length(s), w0))
            rt.evict(s, keep)
            live[s] = max(live[s], keep // BS)
        elif op == "mask":  # a prefix-attention mask over the slot's first positions
            s = r.randrange(n_slots)
            if length(s) == 0:
                continue
            p = r.randint(1, min(length(s), 96))
            mask = torch.tensor([r.random() < 0.6 for _ in range(p)], dtype=torch.bool)
            mask[0] = True
            rt.set_prefix_attention(s, mask)
            orc.set_prefix_attention(s, mask.numpy())
            plen[s] = p
        else:  # release, then a new session in the slot
            s = r.randrange(n_slots)
            rt.set_prefix_attention(s, None)
            orc.set_prefix_attention(s, None)
            plen[s] = 0
            rt.truncate(s, 0)
            for layer in range(2):
                orc.truncate(s, layer, 0)
            live[s] = 0
            import_fresh(s, r.randint(0, 200))
        assert rt.health() == 0, where
    assert steps and accepted, (steps, accepted, refused)
    # stored rows, bit for bit, from the first position the next query sees
    torch.cuda.synchronize()
    for s in range(n_slots):
        L = length(s)
        if L == 0:
            continue
        for layer, start in ((0, max(need(L, w0), live[s] * BS if paged else 0)), (1, need(L, window))):
            k, v, _ = rt.gather(layer, [s], start_pos=[start], mask_dtype=None)
            torch.cuda.synchronize()
            ok_, ov = orc.values(s, layer)
            if k.dtype == torch.bfloat16:
                assert np.array_equal(bits(k[0]), O.f32_to_bf16_bits(ok_[:, start:])), (s, layer)
                assert np.array_equal(bits(v[0]), O.f32_to_bf16_bits(ov[:, start:])), (s, layer)
            else:
                assert np.array_equal(to_np(k[0]), ok_[:, start:]) and np.array_equal(to_np(v[0]), ov[:, start:])
