"""GPU parity against the fp64 oracle over seeded random layer shapes: fused
append + decode attention (head_dim 64 / 128 / 256, CONTIG / RING / PAGED,
bf16 and PAGED int8, 1..8 KV heads, GQA groups 1..8, Q 1 / 2, 1..4 ragged
streams of 1..4000 positions, with and without a window, on the AUTO, VALU and
MFMA decode kernels), chunked prefill (head_dim 64..512, GQA groups 1..8
including 3 and 6, chunks of 1..300 queries over ragged prefixes), appends
and ragged gathers (bit-exact) and the context-free tensor attention (device
lengths, windows, prefix-attention masks). Attention max-abs 1e-2, as every
attention test."""
from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, np_bf16_bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2


def _cases(n_cases: int, seed: int, max_len: int) -> list[tuple]:
    r = random.Random(seed)
    out = []
    while len(out) < n_cases:
        d = r.choice([64, 128, 256])
        layout = r.choice(["contig", "ring", "paged"])
        dtype = "int8" if layout == "paged" and r.random() < 0.5 else "bf16"
        hkv, g, qn = r.choice([1, 2, 4, 8]), r.choice([1, 2, 4, 8]), r.choice([1, 2])
        if g * qn > 16 or (dtype == "int8" and g * qn > 8):
            continue
        kernel = r.choice(["auto", "valu", "mfma"])
        if layout == "ring":
            window = r.choice([64, 200])
        elif layout == "paged":
            window = r.choice([0, 0, 300])
        else:
            window = r.choice([0, 0, 128])
        lens = tuple(r.randint(1, max_len) for _ in range(r.choice([1, 2, 3, 4])))
        out.append((d, layout, dtype, hkv, g, qn, kernel, window, lens))
    return out


# short streams, and streams long enough for many workgroups per (stream,
# head) and the LDS DMA rings (>= 2048 keys)
CASES = _cases(24, 2024, 700) + _cases(16, 7, 4000)


@pytest.mark.parametrize("case", CASES, ids=[
    f"d{c[0]}-{c[1]}-{c[2]}-h{c[3]}g{c[4]}q{c[5]}-{c[6]}-w{c[7]}-n{len(c[8])}" for c in CASES])
def test_random_shape_fused_decode_parity(case):
    from kvrt import KVRuntime, LayerSpec

    d, layout, dtype, hkv, g, qn, kernel, window, lens = case
    gen = torch.Generator().manual_seed(d * 1000 + hkv * 100 + g * 10 + qn + sum(lens))
    n = len(lens)
    cap = max(lens) + 3 * qn + 8
    kw = {}
    if layout == "ring":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="ring", window=window, ring_rows=window + qn + 2)
    elif layout == "paged":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="paged", window=window, dtype=dtype)
        kw = dict(block_size=16, pool_pages=n * ((cap + 15) // 16) + 8, pool_seed=5)
    else:
        spec = LayerSpec(kv_heads=hkv, head_dim=d, window=window)
    rt = KVRuntime([spec], n, cap, max_q=qn, decode_kernel=kernel, device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(hkv, d, window, dtype == "int8")], n)
    for s, length in enumerate(lens):
        k, v = randn_bf16(gen, (1, hkv, length, d)), randn_bf16(gen, (1, hkv, length, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    slots = list(range(n))
    scale = 1.0 / math.sqrt(d)
    worst = 0.0
    for _ in range(3):
        q = randn_bf16(gen, (n, hkv * g, qn, d), 0.5)
        k, v = randn_bf16(gen, (n, hkv, qn, d), 0.5), randn_bf16(gen, (n, hkv, qn, d), 0.5)
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), slots, scale)
        torch.cuda.synchronize()
        for i in slots:
            orc.append(i, 0, to_np(k[i]), to_np(v[i]))
            ref = orc.attend(i, 0, to_np(q[i]), scale)
            worst = max(worst, float(np.abs(to_np(out[i]) - ref).max()))
    assert worst <= ATOL, worst
    assert rt.health() == 0
    rt.close()


def _prefill_cases(n_cases: int, seed: int) -> list[tuple]:
    r = random.Random(seed)
    out = []
    while len(out) < n_cases:
        d = r.choice([64, 128, 256, 512])
        layout = r.choice(["contig", "ring", "paged"] if d < 512 else ["contig", "paged"])
        hkv, g = r.choice([1, 2, 4, 8]), r.choice([1, 2, 3, 4, 6, 8])
        qn = r.choice([1, 5, 16, 33, 100, 300])
        window = r.choice([64, 300]) if layout == "ring" else r.choice([0, 0, 200])
        prefix = tuple(r.randint(0, 1500) for _ in range(r.choice([1, 2, 3, 4])))
        out.append((d, layout, hkv, g, qn, window, prefix))
    return out


PREFILL_CASES = _prefill_cases(20, 11)


@pytest.mark.parametrize("case", PREFILL_CASES, ids=[
    f"d{c[0]}-{c[1]}-h{c[2]}g{c[3]}-q{c[4]}-w{c[5]}-n{len(c[6])}" for c in PREFILL_CASES])
def test_random_shape_prefill_parity(case):
    """Chunked-prefill attention (kvrt_attend_prefill_async) over seeded random
    shapes, GQA groups that are not powers of two included."""
    from kvrt import KVRuntime, LayerSpec

    d, layout, hkv, g, qn, window, prefix = case
    gen = torch.Generator().manual_seed(d + hkv * 10 + g * 100 + qn * 1000 + sum(prefix))
    n = len(prefix)
    cap = max(prefix) + qn + 8
    kw = {}
    if layout == "ring":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="ring", window=window, ring_rows=window + qn - 1)
    elif layout == "paged":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="paged", window=window)
        kw = dict(block_size=16, pool_pages=n * ((cap + 15) // 16) + 8, pool_seed=3)
    else:
        spec = LayerSpec(kv_heads=hkv, head_dim=d, window=window)
    rt = KVRuntime([spec], n, cap, max_q=qn, device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(hkv, d, window)], n)
    for s, p in enumerate(prefix):
        if p:
            k, v = randn_bf16(gen, (1, hkv, p, d)), randn_bf16(gen, (1, hkv, p, d))
            rt.import_(s, 0, k.cuda(), v.cuda())
            orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    k, v = randn_bf16(gen, (n, hkv, qn, d)), randn_bf16(gen, (n, hkv, qn, d))
    rt.append(0, k.cuda(), v.cuda(), list(range(n)))
    for s in range(n):
        orc.append(s, 0, to_np(k[s]), to_np(v[s]))
    q = randn_bf16(gen, (n, hkv * g, qn, d), 0.5)
    scale = 1.0 / math.sqrt(d)
    out = rt.attend_prefill(0, q.cuda(), list(range(n)), scale)
    torch.cuda.synchronize()
    assert rt.health() == 0
    worst = max(float(np.abs(to_np(out[s]) - orc.attend(s, 0, to_np(q[s]), scale)).max()) for s in range(n))
    assert worst <= ATOL, worst
    rt.close()


def _gather_cases(n_cases: int, seed: int) -> list[tuple]:
    r = random.Random(seed)
    out = []
    for _ in range(n_cases):
        d = r.choice([64, 128, 256, 512])
        layout = r.choice(["contig", "ring", "paged"] if d < 512 else ["contig", "paged"])
        dtype = "int8" if layout == "paged" and r.random() < 0.5 else "bf16"
        hkv, qn = r.choice([1, 2, 4, 8]), r.choice([1, 2, 3])
        window = r.choice([64, 200]) if layout == "ring" else 0
        lens = tuple(r.randint(1, 600) for _ in range(r.choice([1, 2, 3, 4])))
        out.append((d, layout, dtype, hkv, qn, window, lens))
    return out


GATHER_CASES = _gather_cases(16, 13)


@pytest.mark.parametrize("case", GATHER_CASES, ids=[
    f"d{c[0]}-{c[1]}-{c[2]}-h{c[3]}-q{c[4]}-w{c[5]}-n{len(c[6])}" for c in GATHER_CASES])
def test_random_shape_append_gather_bitexact(case):
    """Appends (fused with the gather where the layer allows it: bf16 CONTIG /
    RING) then the ragged gather: bit-exact against the oracle's padded batch
    (int8 layers gather dequantised fp32)."""
    from kvrt import KVRuntime, LayerSpec

    d, layout, dtype, hkv, qn, window, lens = case
    gen = torch.Generator().manual_seed(d * 7 + hkv * 31 + qn + sum(lens))
    n = len(lens)
    cap = max(lens) + 3 * qn + 8
    kw = {}
    if layout == "ring":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="ring", window=window, ring_rows=window + qn + 2)
    elif layout == "paged":
        spec = LayerSpec(kv_heads=hkv, head_dim=d, layout="paged", dtype=dtype)
        kw = dict(block_size=16, pool_pages=n * ((cap + 15) // 16) + 8, pool_seed=9)
    else:
        spec = LayerSpec(kv_heads=hkv, head_dim=d)
    rt = KVRuntime([spec], n, cap, max_q=qn, device="cuda", **kw)
    orc = O.OracleCache([O.OracleLayer(hkv, d, window, dtype == "int8")], n)
    for s, length in enumerate(lens):
        k, v = randn_bf16(gen, (1, hkv, length, d)), randn_bf16(gen, (1, hkv, length, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    slots = list(range(n))
    fused = dtype == "bf16" and layout != "paged"
    for _ in range(2):
        k, v = randn_bf16(gen, (n, hkv, qn, d)), randn_bf16(gen, (n, hkv, qn, d))
        for s in slots:
            orc.append(s, 0, to_np(k[s]), to_np(v[s]))
        kept = [min(orc.length(s, 0), window - 1) if window else orc.length(s, 0) for s in slots]
        lmax = max(kept)
        if fused:
            ok = torch.empty((n, hkv, lmax, d), dtype=torch.bfloat16, device="cuda")
            ov = torch.empty_like(ok)
            om = torch.empty((n, lmax), dtype=torch.bool, device="cuda")
            gk, gv, gm = rt.append_gather(0, k.cuda(), v.cuda(), slots, out=(ok, ov, om))
        else:
            rt.append(0, k.cuda(), v.cuda(), slots)
            gk, gv, gm = rt.gather(0, slots, lmax=lmax)
        torch.cuda.synchronize()
        starts = [O.sliding_retained(orc.length(s, 0), window)[0] for s in slots] if window else None
        ko, vo, mo = orc.gather(0, slots, lmax, starts)
        if gk.dtype == torch.bfloat16:
            np.testing.assert_array_equal(bits(gk), np_bf16_bits(ko))
            np.testing.assert_array_equal(bits(gv), np_bf16_bits(vo))
        else:
            np.testing.assert_array_equal(to_np(gk).view(np.uint32), ko.view(np.uint32))
            np.testing.assert_array_equal(to_np(gv).view(np.uint32), vo.view(np.uint32))
        np.testing.assert_array_equal(gm.cpu().numpy(), mo)
    assert rt.health() == 0
    rt.close()


def _tensor_cases(n_cases: int, seed: int) -> list[tuple]:
    r = random.Random(seed)
    out = []
    while len(out) < n_cases:
        d = r.choice([64, 128, 256, 512])
        hkv, g, qn = r.choice([1, 2, 4, 8]), r.choice([1, 2, 4, 8]), r.choice([1, 2, 3, 4])
        if g * qn > 16:  # the tensor path takes up to 16 query rows per kv head
            continue
        lmax = r.randint(8, 1200)
        lens = tuple(r.randint(qn, lmax) for _ in range(r.choice([1, 2, 3, 4])))
        window = r.choice([0, 0, 64, 300]) if d < 512 else 0
        plen = r.choice([0, 0, 34, 200, 512])
        out.append((d, hkv, g, qn, lmax, lens, window, plen))
    return out


TENSOR_CASES = _tensor_cases(12, 17)


@pytest.mark.parametrize("case", TENSOR_CASES, ids=[
    f"d{c[0]}-h{c[1]}g{c[2]}q{c[3]}-L{c[4]}-w{c[6]}-p{c[7]}-n{len(c[5])}" for c in TENSOR_CASES])
def test_random_shape_tensor_attention_parity(case):
    """Context-free attention over caller-owned padded K/V (kvrt_attend_tensors_async)
    with device lengths, windows and prefix-attention masks."""
    from kvrt import attend_tensors

    d, hkv, g, qn, lmax, lens, window, plen = case
    gen = torch.Generator().manual_seed(d + hkv * 3 + g * 5 + qn * 7 + lmax + plen)
    n = len(lens)
    k, v = randn_bf16(gen, (n, hkv, lmax, d)), randn_bf16(gen, (n, hkv, lmax, d))
    q = randn_bf16(gen, (n, hkv * g, qn, d), 0.5)
    pm = None
    if plen:
        pm = torch.randint(0, 2, (n, plen), generator=gen, dtype=torch.int64)
        pm[:, 0] = 1
    scale = 1.0 / math.sqrt(d)
    out = attend_tensors(q.cuda(), k.cuda(), v.cuda(), torch.tensor(lens, dtype=torch.int32).cuda(), scale,
                         window=window, prefix_attention=None if pm is None else pm.cuda())
    torch.cuda.synchronize()
    worst = 0.0
    for b, length in enumerate(lens):
        ref = O.attend(to_np(q[b]), to_np(k[b, :, :length]), to_np(v[b, :, :length]),
                       np.arange(length - qn, length), scale, window=window,
                       prefix_attention=None if pm is None else pm[b].numpy())
        worst = max(worst, float(np.abs(to_np(out[b]) - ref).max()))
    assert worst <= ATOL, worst
