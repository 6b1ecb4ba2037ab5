"""BASELINE.json configs 1-5 as GPU parity cases, through the C ABI.

Shapes, seeds and draw order follow the configs: inputs are seeded N(0,1)
draws rounded to bf16 on the CPU (prefill K, prefill V, then per step q, k,
v), so the HIP path and the oracle see identical bytes. Attention outputs are
checked against the fp64 oracle (max-abs 1e-2) at the steps named in each
test; cache contents (gathered logical views) bit for bit at the end. Long
runs check a fixed subset of steps and layers so the suite stays quick; every
layer of every step runs on the GPU.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from oracle import torch_ref as T
from tests.helpers import bits, np_bf16_bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2


def _err(out, ref):
    return float(np.abs(to_np(out) - ref).max())


def test_config1_single_layer_append_and_attend_100_steps():
    """Config 1: batch 1, 8 q / 1 kv head, D 256, 512 prefilled positions,
    100 steps of append + causal attention, scale 1/sqrt(256), seed 0. Every
    step is also checked against torch's CPU SDPA over torch.cat-grown K/V
    (the reference's own CPU path)."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(0)
    rt = KVRuntime([LayerSpec(kv_heads=1, head_dim=256)], 1, 612, max_q=1, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, 256)], 1)
    ref_layer = T.RefLayer()
    kp, vp = randn_bf16(gen, (1, 1, 512, 256)), randn_bf16(gen, (1, 1, 512, 256))
    rt.import_(0, 0, kp.cuda(), vp.cuda())
    orc.append(0, 0, to_np(kp[0]), to_np(vp[0]))
    ref_layer.update(kp.float(), vp.float())
    scale = 1.0 / 16
    for step in range(100):
        q, k, v = (randn_bf16(gen, s, 0.5) for s in ((1, 8, 1, 256), (1, 1, 1, 256), (1, 1, 1, 256)))
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), [0], scale)
        orc.append(0, 0, to_np(k[0]), to_np(v[0]))
        fk, fv = ref_layer.update(k.float(), v.float())
        sdpa = T.attend(q.float(), fk, fv, scale)
        assert _err(out[0], orc.attend(0, 0, to_np(q[0]), scale)) <= ATOL, step
        assert _err(out, sdpa.numpy()) <= ATOL, step
    ko, vo, _ = orc.gather(0, [0], 612)
    k_all, v_all, _ = rt.gather(0, [0])
    np.testing.assert_array_equal(bits(k_all), np_bf16_bits(ko))
    np.testing.assert_array_equal(bits(v_all), np_bf16_bits(vo))
    assert rt.health() == 0


def test_config2_thinker_stack_ring_and_global_256_steps():
    """Config 2: 30 layers, 5 sliding (512-token ring) : 1 global, 8 q / 1 kv
    head, D 256, prefix 2048, 256 single-token steps, seed 1. Attention of
    every layer at steps 0, 32, ..., 255; logical cache contents at the end."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(1)
    n_layers, w = 30, 512
    glob = [(i + 1) % 6 == 0 for i in range(n_layers)]
    specs = [LayerSpec(kv_heads=1, head_dim=256) if g else
             LayerSpec(kv_heads=1, head_dim=256, layout="ring", window=w, ring_rows=w) for g in glob]
    rt = KVRuntime(specs, 1, 2048 + 256, max_q=1, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, 256, 0 if g else w) for g in glob], 1)
    for layer in range(n_layers):
        kp, vp = randn_bf16(gen, (1, 1, 2048, 256)), randn_bf16(gen, (1, 1, 2048, 256))
        rt.import_(0, layer, kp.cuda(), vp.cuda())
        orc.append(0, layer, to_np(kp[0]), to_np(vp[0]))
    scale = 1.0 / 16
    checks = set(range(0, 256, 32)) | {255}
    for step in range(256):
        for layer in range(n_layers):
            q, k, v = (randn_bf16(gen, s, 0.5) for s in ((1, 8, 1, 256), (1, 1, 1, 256), (1, 1, 1, 256)))
            out = rt.append_attend(layer, q.cuda(), k.cuda(), v.cuda(), [0], scale)
            orc.append(0, layer, to_np(k[0]), to_np(v[0]))
            if step in checks:
                assert _err(out[0], orc.attend(0, layer, to_np(q[0]), scale)) <= ATOL, (step, layer)
    for layer in range(n_layers):
        L = orc.length(0, layer)
        start = [O.sliding_retained(L, w)[0]] if not glob[layer] else None
        ko, vo, _ = orc.gather(layer, [0], L - (start[0] if start else 0), start)
        kg, vg, _ = rt.gather(layer, [0])
        np.testing.assert_array_equal(bits(kg), np_bf16_bits(ko))
        np.testing.assert_array_equal(bits(vg), np_bf16_bits(vo))
    assert rt.seq_length(0, 0) == 2048 + 256
    assert rt.health() == 0


@pytest.mark.parametrize("n_streams", [1, 2, 4])
def test_config3_listener_microbatch_gather_500_steps(n_streams):
    """Config 3: N ragged streams (lengths U[64, 1024]), 16 layers, 8 kv heads,
    D 128; each step appends one listener frame (Q = 2 rows, the reference's
    GEMMA4_STREAM_Q_LEN) per stream, gathers the padded [N, 8, Lmax, 128] batch
    with its mask and attends over it (8 q heads); 500 steps, seed 2. Gather
    bit-exact and attention of every layer at steps 0, 100, ..., 499. Odd
    layers take the fused append + gather call, even ones the two calls."""
    from kvrt import KVRuntime, LayerSpec, attend_tensors

    gen = torch.Generator().manual_seed(2)
    n_layers = 16
    lens = [int(x) for x in torch.randint(64, 1025, (n_streams,), generator=gen)]
    rt = KVRuntime([LayerSpec(kv_heads=8, head_dim=128)] * n_layers, n_streams, max(lens) + 1000 + 8, max_q=2,
                   device="cuda")
    orc = O.OracleCache([O.OracleLayer(8, 128)] * n_layers, n_streams)
    for layer in range(n_layers):
        for s, n in enumerate(lens):
            kp, vp = randn_bf16(gen, (1, 8, n, 128)), randn_bf16(gen, (1, 8, n, 128))
            rt.import_(s, layer, kp.cuda(), vp.cuda())
            orc.append(s, layer, to_np(kp[0]), to_np(vp[0]))
    slots = list(range(n_streams))
    scale = 1.0 / math.sqrt(128)
    checks = {0, 100, 200, 300, 400, 499}
    for step in range(500):
        for layer in range(n_layers):
            q, k, v = (randn_bf16(gen, (n_streams, 8, 2, 128), 0.5) for _ in range(3))
            if layer % 2 == 0:
                rt.append(layer, k.cuda(), v.cuda(), slots)
                kpad, vpad, mask = rt.gather(layer, slots)
            else:  # the fused append + gather (one launch)
                lm = max(rt.seq_length(s, layer) for s in slots) + 2
                kpad = torch.empty((n_streams, 8, lm, 128), dtype=torch.bfloat16, device="cuda")
                vpad = torch.empty_like(kpad)
                mask = torch.empty((n_streams, lm), dtype=torch.bool, device="cuda")
                rt.append_gather(layer, k.cuda(), v.cuda(), slots, out=(kpad, vpad, mask))
            out = attend_tensors(q.cuda(), kpad, vpad, mask.sum(1).to(torch.int32), scale)
            for s in slots:
                orc.append(s, layer, to_np(k[s]), to_np(v[s]))
            if step in checks:
                ko, vo, mo = orc.gather(layer, slots, kpad.shape[2])
                np.testing.assert_array_equal(bits(kpad), np_bf16_bits(ko))
                np.testing.assert_array_equal(bits(vpad), np_bf16_bits(vo))
                np.testing.assert_array_equal(mask.cpu().numpy(), mo)
                for s in slots:
                    assert _err(out[s], orc.attend(s, layer, to_np(q[s]), scale)) <= ATOL, (step, layer, s)
    assert rt.health() == 0


def test_config4_talker_with_turn_local_rollback_1000_steps():
    """Config 4: 28 layers, 16 q / 8 kv heads, D 128, 4 sessions starting at
    U[512, 4096] positions; 1000 decode steps; every 25 steps each session rolls
    back k ~ U{1, 50} positions, then resumes; seed 3. Rollback must move no KV
    bytes. Layers 0, 13 and 27 are mirrored in the oracle: their attention
    after every rollback and their contents at the end."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(3)
    n_layers, n_sess = 28, 4
    mirrored = (0, 13, 27)
    l0 = [int(x) for x in torch.randint(512, 4097, (n_sess,), generator=gen)]
    rt = KVRuntime([LayerSpec(kv_heads=8, head_dim=128)] * n_layers, n_sess, 4096 + 1000 + 8, max_q=1,
                   device="cuda")
    orc = O.OracleCache([O.OracleLayer(8, 128)] * n_layers, n_sess)
    dev_gen = torch.Generator(device="cuda").manual_seed(3)
    for layer in range(n_layers):
        for s, n in enumerate(l0):
            if layer in mirrored:  # seeded CPU draws, mirrored in the oracle
                kp, vp = randn_bf16(gen, (1, 8, n, 128)), randn_bf16(gen, (1, 8, n, 128))
                orc.append(s, layer, to_np(kp[0]), to_np(vp[0]))
                kp, vp = kp.cuda(), vp.cuda()
            else:  # the other layers only need values of the same law
                kp = torch.randn((1, 8, n, 128), generator=dev_gen, device="cuda").to(torch.bfloat16)
                vp = torch.randn((1, 8, n, 128), generator=dev_gen, device="cuda").to(torch.bfloat16)
            rt.import_(s, layer, kp, vp)
    slots = list(range(n_sess))
    scale = 1.0 / math.sqrt(128)
    checked = 0
    for step in range(1000):
        rolled = step > 0 and step % 25 == 0
        if rolled:
            before = bits(rt.storage(0)[0][0, 0, :64]).copy()
            for s in slots:
                kk = int(torch.randint(1, 51, (1,), generator=gen))
                new_len = max(1, rt.seq_length(s, 0) - kk)
                rt.truncate(s, new_len)
                for layer in mirrored:
                    orc.truncate(s, layer, new_len)
            np.testing.assert_array_equal(bits(rt.storage(0)[0][0, 0, :64]), before)
        for layer in range(n_layers):
            q = randn_bf16(gen, (n_sess, 16, 1, 128), 0.5)
            k = randn_bf16(gen, (n_sess, 8, 1, 128), 0.5)
            v = randn_bf16(gen, (n_sess, 8, 1, 128), 0.5)
            out = rt.append_attend(layer, q.cuda(), k.cuda(), v.cuda(), slots, scale)
            if layer in mirrored:
                for s in slots:
                    orc.append(s, layer, to_np(k[s]), to_np(v[s]))
                if rolled or step in (0, 999):
                    for s in slots:
                        assert _err(out[s], orc.attend(s, layer, to_np(q[s]), scale)) <= ATOL, (step, layer, s)
                        checked += 1
    assert checked >= 40 * 3 * 4
    for layer in mirrored:
        for s in slots:
            assert rt.seq_length(s, layer) == orc.length(s, layer)
        kg, vg, _ = rt.gather(layer, slots)
        ko, vo, _ = orc.gather(layer, slots, kg.shape[2])
        np.testing.assert_array_equal(bits(kg), np_bf16_bits(ko))
        np.testing.assert_array_equal(bits(vg), np_bf16_bits(vo))
    assert rt.counters()["truncations"] == 39 * n_sess
    assert rt.health() == 0


def test_config5_paged_int8_under_memory_pressure():
    """Config 5: 16 sessions, 16-token pages from one shared pool handed out in
    a seeded random order, contexts U[256, 8192], int8 K/V with one fp32 scale
    per (token, head), 8 kv heads, D 128, 16 q heads, 28 layers; per step each
    session appends one token (quantised in-kernel), attends over its 4096-token
    window (dequantised in-kernel) and evicts the pages wholly older than the
    window; seed 4. Checked against the oracle's dequantise-then-attend on
    layers 0 and 27 (every 8 steps) and their int8 contents, dequantised."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(4)
    n_layers, n_sess, w, bs = 28, 16, 4096, 16
    mirrored = (0, 27)
    lens = [int(x) for x in torch.randint(256, 8193, (n_sess,), generator=gen)]
    pages = n_sess * (w // bs + 8)
    spec = LayerSpec(kv_heads=8, head_dim=128, layout="paged", dtype="int8", window=w)
    rt = KVRuntime([spec] * n_layers, n_sess, 8192 + 64, max_q=1, block_size=bs, pool_pages=pages, pool_seed=4,
                   device="cuda")
    orc = O.OracleCache([O.OracleLayer(8, 128, w, int8=True)] * n_layers, n_sess)
    dev_gen = torch.Generator(device="cuda").manual_seed(4)
    for layer in range(n_layers):
        for s, n in enumerate(lens):
            # Only what the first query's window can see is stored (and drawn);
            # rows below first_pos are never mapped, read or attended.
            first = max(0, n - w + 1)
            if layer in mirrored:
                kp = torch.zeros((1, 8, n, 128), dtype=torch.bfloat16)
                vp = torch.zeros((1, 8, n, 128), dtype=torch.bfloat16)
                kp[:, :, first:] = randn_bf16(gen, (1, 8, n - first, 128))
                vp[:, :, first:] = randn_bf16(gen, (1, 8, n - first, 128))
                orc.append(s, layer, to_np(kp[0]), to_np(vp[0]))
                kp, vp = kp.cuda(), vp.cuda()
            else:
                kp = torch.zeros((1, 8, n, 128), dtype=torch.bfloat16, device="cuda")
                vp = torch.zeros((1, 8, n, 128), dtype=torch.bfloat16, device="cuda")
                kp[:, :, first:] = torch.randn((1, 8, n - first, 128), generator=dev_gen, device="cuda")
                vp[:, :, first:] = torch.randn((1, 8, n - first, 128), generator=dev_gen, device="cuda")
            rt.import_(s, layer, kp, vp, first_pos=first)
    slots = list(range(n_sess))
    scale = 1.0 / math.sqrt(128)
    pt0 = rt.counters()["pages_in_use"]
    assert pt0 <= pages
    for step in range(32):
        for layer in range(n_layers):
            q = randn_bf16(gen, (n_sess, 16, 1, 128), 0.5)
            k = randn_bf16(gen, (n_sess, 8, 1, 128))
            v = randn_bf16(gen, (n_sess, 8, 1, 128))
            out = rt.append_attend(layer, q.cuda(), k.cuda(), v.cuda(), slots, scale)
            if layer in mirrored:
                for s in slots:
                    orc.append(s, layer, to_np(k[s]), to_np(v[s]))
                if step % 8 == 0 or step == 31:
                    for s in slots:
                        assert _err(out[s], orc.attend(s, layer, to_np(q[s]), scale)) <= ATOL, (step, layer, s)
        for s in slots:  # pages wholly below the next query's window (position L) are released
            rt.evict(s, max(0, rt.seq_length(s, 0) + 1 - w))
    c = rt.counters()
    assert c["pages_in_use"] <= pages and c["pages_evicted"] > 0
    for layer in mirrored:
        starts = [max(0, orc.length(s, layer) - w + 1) for s in slots]
        kg, vg, _ = rt.gather(layer, slots, start_pos=starts)
        ko, vo, _ = orc.gather(layer, slots, kg.shape[2], starts)
        np.testing.assert_array_equal(to_np(kg).view(np.uint32), ko.view(np.uint32))
        np.testing.assert_array_equal(to_np(vg).view(np.uint32), vo.view(np.uint32))
    assert rt.health() == 0
