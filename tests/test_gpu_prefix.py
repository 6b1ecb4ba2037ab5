"""GPU parity of the listener prefix-attention mask (key k < P visible only
where prefix_attention[k] != 0, on top of causal and window visibility;
gemma4_listener_kernels.cuh:517-518) against the oracle at max-abs 1e-2:
the golden vectors on both decode kernels and the prefill kernel, the
canonical 34-position mask and random masks up to 512 positions at the
listener's shapes (D 256 / 512, Q 1 / 2, CONTIG / RING / PAGED), the padded
tensor path, and the mask's lifecycle (clones and cross-context copies carry
it, reset and release clear it, rewinds below it are refused, rollover keeps
it) including the 35-layer Gemma-4 topology after a clone."""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2
GOLD = np.load(Path(__file__).resolve().parent / "golden" / "attention_prefix_small.npz")
CASES = sorted({k.split(".")[0] for k in GOLD.files})


def _mask(kind: str, plen: int, gen: torch.Generator) -> np.ndarray:
    if kind == "canonical":
        return O.canonical_prefix_mask(plen)
    if kind == "zeros":
        return np.zeros(plen, np.int64)
    m = torch.randint(0, 2, (plen,), generator=gen).numpy().astype(np.int64)
    m[0] = 1
    return m


@pytest.mark.parametrize("path", ["valu", "mfma", "prefill"])
@pytest.mark.parametrize("name", CASES)
def test_prefix_golden_vectors(name, path):
    from kvrt import KVRuntime, LayerSpec

    hq, hkv, d, n_keys, qn, window = (int(x) for x in GOLD[f"{name}.meta"])
    k = torch.from_numpy(GOLD[f"{name}.k"].view(np.int16)).view(torch.bfloat16)
    v = torch.from_numpy(GOLD[f"{name}.v"].view(np.int16)).view(torch.bfloat16)
    q = torch.from_numpy(GOLD[f"{name}.q"].view(np.int16)).view(torch.bfloat16)
    mask = torch.from_numpy(GOLD[f"{name}.mask"])
    scale = float(GOLD[f"{name}.scale"][0])
    rt = KVRuntime([LayerSpec(kv_heads=hkv, head_dim=d, window=window)], 2, 128, max_q=qn,
                   decode_kernel="mfma" if path == "mfma" else "valu", device="cuda")
    rt.import_(1, 0, k[None].cuda(), v[None].cuda())
    rt.set_prefix_attention(1, mask.cuda())
    assert rt.slot_info(1)["prefix_len"] == mask.numel()
    if path == "prefill":
        out = rt.attend_prefill(0, q[None].cuda(), [1], scale)
    else:
        out = rt.attend(0, q[None].cuda(), [1], scale)
    torch.cuda.synchronize()
    np.testing.assert_allclose(to_np(out[0]), GOLD[f"{name}.out"], atol=ATOL, rtol=0)
    assert rt.health() == 0


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
@pytest.mark.parametrize("layout", ["contig", "ring", "paged"])
@pytest.mark.parametrize("d,qn", [(256, 2), (256, 1), (512, 2), (512, 1)])
def test_prefix_mask_decode_parity(d, qn, layout, kernel):
    """Four slots in one launch: the canonical mask, a random 512-position mask,
    an all-zero 200-position mask and no mask; fused append + attend steps
    whose key ranges put the masked prefix across many wave splits."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(d * 10 + qn + len(layout))
    window = 512 if d == 256 else 0
    if layout == "ring" and window == 0:
        pytest.skip("a ring holds a sliding window")
    kw = dict(block_size=16, pool_pages=4 * 1400 // 16 + 8) if layout == "paged" else {}
    ring = dict(ring_rows=window + qn - 1) if layout == "ring" else {}
    spec = LayerSpec(kv_heads=1, head_dim=d, layout=layout, window=window, **ring)
    rt = KVRuntime([spec], 4, 1400, max_q=qn, decode_kernel=kernel, **kw, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, d, window)], 4)
    masks = [_mask("canonical", 34, gen), _mask("random", 512, gen), _mask("zeros", 200, gen), None]
    lens = [40, 540, 260, 300] if window else [600, 1200, 900, 700]
    for s, (n, m) in enumerate(zip(lens, masks)):
        k, v = randn_bf16(gen, (1, 1, n, d)), randn_bf16(gen, (1, 1, n, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
        if m is not None:
            rt.set_prefix_attention(s, torch.from_numpy(m).cuda())
            orc.set_prefix_attention(s, m)
    slots = [0, 1, 2, 3]
    worst = 0.0
    for _ in range(3):
        q = randn_bf16(gen, (4, 8, qn, d), 1.0 / math.sqrt(d))
        k, v = randn_bf16(gen, (4, 1, qn, d)), randn_bf16(gen, (4, 1, qn, d))
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), slots, 1.0)
        torch.cuda.synchronize()
        for i, s in enumerate(slots):
            orc.append(s, 0, to_np(k[i]), to_np(v[i]))
            worst = max(worst, float(np.abs(to_np(out[i]) - orc.attend(s, 0, to_np(q[i]), 1.0)).max()))
    assert worst <= ATOL
    assert rt.health() == 0


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
@pytest.mark.parametrize("d,hq,qn", [(128, 8, 1), (128, 2, 1), (64, 4, 2)])
def test_prefix_mask_int8_paged_decode_parity(d, hq, qn, kernel):
    """int8 PAGED decodes under prefix masks: the VALU decode and (forced
    MFMA, head_dim 64 / 128) the int8 MFMA ring kernel, whose 32-key tiles
    test the mask per key; fused append + attend steps quantise the new rows
    in the launch."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(d + hq * 7 + qn)
    spec = LayerSpec(kv_heads=1, head_dim=d, layout="paged", dtype="int8")
    rt = KVRuntime([spec], 4, 1400, max_q=qn, decode_kernel=kernel, block_size=16,
                   pool_pages=4 * 1400 // 16 + 8, pool_seed=6, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, d, 0, int8=True)], 4)
    masks = [_mask("canonical", 34, gen), _mask("random", 512, gen), _mask("zeros", 200, gen), None]
    lens = [600, 1200, 900, 700]
    for s, (n, m) in enumerate(zip(lens, masks)):
        k, v = randn_bf16(gen, (1, 1, n, d)), randn_bf16(gen, (1, 1, n, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
        if m is not None:
            rt.set_prefix_attention(s, torch.from_numpy(m).cuda())
            orc.set_prefix_attention(s, m)
    slots = [0, 1, 2, 3]
    worst = 0.0
    for _ in range(3):
        q = randn_bf16(gen, (4, hq, qn, d), 1.0 / math.sqrt(d))
        k, v = randn_bf16(gen, (4, 1, qn, d)), randn_bf16(gen, (4, 1, qn, d))
        c0 = rt.counters()
        out = rt.append_attend(0, q.cuda(), k.cuda(), v.cuda(), slots, 1.0)
        torch.cuda.synchronize()
        assert rt.counters()["mfma_decodes"] - c0["mfma_decodes"] == (1 if kernel == "mfma" else 0)
        for i, s in enumerate(slots):
            orc.append(s, 0, to_np(k[i]), to_np(v[i]))
            worst = max(worst, float(np.abs(to_np(out[i]) - orc.attend(s, 0, to_np(q[i]), 1.0)).max()))
    assert worst <= ATOL
    assert rt.health() == 0


@pytest.mark.parametrize("d,layout,qn,plen", [(256, "ring", 291, 34), (512, "contig", 291, 34),
                                              (256, "contig", 64, 512), (512, "paged", 40, 300)])
def test_prefix_mask_prefill_parity(d, layout, qn, plen):
    """A chunk whose first queries sit right after the masked prefix (Q 291
    after the canonical 34-position mask, the reference's canonical prefill),
    and chunks over random masks up to 512 positions."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(plen + qn)
    window = 512 if d == 256 else 0
    ring = dict(ring_rows=window + qn - 1) if layout == "ring" else {}
    kw = dict(block_size=16, pool_pages=2 * 1024 // 16) if layout == "paged" else {}
    spec = LayerSpec(kv_heads=1, head_dim=d, layout=layout, window=window, **ring)
    rt = KVRuntime([spec], 2, 1024, max_q=qn, **kw, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, d, window)], 2)
    m = _mask("canonical" if plen == 34 else "random", plen, gen)
    for s, n in ((0, plen), (1, plen + 200)):
        k, v = randn_bf16(gen, (1, 1, n, d)), randn_bf16(gen, (1, 1, n, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
        rt.set_prefix_attention(s, torch.from_numpy(m).cuda())
        orc.set_prefix_attention(s, m)
    k, v = randn_bf16(gen, (2, 1, qn, d)), randn_bf16(gen, (2, 1, qn, d))
    rt.append(0, k.cuda(), v.cuda(), [0, 1])
    q = randn_bf16(gen, (2, 8, qn, d), 1.0 / math.sqrt(d))
    out = rt.attend_prefill(0, q.cuda(), [0, 1], 1.0)
    torch.cuda.synchronize()
    for s in (0, 1):
        orc.append(s, 0, to_np(k[s]), to_np(v[s]))
        ref = orc.attend(s, 0, to_np(q[s]), 1.0)
        assert float(np.abs(to_np(out[s]) - ref).max()) <= ATOL
    assert rt.health() == 0


def test_prefix_mask_talker_sized_prefill_parity():
    """Prefix masks on a talker-sized prefill grid (head_dim 128, >= 512
    workgroups: pairs of 16-query blocks share a workgroup's tiles, each
    block's keys over two waves): ragged prefixes around the mask lengths, one
    stream without a mask."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(128)
    hq, hkv, d, qn = 16, 8, 128, 300
    rt = KVRuntime([LayerSpec(kv_heads=hkv, head_dim=d)], 4, 1200, max_q=qn, device="cuda")
    orc = O.OracleCache([O.OracleLayer(hkv, d)], 4)
    masks = [_mask("canonical", 34, gen), _mask("random", 512, gen), _mask("random", 120, gen), None]
    for s, (n, m) in enumerate(zip((34, 600, 150, 90), masks)):
        k, v = randn_bf16(gen, (1, hkv, n, d)), randn_bf16(gen, (1, hkv, n, d))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
        if m is not None:
            rt.set_prefix_attention(s, torch.from_numpy(m).cuda())
            orc.set_prefix_attention(s, m)
    k, v = randn_bf16(gen, (4, hkv, qn, d)), randn_bf16(gen, (4, hkv, qn, d))
    rt.append(0, k.cuda(), v.cuda(), [0, 1, 2, 3])
    q = randn_bf16(gen, (4, hq, qn, d), 1.0 / math.sqrt(d))
    out = rt.attend_prefill(0, q.cuda(), [0, 1, 2, 3], 1.0)
    torch.cuda.synchronize()
    for s in range(4):
        orc.append(s, 0, to_np(k[s]), to_np(v[s]))
        ref = orc.attend(s, 0, to_np(q[s]), 1.0)
        assert float(np.abs(to_np(out[s]) - ref).max()) <= ATOL, s
    assert rt.health() == 0


def test_prefix_mask_on_the_padded_tensor_path():
    from kvrt import attend_padded, gather
    from kvrt import KVRTCache, KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(77)
    rt = KVRuntime([LayerSpec(kv_heads=2, head_dim=128)], 3, 600, max_q=2, device="cuda")
    caches = [KVRTCache(rt) for _ in range(3)]
    orc = O.OracleCache([O.OracleLayer(2, 128)], 3)
    masks = [_mask("canonical", 34, gen), _mask("random", 120, gen), np.ones(120, np.int64)]
    for i, (c, n) in enumerate(zip(caches, (90, 300, 170))):
        k, v = randn_bf16(gen, (1, 2, n, 128)), randn_bf16(gen, (1, 2, n, 128))
        c.update(k.cuda(), v.cuda(), 0)
        orc.append(c.slot, 0, to_np(k[0]), to_np(v[0]))
        orc.set_prefix_attention(c.slot, masks[i])
    pm = np.ones((3, 120), np.int64)
    pm[0, :34] = masks[0]
    pm[1] = masks[1]
    kp, vp, mask = gather(caches, 0)
    q = randn_bf16(gen, (3, 8, 2, 128), 0.3)
    out = attend_padded(q.cuda(), kp, vp, mask.sum(1).to(torch.int32), 0.09,
                        prefix_attention=torch.from_numpy(pm).cuda())
    torch.cuda.synchronize()
    for i, c in enumerate(caches):
        assert float(np.abs(to_np(out[i]) - orc.attend(c.slot, 0, to_np(q[i]), 0.09)).max()) <= ATOL
    from kvrt.runtime import tensors_status

    assert tensors_status() == 0


def test_clone_copy_reset_and_rewind_floor_carry_the_mask():
    from kvrt import KVRTError, KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(9)
    specs = [LayerSpec(kv_heads=1, head_dim=256, layout="ring", window=512, ring_rows=513),
             LayerSpec(kv_heads=1, head_dim=512)]
    rt = KVRuntime(specs, 4, 1200, max_q=2, device="cuda")
    other = KVRuntime(specs, 2, 1200, max_q=2, device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, 256, 512), O.OracleLayer(1, 512)], 6)
    m = _mask("canonical", 34, gen)
    layers = []
    for layer, s in enumerate(specs):
        k, v = randn_bf16(gen, (1, 1, 100, s.head_dim)), randn_bf16(gen, (1, 1, 100, s.head_dim))
        layers.append((k.cuda(), v.cuda()))
        orc.append(0, layer, to_np(k[0]), to_np(v[0]))
    gen0 = rt.import_session(0, layers, torch.from_numpy(m).cuda())
    orc.set_prefix_attention(0, m)
    assert rt.slot_info(0) == {"generation": gen0, "prefix_len": 34, "min_len": 100, "max_len": 100}
    # clone within the runtime and copy into another one: rows and mask travel
    gen1 = rt.copy_prefix(0, 1, 100, generation=gen0)
    other.synchronize()
    rt.synchronize()
    other.copy_session(1, rt, 0, 100, generation=gen0)
    for layer in range(2):
        orc.copy_prefix(0, 1, layer, 100)
    orc.copy_prefix_attention(0, 1)
    assert gen1 != gen0 and rt.slot_info(1)["prefix_len"] == 34 and other.slot_info(1)["prefix_len"] == 34

    def check(runtime, slot, oslot):
        worst = 0.0
        for layer, s in enumerate(specs):
            q = randn_bf16(gen, (1, 8, 2, s.head_dim), 1.0 / math.sqrt(s.head_dim))
            out = runtime.attend(layer, q.cuda(), [slot], 1.0)
            torch.cuda.synchronize()
            worst = max(worst, float(np.abs(to_np(out[0]) - orc.attend(oslot, layer, to_np(q[0]), 1.0)).max()))
        return worst

    assert check(rt, 0, 0) <= ATOL and check(rt, 1, 1) <= ATOL
    other.synchronize()
    assert check(other, 1, 1) <= ATOL
    # rewinds below the mask and copies that would end inside it are refused
    before = rt.counters()
    for call in (lambda: rt.truncate(0, 33), lambda: rt.copy_prefix(0, 2, 20),
                 lambda: rt.rollover(0, 20, 40)):
        with pytest.raises(KVRTError) as e:
            call()
        assert e.value.code == -2
    assert rt.counters() == before and rt.seq_length(0, 0) == 100
    rt.truncate(0, 34, generation=gen0)  # the floor itself is allowed
    for layer in range(2):
        orc.truncate(0, layer, 34)
    assert check(rt, 0, 0) <= ATOL
    # reset and release clear the mask
    gen2 = rt.reset_slot(1)
    assert gen2 not in (gen0, gen1) and rt.slot_info(1)["prefix_len"] == 0
    rt.set_prefix_attention(0, None)
    assert rt.slot_info(0)["prefix_len"] == 0
    rt.truncate(0, 0)
    assert rt.health() == 0 and other.health() == 0


def test_gemma_topology_with_canonical_mask_steps_clones_and_rolls_over():
    """The 35-layer listener topology with the canonical mask on every slot:
    Q 2 steps on all layers (shared ones over 13 / 14), a rollover that keeps
    the 34-position prefix, a clone, and steps on the clone."""
    from kvrt import KVRuntime
    from tests.test_gpu_lifecycle import _gemma_specs

    gen = torch.Generator().manual_seed(350)
    specs = _gemma_specs(2)
    rt = KVRuntime(specs, 3, 2048, max_q=2, device="cuda")
    owner = [i if s.shared_src < 0 else s.shared_src for i, s in enumerate(specs)]
    orc = O.OracleCache([O.OracleLayer(1, s.head_dim, s.window) for s in specs], 3)
    m = O.canonical_prefix_mask()
    for slot, n in ((0, 600), (1, 34)):
        layers = []
        for layer in range(15):
            k = randn_bf16(gen, (1, 1, n, specs[layer].head_dim))
            v = randn_bf16(gen, (1, 1, n, specs[layer].head_dim))
            layers.append((k.cuda(), v.cuda()))
            orc.append(slot, layer, to_np(k[0]), to_np(v[0]))
        rt.import_session(slot, layers, torch.from_numpy(m).cuda())
        orc.set_prefix_attention(slot, m)
    inv_s, inv_f = O.gemma_inv_freq(256, 1e4), O.gemma_inv_freq(512, 1e6, 64)
    for layer in range(15):
        rt.set_layer_rope(layer, (inv_f if layer % 5 == 4 else inv_s).tolist())

    def step(slots):
        n = len(slots)
        worst = 0.0
        for layer, s in enumerate(specs):
            q = randn_bf16(gen, (n, 8, 2, s.head_dim), 0.5 / s.head_dim ** 0.5)
            if owner[layer] == layer:
                k = randn_bf16(gen, (n, 1, 2, s.head_dim))
                v = randn_bf16(gen, (n, 1, 2, s.head_dim))
                out = rt.append_attend(layer, q.cuda(), k.cuda(), v.cuda(), slots, 1.0)
                for i, slot in enumerate(slots):
                    orc.append(slot, layer, to_np(k[i]), to_np(v[i]))
            else:
                out = rt.attend(layer, q.cuda(), slots, 1.0)
            torch.cuda.synchronize()
            for i, slot in enumerate(slots):
                ref = orc.attend(slot, owner[layer], to_np(q[i]), 1.0)
                worst = max(worst, float(np.abs(to_np(out[i]) - ref).max()))
        return worst

    assert step([0, 1]) <= ATOL
    g0 = rt.slot_generation(0)
    rt.rollover(0, 34, 128, generation=g0)
    for layer in range(15):
        orc.rollover(0, layer, 34, 128, inv_f if layer % 5 == 4 else inv_s)
    assert rt.slot_info(0)["prefix_len"] == 34
    assert step([1, 0]) <= ATOL
    rt.copy_prefix(0, 2, rt.seq_length(0), generation=g0)
    for layer in range(15):
        orc.copy_prefix(0, 2, layer, orc.length(0, layer))
    orc.copy_prefix_attention(0, 2)
    assert step([0, 2]) <= ATOL
    assert rt.health() == 0


def test_masked_paged_d512_decode_runs_on_the_valu_kernel():
    """PAGED D 512 decodes with a mask take the VALU kernel even when the MFMA
    kernel is forced (its PAGED D 512 variant has no registers for a mask)."""
    from kvrt import KVRuntime, LayerSpec

    gen = torch.Generator().manual_seed(512)
    rt = KVRuntime([LayerSpec(kv_heads=1, head_dim=512, layout="paged")], 2, 800, max_q=2, block_size=16,
                   pool_pages=110, decode_kernel="mfma", device="cuda")
    orc = O.OracleCache([O.OracleLayer(1, 512)], 2)
    m = _mask("random", 300, gen)
    for s in (0, 1):
        k, v = randn_bf16(gen, (1, 1, 700, 512)), randn_bf16(gen, (1, 1, 700, 512))
        rt.import_(s, 0, k.cuda(), v.cuda())
        orc.append(s, 0, to_np(k[0]), to_np(v[0]))
    rt.set_prefix_attention(1, torch.from_numpy(m).cuda())
    orc.set_prefix_attention(1, m)
    q = randn_bf16(gen, (2, 8, 2, 512), 1.0 / math.sqrt(512))
    out = rt.attend(0, q.cuda(), [0, 1], 1.0)
    torch.cuda.synchronize()
    for s in (0, 1):
        assert float(np.abs(to_np(out[s]) - orc.attend(s, 0, to_np(q[s]), 1.0)).max()) <= ATOL
    assert rt.health() == 0
