"""GPU parity of the reference-API mirror: KVRTCache as an HF cache, the
kv_cache / thinker_cache / talker helpers over kvrt storage, and the golden
attention vectors through the HIP kernel. Cache contents are compared bit for
bit with the oracle, with torch.cat / slicing results, or with the reference
tests' own expectations; attention within 1e-2 max-abs."""
from __future__ import annotations

import copy
import math
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, np_bf16_bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2
GOLDEN = Path(__file__).resolve().parent / "golden"


def _runtime(specs, n_slots=4, capacity=256, **kw):
    from kvrt import KVRuntime

    return KVRuntime(specs, n_slots, capacity, device="cuda", **kw)


def test_kvrt_cache_update_matches_hf_dynamic_layer_bitwise():
    from kvrt import KVRTCache, LayerSpec
    from transformers.cache_utils import DynamicLayer

    gen = torch.Generator().manual_seed(31)
    rt = _runtime([LayerSpec(kv_heads=2, head_dim=64)] * 2, capacity=64, max_q=4)
    cache = KVRTCache(rt)
    hf = [DynamicLayer(), DynamicLayer()]
    for q in (3, 1, 4, 2):
        for layer in range(2):
            k = randn_bf16(gen, (1, 2, q, 64)).cuda()
            v = randn_bf16(gen, (1, 2, q, 64)).cuda()
            got_k, got_v = cache.update(k, v, layer)
            want_k, want_v = hf[layer].update(k, v)
            np.testing.assert_array_equal(bits(got_k), bits(want_k))
            np.testing.assert_array_equal(bits(got_v), bits(want_v))
    assert cache.get_seq_length() == 10 and cache.get_seq_length(1) == 10
    np.testing.assert_array_equal(bits(cache.layers[1].keys), bits(hf[1].keys))
    pairs = list(cache)
    assert len(pairs) == 2 and pairs[0][0].shape == (1, 2, 10, 64)


def test_sliding_layer_update_returns_what_hf_sliding_layer_returns():
    from kvrt import KVRTCache, LayerSpec
    from transformers.cache_utils import DynamicSlidingWindowLayer

    gen = torch.Generator().manual_seed(32)
    w = 8
    rt = _runtime([LayerSpec(kv_heads=1, head_dim=128, layout="ring", window=w, ring_rows=w + 3)], capacity=200,
                  max_q=4)
    cache = KVRTCache(rt)
    hf = DynamicSlidingWindowLayer(sliding_window=w)
    for q in (4, 1, 3, 4, 1, 2, 4, 1):
        k = randn_bf16(gen, (1, 1, q, 128))
        v = randn_bf16(gen, (1, 1, q, 128))
        got_k, got_v = cache.update(k.cuda(), v.cuda(), 0)
        want_k, want_v = hf.update(k, v)
        np.testing.assert_array_equal(bits(got_k), bits(want_k))
        np.testing.assert_array_equal(bits(got_v), bits(want_v))
        np.testing.assert_array_equal(bits(cache.layers[0].keys), bits(hf.keys))
    assert cache.get_seq_length() == hf.get_seq_length()


def test_positional_writes_follow_the_slot_kv_cache_contract():
    """The reference's _SlotKVCache cases (test_future_prefix_slot_kv_cache.py:24-86)."""
    from kvrt import KVRTCache, LayerSpec

    rt = _runtime([LayerSpec(kv_heads=1, head_dim=64)] * 2, capacity=16, max_q=4)
    cache = KVRTCache(rt)

    def write(layer, positions, value=1.0):
        x = torch.full((1, 1, len(positions), 64), value, dtype=torch.bfloat16, device="cuda")
        k_all, v_all = cache.update(x, x, layer, {"cache_position": torch.tensor(positions, dtype=torch.long)})
        # like _SlotKVCache.update (future_prefix.py:544-565): the slot's whole
        # [1, H, max_cache_len, D] storage, matching masks built at capacity
        assert tuple(k_all.shape) == tuple(v_all.shape) == (1, 1, 16, 64)
        assert k_all.data_ptr() == rt.storage(layer)[0][cache.slot].data_ptr()  # zero-copy view of the slot
        return k_all

    write(0, [0, 1])
    assert cache.get_seq_length() == 2
    write(0, [2, 4], 2.0)  # joint frame: prefix row 2 + audio row 4
    assert cache.get_seq_length() == 5
    keys = cache.layers[0].keys
    assert float(keys[0, 0, 4, 0]) == 2.0 and float(keys[0, 0, 3].abs().sum()) == 0.0  # hole reads zero
    write(0, [3, 5])
    assert cache.get_seq_length() == 6
    assert cache.get_seq_length(1) == 0  # per-layer lengths
    one = torch.ones((1, 1, 2, 64), dtype=torch.bfloat16, device="cuda")
    cache.update(one, one, 1)  # no position: append at the layer's own length
    assert cache.get_seq_length(1) == 2
    empty = torch.empty((1, 1, 0, 64), dtype=torch.bfloat16, device="cuda")
    cache.update(empty, empty, 0, {"cache_position": torch.empty((0,), dtype=torch.long)})
    assert cache.get_seq_length(0) == 6
    for bad in (-1, 16):
        with pytest.raises(OverflowError):
            write(1, [bad])
    assert cache.get_seq_length(1) == 2
    cache.reset()
    assert cache.get_seq_length(0) == 0 and cache.get_seq_length(1) == 0
    write(0, [3])
    assert cache.get_seq_length(0) == 4
    assert float(cache.layers[0].keys[0, 0, :3].abs().sum()) == 0.0  # reset zeroed the rows
    assert rt.health() == 0


def test_crop_truncate_and_deepcopy_semantics():
    from kvrt import KVRTCache, LayerSpec

    gen = torch.Generator().manual_seed(33)
    rt = _runtime([LayerSpec(kv_heads=2, head_dim=128)] * 3, capacity=128, max_q=4)
    cache = KVRTCache(rt)
    rows = [randn_bf16(gen, (1, 2, 20, 128)).cuda() for _ in range(3)]
    for layer in range(3):
        cache.update(rows[layer], rows[layer], layer)
    cache.crop(25)  # positive and not shorter: no-op
    assert cache.get_seq_length() == 20
    cache.crop(0)
    assert cache.get_seq_length() == 20
    cache.crop(-3)
    assert [cache.get_seq_length(l) for l in range(3)] == [17, 17, 17]
    cache.crop(12)
    assert cache.get_seq_length(2) == 12
    snap = copy.deepcopy(cache)
    assert snap.slot != cache.slot and snap.get_seq_length(1) == 12
    extra = randn_bf16(gen, (1, 2, 4, 128)).cuda()
    cache.update(extra, extra, 0)
    for layer in range(3):
        np.testing.assert_array_equal(bits(snap.layers[layer].keys), bits(rows[layer][:, :, :12]))
    assert snap.get_seq_length(0) == 12 and cache.get_seq_length(0) == 16
    free_before = len(rt._free_slots)
    snap.release()
    assert len(rt._free_slots) == free_before + 1


def test_talker_prefix_turn_rollback_is_a_length_edit():
    from kvrt import KVRTCache, LayerSpec
    from kvrt.kv_cache import TalkerPrefixKV, TurnKVState, _kv_seq_len, kv_memory_bytes

    gen = torch.Generator().manual_seed(34)
    rt = _runtime([LayerSpec(kv_heads=8, head_dim=128)] * 2, capacity=512, max_q=2)
    live = KVRTCache(rt)
    prefix_rows = [randn_bf16(gen, (1, 8, 100, 128)).cuda() for _ in range(2)]
    for layer in range(2):
        live.update(prefix_rows[layer], prefix_rows[layer], layer)
    prefix = TalkerPrefixKV()
    prefix.store(live)  # device snapshot in another slot
    assert prefix.seq_len == 100 and isinstance(prefix.kv, KVRTCache) and prefix.kv.slot != live.slot
    turn = TurnKVState()
    turn.start_from_prefix(prefix)
    turn.kv = live  # the engine decodes on its live cache
    for _ in range(7):
        for layer in range(2):
            x = randn_bf16(gen, (1, 8, 1, 128)).cuda()
            live.update(x, x, layer)
        turn.append(live)
    assert _kv_seq_len(turn.kv) == 107
    storage_before = bits(rt.storage(0)[0]).copy()
    turn.truncate_to_prefix()
    torch.cuda.synchronize()
    assert live.get_seq_length() == 100 and live.get_seq_length(1) == 100
    np.testing.assert_array_equal(bits(rt.storage(0)[0]), storage_before)  # no KV byte moved
    for layer in range(2):
        np.testing.assert_array_equal(bits(prefix.kv.layers[layer].keys), bits(prefix_rows[layer]))
    assert kv_memory_bytes(live) == 2 * 2 * 8 * 100 * 128 * 2


def test_tuple_slice_and_clone_on_device_tensors():
    from kvrt.kv_cache import _clone_kv, _slice_kv

    gen = torch.Generator().manual_seed(35)
    pairs = tuple((randn_bf16(gen, (1, 8, 30, 128)).cuda(), randn_bf16(gen, (1, 8, 30, 128)).cuda())
                  for _ in range(3))
    sliced = _slice_kv(pairs, 17)
    clones = _clone_kv(pairs)
    torch.cuda.synchronize()
    for (k, v), (ks, vs), (kc, vc) in zip(pairs, sliced, clones):
        np.testing.assert_array_equal(bits(ks), bits(k[:, :, :17]))
        np.testing.assert_array_equal(bits(vs), bits(v[:, :, :17]))
        assert ks.is_contiguous() and ks.data_ptr() != k.data_ptr()
        np.testing.assert_array_equal(bits(kc), bits(k))
        assert kc.data_ptr() != k.data_ptr()
    neg = _slice_kv(pairs, -5)
    np.testing.assert_array_equal(bits(neg[0][0]), bits(pairs[0][0][:, :, :-5]))


def _static_cache(max_cache_len=8):
    from transformers import PretrainedConfig, StaticCache

    config = PretrainedConfig()
    config.num_hidden_layers = 2
    config.layer_types = ["full_attention", "full_attention"]
    config.sliding_window = None
    config.attention_chunk_size = None
    return StaticCache(config=config, max_cache_len=max_cache_len, max_batch_size=1, device="cuda",
                       dtype=torch.float32)


def test_static_cache_prefix_copy_on_device_matches_reference_test():
    """test_thinker_cache_prefix.py:42-66 on GPU StaticCache objects."""
    from kvrt.thinker_cache import copy_static_cache_prefix

    source = _static_cache()
    for i, layer in enumerate(source.layers):
        keys = torch.arange(5 * 8, dtype=torch.float32, device="cuda").reshape(1, 2, 5, 4)
        source.update(keys, keys + 1000.0 + i, i)
    target = _static_cache()
    res = copy_static_cache_prefix(source, target, 3)
    assert (res.copied_tokens, res.layer_count, res.copied_bytes) == (3, 2, 384)
    assert int(target.get_seq_length()) == 3
    for s, t in zip(source.layers, target.layers):
        assert s.keys.shape == t.keys.shape
        assert torch.equal(t.keys[:, :, :3], s.keys[:, :, :3])
        assert torch.equal(t.values[:, :, :3], s.values[:, :, :3])
        assert int(torch.count_nonzero(t.keys[:, :, 3:])) == 0
    src_prefix = source.layers[0].keys[:, :, :3].clone()
    nk = torch.full((1, 2, 1, 4), -7.0, device="cuda")
    target.update(nk, nk, 0)
    assert int(source.get_seq_length()) == 5 and int(target.get_seq_length()) == 4
    assert torch.equal(source.layers[0].keys[:, :, :3], src_prefix)
    assert not torch.equal(source.layers[0].keys[:, :, 3:4], nk)


def test_kvrt_slot_prefix_copy_for_branch_reuse():
    from kvrt import KVRTCache, LayerSpec
    from kvrt.thinker_cache import (CachePrefixCopyError, copy_static_cache_prefix,
                                    longest_common_prefix_length)

    gen = torch.Generator().manual_seed(36)
    specs = [LayerSpec(kv_heads=1, head_dim=256), LayerSpec(kv_heads=1, head_dim=256, shared_src=0),
             LayerSpec(kv_heads=1, head_dim=512)]
    rt = _runtime(specs, n_slots=3, capacity=300, max_q=2)
    src, dst = KVRTCache(rt), KVRTCache(rt)
    rows = {0: randn_bf16(gen, (1, 1, 40, 256)).cuda(), 2: randn_bf16(gen, (1, 1, 40, 512)).cuda()}
    for layer, r in rows.items():
        src.update(r, r, layer)
    n = longest_common_prefix_length(list(range(40)), list(range(25)) + [99])
    res = copy_static_cache_prefix(src, dst, n)
    assert res.copied_tokens == 25 and res.layer_count == 2
    assert res.copied_bytes == 2 * 25 * (256 + 512) * 2
    for layer, r in rows.items():
        np.testing.assert_array_equal(bits(dst.layers[layer].keys), bits(r[:, :, :25]))
    np.testing.assert_array_equal(bits(dst.layers[1].keys), bits(rows[0][:, :, :25]))  # shared alias
    with pytest.raises(CachePrefixCopyError, match="not empty"):
        copy_static_cache_prefix(src, dst, 3)


def test_talker_import_from_hf_shaped_cache():
    from kvrt import KVRTCache, LayerSpec
    from kvrt.talker import import_dynamic_cache

    gen = torch.Generator().manual_seed(37)
    rt = _runtime([LayerSpec(kv_heads=8, head_dim=128)] * 28, n_slots=2, capacity=160, max_q=2)
    seq = 131
    pairs = [(randn_bf16(gen, (1, 8, seq, 128)).cuda(), randn_bf16(gen, (1, 8, seq, 128)).cuda()) for _ in range(28)]
    hf = SimpleNamespace(layers=[SimpleNamespace(keys=k, values=v) for k, v in pairs], get_seq_length=lambda: seq)
    cache = KVRTCache(rt)
    junk = torch.ones((1, 8, 150, 128), dtype=torch.bfloat16, device="cuda")
    cache.update(junk, junk, 0)  # stale rows beyond the import must be cleared
    assert import_dynamic_cache(hf, cache) == seq
    for layer in (0, 13, 27):
        np.testing.assert_array_equal(bits(cache.layers[layer].keys), bits(pairs[layer][0]))
        np.testing.assert_array_equal(bits(cache.layers[layer].values), bits(pairs[layer][1]))
    k0 = rt.storage(0)[0][cache.slot]
    assert int(torch.count_nonzero(k0[:, seq:])) == 0


@pytest.mark.parametrize("n_streams", [1, 2, 4])
def test_gather_and_attend_over_ragged_streams(n_streams):
    """Listener micro-batch (N in {1, 2, 4}): gather = zero-padded batch + mask,
    attend per stream and attend over the padded batch agree with the oracle."""
    from kvrt import KVRTCache, LayerSpec
    from kvrt.cache import append_attend, attend, attend_padded, gather

    gen = torch.Generator().manual_seed(40 + n_streams)
    spec = LayerSpec(kv_heads=8, head_dim=128)
    rt = _runtime([spec], n_slots=4, capacity=1100, max_q=2)
    orc = O.OracleCache([O.OracleLayer(8, 128)], 4)
    caches = [KVRTCache(rt) for _ in range(n_streams)]
    lens = [int(x) for x in torch.randint(64, 1025, (n_streams,), generator=gen)]
    for c, n in zip(caches, lens):
        k, v = randn_bf16(gen, (1, 8, n, 128)), randn_bf16(gen, (1, 8, n, 128))
        c.update(k.cuda(), v.cuda(), 0)
        orc.append(c.slot, 0, to_np(k[0]), to_np(v[0]))
    scale = 1 / math.sqrt(128)
    for _ in range(3):  # one listener frame = 2 rows per stream
        q = randn_bf16(gen, (n_streams, 8, 2, 128), 0.5)
        k = randn_bf16(gen, (n_streams, 8, 2, 128))
        v = randn_bf16(gen, (n_streams, 8, 2, 128))
        out = append_attend(q.cuda(), k.cuda(), v.cuda(), caches, 0, scale)
        for i, c in enumerate(caches):
            orc.append(c.slot, 0, to_np(k[i]), to_np(v[i]))
            assert np.abs(to_np(out[i]) - orc.attend(c.slot, 0, to_np(q[i]), scale)).max() <= ATOL
    kp, vp, mask = gather(caches, 0)
    ko, vo, mo = orc.gather(0, [c.slot for c in caches], kp.shape[2])
    np.testing.assert_array_equal(bits(kp), np_bf16_bits(ko))
    np.testing.assert_array_equal(bits(vp), np_bf16_bits(vo))
    np.testing.assert_array_equal(mask.cpu().numpy(), mo)
    _, _, fmask = gather(caches, 0, target_length=kp.shape[2] + 5, mask_dtype=torch.float32)
    assert float(fmask[0, -1]) == torch.finfo(torch.float32).min and float(fmask[0, 0]) == 0.0
    q = randn_bf16(gen, (n_streams, 8, 2, 128), 0.5).cuda()
    a = attend(q, caches, 0, scale)
    b = attend_padded(q, kp, vp, mask.sum(1).to(torch.int32), scale)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(a), bits(b))


def _golden_cases():
    data = np.load(GOLDEN / "attention_small.npz", allow_pickle=False)
    names = sorted({k.split(".")[0] for k in data.files})
    return [(n, {f: data[f"{n}.{f}"] for f in ("q", "k", "v", "out", "meta", "scale")}) for n in names]


@pytest.mark.parametrize("name,case", _golden_cases())
def test_golden_attention_vectors_through_the_hip_kernel(name, case):
    from kvrt import KVRuntime, LayerSpec

    hq, hkv, d, n_keys, qn, window = [int(x) for x in case["meta"]]
    as_bf16 = lambda b: torch.from_numpy(b.view(np.int16).copy()).view(torch.bfloat16)  # noqa: E731
    q, k, v = as_bf16(case["q"]), as_bf16(case["k"]), as_bf16(case["v"])
    rt = KVRuntime([LayerSpec(kv_heads=hkv, head_dim=d, window=window)], 1, 64, max_q=2, device="cuda")
    rt.import_(0, 0, k[None].cuda(), v[None].cuda())
    out = rt.attend(0, q[None].cuda(), [0], float(case["scale"][0]))
    err = np.abs(to_np(out[0]) - case["out"]).max()
    assert err <= ATOL, err


@pytest.mark.parametrize("seed", range(8))
def test_random_update_crop_and_copy_sequences_match_hf_caches(seed):
    """Seeded random sequences on a KVRTCache with two global layers and a
    sliding one, mirrored on transformers' DynamicLayer /
    DynamicSlidingWindowLayer: appends of 1..4 rows (the returned states and
    the stored layers bit for bit), crops of the global layers by a negative
    count, to an absolute length or by 0, and deep copies that must keep their
    contents while the original moves on."""
    import random

    from kvrt import KVRTCache, LayerSpec
    from transformers.cache_utils import DynamicLayer, DynamicSlidingWindowLayer

    r = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    d, hkv, w = r.choice([64, 128]), r.choice([1, 2]), r.choice([5, 16])
    rt = _runtime([LayerSpec(kv_heads=hkv, head_dim=d)] * 2
                  + [LayerSpec(kv_heads=hkv, head_dim=d, layout="ring", window=w, ring_rows=w + 3 + r.choice([0, 6]))],
                  n_slots=8, capacity=400, max_q=4)
    cache = KVRTCache(rt)
    hf = [DynamicLayer(), DynamicLayer(), DynamicSlidingWindowLayer(sliding_window=w)]
    snaps = []
    for _ in range(30):
        op = r.choice(["update"] * 3 + ["crop", "copy"])
        if op == "update" and cache.get_seq_length(0) + 4 <= 400:
            q = r.randint(1, 4)
            for layer in (0, 1):
                k, v = randn_bf16(gen, (1, hkv, q, d)).cuda(), randn_bf16(gen, (1, hkv, q, d)).cuda()
                got, want = cache.update(k, v, layer), hf[layer].update(k, v)
                for a, b in zip(got, want):
                    np.testing.assert_array_equal(bits(a), bits(b))
            k, v = randn_bf16(gen, (1, hkv, q, d)), randn_bf16(gen, (1, hkv, q, d))
            got, want = cache.update(k.cuda(), v.cuda(), 2), hf[2].update(k, v)
            for a, b in zip(got, want):
                np.testing.assert_array_equal(bits(a), bits(b))
        elif op == "crop" and hf[0].is_initialized:
            L = cache.get_seq_length(0)
            tokens = r.choice([0, -r.randint(1, 6), r.randint(0, L + 3)])
            for layer in (0, 1):
                cache._crop_layer(layer, tokens)
                hf[layer].crop(tokens)
                assert cache.get_seq_length(layer) == hf[layer].get_seq_length()
        elif op == "copy" and hf[0].is_initialized and cache.get_seq_length(0) == cache.get_seq_length(2) \
                and len(snaps) < 4:
            snaps.append((copy.deepcopy(cache), [copy.deepcopy(h) for h in hf[:2]]))
        for layer in (0, 1):
            if hf[layer].is_initialized:
                np.testing.assert_array_equal(bits(cache.layers[layer].keys), bits(hf[layer].keys))
                np.testing.assert_array_equal(bits(cache.layers[layer].values), bits(hf[layer].values))
    for snap, hfs in snaps:
        for layer in (0, 1):
            assert snap.get_seq_length(layer) == hfs[layer].get_seq_length()
            np.testing.assert_array_equal(bits(snap.layers[layer].keys), bits(hfs[layer].keys))
        snap.release()
    cache.release()
    assert rt.health() == 0 and len(rt._free_slots) == 8
