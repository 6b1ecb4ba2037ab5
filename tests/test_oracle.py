"""Pins the CPU oracle (oracle/kv_oracle.py) before any GPU result is judged by it.

Each check is chosen so that a plausible mistake in the oracle fails it:
the reference's own known answers (tests/golden/reference_kats.json), golden
vectors from an independent pure-Python brute force, library routines that
compute the same thing (torch's bf16 cast, torch.cat, transformers'
DynamicSlidingWindowLayer, torch SDPA with repeat_kv), and closed forms.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kv_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
KATS = json.loads((GOLDEN / "reference_kats.json").read_text())


def _bits_to_f32(b: np.ndarray) -> np.ndarray:
    return O.bf16_bits_to_f32(b)


# ---------------------------------------------------------------------------
# bf16 rounding
# ---------------------------------------------------------------------------
def test_bf16_rounding_matches_torch_cast_including_ties_and_specials():
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(20000, generator=gen) * 10.0
    ties = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 2 ** -130, 3.0e38, -0.0,
                         float("inf"), float("-inf")], dtype=torch.float32)
    x = torch.cat([x, ties])
    want = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_bf16_bits(x.numpy())
    np.testing.assert_array_equal(got, want)
    nan = O.f32_to_bf16_bits(np.array([np.nan], np.float32))
    assert np.isnan(O.bf16_bits_to_f32(nan)).all()


# ---------------------------------------------------------------------------
# window / position math: the reference's known answers
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", KATS["q_range_from_position"]["cases"])
def test_q_range_from_position_matches_reference_static_asserts(case):
    total, start, valid = O.q_range_from_position(case["base"], case["q"], case["capacity"], case["window"])
    if "total" in case:
        assert total == case["total"]
    if "start" in case:
        assert start == case["start"]
    if "valid" in case:
        assert valid == case["valid"]


def test_visible_range_matches_reference_history_batch_limits():
    kat = KATS["history_batch_visibility"]
    for qi, limit in kat["causal_key_limit"]:
        lo, hi = O.visible_range(kat["prefix"] + qi, 0)
        assert (lo, hi + 1) == (0, limit)
    for qi, start in kat["sliding_start"]:
        lo, _ = O.visible_range(kat["prefix"] + qi, kat["sliding_window"])
        assert lo == start


@pytest.mark.parametrize("case", KATS["sliding_capacity"]["cases"])
def test_ring_capacity_matches_reference_contract(case):
    assert O.ring_capacity(case["window"], case["max_q"], case["max_seq_len"]) == case["capacity"]


def test_visible_range_agrees_with_q_range_window_start():
    # The decode window of the last query of a step starts where the native
    # range helper says (base = position of the first new row).
    for base in (0, 5, 511, 512, 513, 4000):
        for w in (1, 64, 512):
            _, start, _ = O.q_range_from_position(base, 1, 1 << 20, w)
            assert O.visible_range(base, w)[0] == start


# ---------------------------------------------------------------------------
# append / truncate / gather / sliding retention against library routines
# ---------------------------------------------------------------------------
def test_append_truncate_gather_match_torch_cat_and_slicing():
    gen = torch.Generator().manual_seed(1)
    layer = O.OracleLayer(kv_heads=2, head_dim=8)
    orc = O.OracleCache([layer], 2)
    ref = {0: None, 1: None}
    for step, q in enumerate([3, 1, 2, 1, 4]):
        for s in (0, 1):
            k = torch.randn((1, 2, q + s, 8), generator=gen).to(torch.bfloat16)
            ref[s] = k if ref[s] is None else torch.cat([ref[s], k], dim=-2)
            orc.append(s, 0, k[0].float().numpy(), k[0].float().numpy())
    orc.truncate(1, 0, 7)
    ref[1] = ref[1][:, :, :7].contiguous()
    lmax = 16
    ko, vo, mask = orc.gather(0, [1, 0], lmax)
    for i, s in enumerate((1, 0)):
        n = ref[s].shape[2]
        np.testing.assert_array_equal(ko[i, :, :n], ref[s][0].float().numpy())
        assert (ko[i, :, n:] == 0).all() and mask[i].sum() == n and mask[i, :n].all()


def test_sliding_retention_matches_transformers_sliding_layer():
    from transformers.cache_utils import DynamicSlidingWindowLayer

    w = 6
    hf = DynamicSlidingWindowLayer(sliding_window=w)
    gen = torch.Generator().manual_seed(2)
    total = 0
    history = []
    for q in (4, 1, 1, 3, 1, 2, 5):
        k = torch.randn((1, 1, q, 4), generator=gen)
        hf.update(k, k)
        history.append(k)
        total += q
        lo, hi = O.sliding_retained(total, w)
        want = torch.cat(history, dim=-2)[:, :, lo:hi]
        assert torch.equal(hf.keys, want), (total, lo, hi)


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
def _golden_cases():
    data = np.load(GOLDEN / "attention_small.npz", allow_pickle=False)
    names = sorted({k.split(".")[0] for k in data.files})
    return [(n, {f: data[f"{n}.{f}"] for f in ("q", "k", "v", "out", "meta", "scale")}) for n in names]


@pytest.mark.parametrize("name,case", _golden_cases())
def test_attend_matches_bruteforce_golden_vectors(name, case):
    hq, hkv, d, n_keys, qn, window = [int(x) for x in case["meta"]]
    q, k, v = (_bits_to_f32(case[x]) for x in ("q", "k", "v"))
    pos = np.arange(n_keys - qn, n_keys)
    got = O.attend(q, k, v, pos, float(case["scale"][0]), window)
    np.testing.assert_allclose(got, case["out"], rtol=0, atol=2e-6)


def test_attend_matches_torch_sdpa_with_repeat_kv_in_float64():
    """GQA head map h -> h // g as HF repeat_kv, causal + sliding mask, fp64."""
    gen = torch.Generator().manual_seed(3)
    hq, hkv, d, n, qn, w = 8, 2, 32, 50, 3, 20
    q = torch.randn((hq, qn, d), generator=gen, dtype=torch.float64)
    k = torch.randn((hkv, n, d), generator=gen, dtype=torch.float64)
    v = torch.randn((hkv, n, d), generator=gen, dtype=torch.float64)
    g = hq // hkv
    kr = k.repeat_interleave(g, dim=0)  # transformers repeat_kv order
    vr = v.repeat_interleave(g, dim=0)
    qpos = torch.arange(n - qn, n)[:, None]
    kpos = torch.arange(n)[None, :]
    mask = (kpos <= qpos) & (kpos >= qpos - w + 1)
    want = F.scaled_dot_product_attention(q[None], kr[None], vr[None], attn_mask=mask, scale=0.2)[0]
    got = O.attend(q.numpy(), k.numpy(), v.numpy(), np.arange(n - qn, n), 0.2, w)
    np.testing.assert_allclose(got, want.numpy(), atol=1e-6)


def test_attend_closed_forms():
    rng = np.random.default_rng(4)
    # one visible key -> the output is that key's value row
    q = rng.standard_normal((4, 1, 16)).astype(np.float32)
    k = rng.standard_normal((2, 1, 16)).astype(np.float32)
    v = rng.standard_normal((2, 1, 16)).astype(np.float32)
    out = O.attend(q, k, v, np.array([0]), 0.3)
    np.testing.assert_allclose(out[:, 0], np.repeat(v[:, 0], 2, axis=0), atol=1e-7)
    # equal keys -> uniform weights -> mean of the visible values
    k = np.repeat(rng.standard_normal((1, 1, 16)), 30, axis=1).astype(np.float32)
    v = rng.standard_normal((1, 30, 16)).astype(np.float32)
    q = rng.standard_normal((3, 1, 16)).astype(np.float32)
    out = O.attend(q, k, v, np.array([29]), 0.5)
    np.testing.assert_allclose(out[:, 0], np.repeat(v[0].mean(0, keepdims=True), 3, 0), atol=1e-6)
    # window W keeps only the last W keys
    out_w = O.attend(q, k, v, np.array([29]), 0.5, window=4)
    np.testing.assert_allclose(out_w[:, 0], np.repeat(v[0, 26:].mean(0, keepdims=True), 3, 0), atol=1e-6)


def test_attend_is_invariant_to_key_order_when_all_keys_are_visible():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((4, 1, 16)).astype(np.float32)
    k = rng.standard_normal((2, 20, 16)).astype(np.float32)
    v = rng.standard_normal((2, 20, 16)).astype(np.float32)
    perm = rng.permutation(20)
    a = O.attend(q, k, v, np.array([19]), 0.25)
    b = O.attend(q, k[:, perm], v[:, perm], np.array([19]), 0.25)
    np.testing.assert_allclose(a, b, atol=1e-6)


def test_attend_with_explicit_key_positions_matches_contiguous():
    """Ring / paged views hand the oracle keys with absolute positions."""
    rng = np.random.default_rng(6)
    q = rng.standard_normal((2, 2, 8)).astype(np.float32)
    k = rng.standard_normal((1, 12, 8)).astype(np.float32)
    v = rng.standard_normal((1, 12, 8)).astype(np.float32)
    pos = np.array([10, 11])
    a = O.attend(q, k, v, pos, 0.3, window=5)
    kp = np.arange(12)
    keep = kp >= 6  # a ring that retains positions 6..11
    b = O.attend(q, k[:, keep], v[:, keep], pos, 0.3, window=5, key_positions=kp[keep])
    np.testing.assert_allclose(a, b, atol=1e-7)


# ---------------------------------------------------------------------------
# int8
# ---------------------------------------------------------------------------
def test_int8_quantisation_matches_golden_half_even_rows():
    data = np.load(GOLDEN / "int8_small.npz", allow_pickle=False)
    x = _bits_to_f32(data["x"])
    q, s = O.quantize_int8(x)
    np.testing.assert_array_equal(q, data["q"])
    np.testing.assert_array_equal(s.view(np.uint32), data["scale"].view(np.uint32))


def test_int8_closed_forms():
    scale = np.float32(0.5)
    ints = np.arange(-127, 128, dtype=np.float32)
    x = (ints * scale)[None]
    q, s = O.quantize_int8(x)  # amax = 63.5 -> scale exactly 0.5: exact round trip
    assert s[0] == scale
    np.testing.assert_array_equal(q[0], ints.astype(np.int8))
    np.testing.assert_array_equal(O.dequantize_int8(q, s), x)
    q0, s0 = O.quantize_int8(np.zeros((1, 8), np.float32))
    assert s0[0] == 0 and not q0.any()
    assert np.abs(O.quantize_int8(np.random.default_rng(0).standard_normal((50, 128)))[0]).max() == 127


def test_oracle_cache_int8_layer_dequantises_what_it_stored():
    rng = np.random.default_rng(8)
    orc = O.OracleCache([O.OracleLayer(2, 16, int8=True)], 1)
    k = rng.standard_normal((2, 5, 16)).astype(np.float32)
    orc.append(0, 0, k, k)
    kd, _ = orc.values(0, 0)
    q, s = O.quantize_int8(k)
    np.testing.assert_array_equal(kd, q.astype(np.float32) * s[..., None])
    assert np.abs(kd - k).max() <= np.abs(k).max() / 127 / 2 + 1e-6


# ---------------------------------------------------------------------------
# planted mistakes are caught (the checks above are not tautologies)
# ---------------------------------------------------------------------------
def test_a_wrong_gqa_head_map_fails_the_sdpa_check():
    gen = torch.Generator().manual_seed(3)
    hq, hkv, d, n = 4, 2, 8, 10
    q = torch.randn((hq, 1, d), generator=gen, dtype=torch.float64)
    k = torch.randn((hkv, n, d), generator=gen, dtype=torch.float64)
    v = torch.randn((hkv, n, d), generator=gen, dtype=torch.float64)
    want = F.scaled_dot_product_attention(q[None], k.repeat_interleave(2, 0)[None], v.repeat_interleave(2, 0)[None],
                                          scale=0.3)[0].numpy()
    good = O.attend(q.numpy(), k.numpy(), v.numpy(), np.array([n - 1]), 0.3)
    # h % Hkv instead of h // g: the interleaved map of a different GQA layout
    bad = np.stack([O.attend(q[h:h + 1].numpy(), k[h % hkv:h % hkv + 1].numpy(), v[h % hkv:h % hkv + 1].numpy(),
                             np.array([n - 1]), 0.3)[0] for h in range(hq)])
    assert np.abs(good - want).max() < 1e-6  # the oracle returns float32
    assert np.abs(bad - want).max() > 1e-3


def test_an_off_by_one_window_fails_the_golden_vectors():
    name, case = [c for c in _golden_cases() if c[0] == "gqa8_sliding_q2"][0]
    hq, hkv, d, n_keys, qn, window = [int(x) for x in case["meta"]]
    q, k, v = (_bits_to_f32(case[x]) for x in ("q", "k", "v"))
    pos = np.arange(n_keys - qn, n_keys)
    bad = O.attend(q, k, v, pos, float(case["scale"][0]), window + 1)
    assert np.abs(bad - case["out"]).max() > 1e-3


def test_bruteforce_and_vectorised_oracles_agree_on_random_tiny_cases():
    rng = np.random.default_rng(9)
    for _ in range(5):
        hkv = int(rng.integers(1, 3))
        hq = hkv * int(rng.integers(1, 4))
        n = int(rng.integers(1, 9))
        qn = int(rng.integers(1, min(n, 3) + 1))
        w = int(rng.integers(0, 4))
        q = rng.standard_normal((hq, qn, 4))
        k = rng.standard_normal((hkv, n, 4))
        v = rng.standard_normal((hkv, n, 4))
        pos = list(range(n - qn, n))
        a = O.attend(q, k, v, np.array(pos), 0.7, w)
        b = np.asarray(O.attend_bruteforce(q.tolist(), k.tolist(), v.tolist(), pos, 0.7, w))
        assert math.isclose(float(np.abs(a - b).max()), 0.0, abs_tol=1e-6)


# ---------------------------------------------------------------------------
# listener prefix-attention mask (gemma4_listener_kernels.cuh:517-518)
# ---------------------------------------------------------------------------
PREFIX_GOLD = np.load(GOLDEN / "attention_prefix_small.npz")
PREFIX_CASES = sorted({k.split(".")[0] for k in PREFIX_GOLD.files})


def test_canonical_prefix_mask_matches_reference_known_answer():
    kat = KATS["canonical_prefix_mask"]
    m = O.canonical_prefix_mask(kat["length"])
    assert m.dtype == np.int64 and m.shape == (kat["length"],)
    assert list(np.flatnonzero(m)) == kat["visible"]
    # the same rule at other lengths: first and last position only
    assert list(np.flatnonzero(O.canonical_prefix_mask(7))) == [0, 6]


def _prefix_case(name):
    g = PREFIX_GOLD
    hq, hkv, d, n_keys, qn, window = (int(x) for x in g[f"{name}.meta"])
    q = _bits_to_f32(g[f"{name}.q"])
    k = _bits_to_f32(g[f"{name}.k"])
    v = _bits_to_f32(g[f"{name}.v"])
    return q, k, v, g[f"{name}.mask"], np.arange(n_keys - qn, n_keys), window, float(g[f"{name}.scale"][0]), \
        g[f"{name}.out"]


@pytest.mark.parametrize("name", PREFIX_CASES)
def test_prefix_attend_matches_bruteforce_golden(name):
    q, k, v, mask, pos, window, scale, want = _prefix_case(name)
    got = O.attend(q, k, v, pos, scale, window, prefix_attention=mask)
    np.testing.assert_allclose(got, want, atol=1e-6, rtol=0)


def test_prefix_attend_is_attention_over_the_visible_key_subset():
    """Closed form: masking keys is attention over the keys that remain
    (torch SDPA in fp64 over the subset, repeat_kv GQA)."""
    gen = torch.Generator().manual_seed(5)
    hq, hkv, d, n_keys = 8, 2, 32, 50
    q = torch.randn(hq, 1, d, generator=gen, dtype=torch.float64)
    k = torch.randn(hkv, n_keys, d, generator=gen, dtype=torch.float64)
    v = torch.randn(hkv, n_keys, d, generator=gen, dtype=torch.float64)
    mask = torch.randint(0, 2, (20,), generator=gen).numpy()
    keep = [j for j in range(n_keys) if j >= 20 or mask[j]]
    ref = F.scaled_dot_product_attention(q[None], k[:, keep].repeat_interleave(hq // hkv, 0)[None],
                                         v[:, keep].repeat_interleave(hq // hkv, 0)[None], scale=0.2)[0]
    got = O.attend(q.numpy(), k.numpy(), v.numpy(), np.array([n_keys - 1]), 0.2, prefix_attention=mask)
    np.testing.assert_allclose(got, ref.numpy(), atol=1e-6)


def test_prefix_attend_closed_forms():
    gen = torch.Generator().manual_seed(6)
    q = torch.randn(4, 1, 16, generator=gen).numpy()
    k = torch.randn(1, 40, 16, generator=gen).numpy()
    v = torch.randn(1, 40, 16, generator=gen).numpy()
    # an all-ones mask changes nothing
    np.testing.assert_array_equal(O.attend(q, k, v, np.array([39]), 0.3, prefix_attention=np.ones(34, np.int64)),
                                  O.attend(q, k, v, np.array([39]), 0.3))
    # one visible key inside the prefix, query at the prefix's last position: o = v[j]
    one = np.zeros(34, np.int64)
    one[9] = 1
    out = O.attend(q, k[:, :34], v[:, :34], np.array([33]), 0.3, prefix_attention=one)
    np.testing.assert_allclose(out, np.broadcast_to(v[0, 9], out.shape), atol=1e-6)
    # a zero mask hides the whole prefix: attention over keys P.. only
    zero = np.zeros(34, np.int64)
    np.testing.assert_allclose(O.attend(q, k, v, np.array([39]), 0.3, prefix_attention=zero),
                               O.attend(q, k[:, 34:], v[:, 34:], np.array([39]), 0.3,
                                        key_positions=np.arange(34, 40)), atol=1e-6)
    # the canonical mask with the first query after it: keys {0, 33, 34}
    out = O.attend(q, k[:, :35], v[:, :35], np.array([34]), 0.3, prefix_attention=O.canonical_prefix_mask())
    sub = [0, 33, 34]
    np.testing.assert_allclose(out, O.attend(q, k[:, sub], v[:, sub], np.array([34]), 0.3,
                                             key_positions=np.array(sub)), atol=1e-6)
    # a key below P is hidden from every query, also one whose window starts before it
    w_out = O.attend(q, k, v, np.array([39]), 0.3, window=8, prefix_attention=np.zeros(34, np.int64))
    np.testing.assert_allclose(w_out, O.attend(q, k[:, 34:], v[:, 34:], np.array([39]), 0.3, window=8,
                                               key_positions=np.arange(34, 40)), atol=1e-6)


@pytest.mark.parametrize("slip", ["polarity", "shifted", "inclusive_end", "ignored"])
def test_planted_prefix_slips_fail_the_golden_vectors(slip):
    """Plausible mistakes in the prefix term each change a golden output."""
    failed = 0
    for name in PREFIX_CASES:
        q, k, v, mask, pos, window, scale, want = _prefix_case(name)
        if slip == "polarity":
            m = 1 - mask
        elif slip == "shifted":
            m = np.roll(mask, 1)
        elif slip == "inclusive_end":  # key P consulted as if masked
            m = np.concatenate([mask, [0]])
        else:
            m = None
        got = O.attend(q, k, v, pos, scale, window, prefix_attention=m)
        failed += not np.allclose(got, want, atol=1e-3)
    assert failed > 0, f"slip {slip} passed every golden case"


def test_oracle_cache_carries_the_prefix_mask_through_copies():
    cache = O.OracleCache([O.OracleLayer(1, 16)], 3)
    gen = torch.Generator().manual_seed(8)
    k = torch.randn(1, 40, 16, generator=gen).numpy()
    v = torch.randn(1, 40, 16, generator=gen).numpy()
    q = torch.randn(2, 1, 16, generator=gen).numpy()
    cache.append(0, 0, k, v)
    cache.set_prefix_attention(0, O.canonical_prefix_mask())
    cache.copy_prefix(0, 1, 0, 40)
    cache.copy_prefix_attention(0, 1)
    np.testing.assert_array_equal(cache.attend(1, 0, q, 0.25), cache.attend(0, 0, q, 0.25))
    want = O.attend(q, k, v, np.array([39]), 0.25, prefix_attention=O.canonical_prefix_mask())
    np.testing.assert_allclose(cache.attend(0, 0, q, 0.25), want, atol=0)
    cache.set_prefix_attention(0, None)
    np.testing.assert_allclose(cache.attend(0, 0, q, 0.25), O.attend(q, k, v, np.array([39]), 0.25), atol=0)
