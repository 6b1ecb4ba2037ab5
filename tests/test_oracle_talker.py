"""Pins the talker-mask oracle (oracle.kv_oracle.talker_mask / attend_masked).

Known answers come from the reference's own tests of the talker visibility:
  * tests/kernel/test_qwen_native_audio_q1.py:156-182 (audio query after all
    real prefix frames: prefix and causal audio visible, the next key masked);
  * tests/kernel/test_virtual_prefix_g0_contract.py:22-43 (mode 1 hides the
    prefix from the audio query only; mode 2 adds gate - log(count) on the
    visible prefix and masks the rest).
Those tests build the mask in float32 on the Python path; the native kernels
(qwen_talker_kernels.cu:296-347) store it as bf16, so the gated value is
checked as the bf16 rounding of the same number. The attention side is pinned
by closed forms that reduce it to the (golden-pinned) causal oracle, by a
log-sum-exp decomposition of the gate, and by torch's SDPA with an additive
mask — the routine the reference runs (qwen_talker_aten_attention.cpp:150-160).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from scipy.special import logsumexp

from oracle import kv_oracle as O

FLOOR = O.MASKED_BF16


def test_masked_value_is_bf16_finfo_min():
    assert O.MASKED_BF16 == float(torch.finfo(torch.bfloat16).min)
    assert O.MASKED_BF16 == -3.3895313892515355e38


def test_q1_suffix_mask_kat():
    # test_qwen_native_audio_q1.py:156-182: prefix_start 4, 3 real prefix
    # frames, audio_start 7, query at audio frame 3 (position 10)
    ps, frames = 4, 3
    as_ = ps + frames
    total = as_ + 8 + 1
    qpos = as_ + frames
    m = O.talker_mask(1, total, ps, as_, as_ - 1, qpos, mode=0)[0]
    assert np.all(m[ps:as_] == 0)
    assert np.all(m[as_:qpos + 1] == 0)
    assert m[qpos + 1] == FLOOR
    assert np.all(m[:ps] == 0)  # stable text
    assert np.all(m[qpos + 1:] == FLOOR)


def test_g0_mode_hides_prefix_from_audio_query_only():
    # test_virtual_prefix_g0_contract.py:22-33: prefix_start 2, audio_start 8,
    # positions [2, 8], visible_prefix_end 0 -> prefix position 2
    m = O.talker_mask(2, 12, 2, 8, 2, 8, mode=1)
    assert m[0, 2] == 0.0
    assert m[1, 0] == 0.0
    assert m[1, 2] == FLOOR
    assert m[1, 8] == 0.0
    assert np.all(m[0, 3:] == FLOOR)  # the prefix query sees no audio
    assert np.all(m[1, 3:8] == FLOOR) and np.all(m[1, 9:] == FLOOR)


def test_gated_mode_uses_visible_prefix_count_normalization():
    # test_virtual_prefix_g0_contract.py:36-43: positions [4, 10], prefix
    # frames 2..4 visible (three keys), gate -8
    m = O.talker_mask(2, 12, 2, 8, 4, 10, mode=2, visible_prefix_count=3, prefix_log_gate=-8.0)
    expected = -8.0 - math.log(3.0)
    assert m[1, 4] == float(O.round_bf16(np.array([expected], np.float32))[0])
    assert abs(m[1, 4] - expected) <= abs(expected) * 2.0 ** -8
    assert np.all(m[1, 2:5] == m[1, 4])
    assert m[1, 5] == FLOOR
    assert np.all(m[0, 2:5] == 0.0)  # the prefix query's own rows carry no gate
    assert np.all(m[1, :2] == 0.0) and np.all(m[1, 8:11] == 0.0)


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_mask_rows_against_the_kernel_formula_enumerated(mode):
    """Every (prefix_start, prefix_pos, audio_start, audio_pos) of a 10-key
    cache: the prefix row is the plain causal range [0, prefix_pos]; the
    audio row is stable + audio + (prefix unless mode 1)."""
    L = 10
    for ps in range(0, 4):
        for pp in range(ps, 6):
            for as_ in range(pp + 1, 8):
                for ap in range(as_, L):
                    j = O.talker_mask(2, L, ps, as_, pp, ap, mode, 2, -1.0)
                    a = O.talker_mask(1, L, ps, as_, pp, ap, mode, 2, -1.0)
                    keys = np.arange(L)
                    assert np.array_equal(j[0] == 0, keys <= pp)
                    want = (keys < ps) | ((keys >= as_) & (keys <= ap))
                    if mode != 1:
                        want |= (keys >= ps) & (keys <= pp)
                    assert np.array_equal(j[1] > FLOOR, want)
                    assert np.array_equal(a[0], j[1])


def _case(seed, hq=4, hkv=2, d=16, L=24):
    rng = np.random.default_rng(seed)
    q = O.round_bf16(rng.standard_normal((hq, 2, d)).astype(np.float32))
    k = O.round_bf16(rng.standard_normal((hkv, L, d)).astype(np.float32))
    v = O.round_bf16(rng.standard_normal((hkv, L, d)).astype(np.float32))
    return q, k, v


def test_all_prefix_visible_reduces_to_causal_attention():
    q, k, v = _case(1)
    ps, as_, ap = 5, 11, 17
    pp = as_ - 1
    m = O.talker_mask(2, k.shape[1], ps, as_, pp, ap, mode=0)
    got = O.attend_masked(q, k, v, m, 0.3)
    want = O.attend(q, k, v, np.array([pp, ap]), 0.3)  # causal rows at the two positions
    np.testing.assert_allclose(got, want, atol=1e-6)


def test_hidden_prefix_equals_attention_over_the_key_subset():
    q, k, v = _case(2)
    ps, pp, as_, ap = 3, 7, 12, 20
    m = O.talker_mask(1, k.shape[1], ps, as_, pp, ap, mode=1)
    got = O.attend_masked(q[:, 1:], k, v, m, 0.25)
    keep = np.r_[0:ps, as_:ap + 1]
    want = O.attend(q[:, 1:], k[:, keep], v[:, keep], np.array([ap]), 0.25, key_positions=keep)
    np.testing.assert_allclose(got, want, atol=1e-6)


@pytest.mark.parametrize("gate,count", [(-8.0, 3), (2.5, 1), (-0.7, 5)])
def test_gate_scales_the_prefix_partition_by_exp_gate(gate, count):
    """softmax with +g on a key subset B = (e^{lse_A} o_A + e^{g + lse_B} o_B) /
    (e^{lse_A} + e^{g + lse_B}), o_X the attention over X alone."""
    q, k, v = _case(3)
    ps, pp, as_, ap = 4, 9, 13, 21
    scale = 0.3
    m = O.talker_mask(1, k.shape[1], ps, as_, pp, ap, 2, count, gate)
    got = O.attend_masked(q[:, 1:], k, v, m, scale).astype(np.float64)
    g = O.talker_gate(2, count, gate)
    a_keys = np.r_[0:ps, as_:ap + 1]
    b_keys = np.arange(ps, pp + 1)
    hq, g_heads = q.shape[0], q.shape[0] // k.shape[0]
    for h in range(hq):
        kh = h // g_heads
        s = (q[h, 1].astype(np.float64) @ k[kh].T.astype(np.float64)) * scale
        la, lb = logsumexp(s[a_keys]), g + logsumexp(s[b_keys])
        oa = O.attend(q[h:h + 1, 1:], k[kh:kh + 1, a_keys], v[kh:kh + 1, a_keys], np.array([ap]), scale,
                      key_positions=a_keys)[0, 0]
        ob = O.attend(q[h:h + 1, 1:], k[kh:kh + 1, b_keys], v[kh:kh + 1, b_keys], np.array([ap]), scale,
                      key_positions=b_keys)[0, 0]
        top = max(la, lb)
        wa, wb = math.exp(la - top), math.exp(lb - top)
        np.testing.assert_allclose(got[h, 0], (wa * oa + wb * ob) / (wa + wb), atol=1e-6)


def test_attend_masked_matches_torch_sdpa_with_additive_mask():
    q, k, v = _case(4, hq=8, hkv=2, d=32, L=40)
    m = O.talker_mask(2, 40, 6, 20, 12, 33, 2, 7, -3.0)
    got = O.attend_masked(q, k, v, m, 0.17)
    g = q.shape[0] // k.shape[0]
    kt = torch.from_numpy(np.repeat(k, g, axis=0)).double()[None]
    vt = torch.from_numpy(np.repeat(v, g, axis=0)).double()[None]
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).double()[None], kt, vt, attn_mask=torch.from_numpy(m).double()[None, None], scale=0.17)
    np.testing.assert_allclose(got, ref[0].numpy(), atol=1e-6)


def _kat_failures(build) -> list[str]:
    """Which reference known answers a mask builder (talker_mask's signature) violates."""
    bad = []
    m = build(1, 16, 4, 7, 6, 10, 0)[0]
    if not (np.all(m[4:11] == 0) and m[11] == FLOOR):
        bad.append("q1 suffix")
    m = build(2, 12, 2, 8, 2, 8, 1)
    if not (m[0, 2] == 0 and m[1, 0] == 0 and m[1, 2] == FLOOR and m[1, 8] == 0):
        bad.append("g0")
    m = build(2, 12, 2, 8, 4, 10, 2, 3, -8.0)
    if not (abs(m[1, 4] - (-8.0 - math.log(3.0))) <= 0.04 and m[1, 5] == FLOOR and m[0, 4] == 0):
        bad.append("gated")
    return bad


def test_planted_mistakes_fail_a_known_answer():
    """Plausible slips planted in a copy of the oracle each break a KAT."""
    assert _kat_failures(O.talker_mask) == []

    def gate_on_both_rows(rows, L, ps, as_, pp, ap, mode, cnt=0, gate=-8.0):
        m = O.talker_mask(rows, L, ps, as_, pp, ap, mode, cnt, gate)
        if mode == 2:
            m[:, ps:pp + 1] = O.talker_gate(mode, cnt, gate)
        return m

    def audio_end_exclusive(rows, L, ps, as_, pp, ap, mode, cnt=0, gate=-8.0):
        return O.talker_mask(rows, L, ps, as_, pp, ap - 1, mode, cnt, gate)

    def count_not_normalised(rows, L, ps, as_, pp, ap, mode, cnt=0, gate=-8.0):
        m = O.talker_mask(rows, L, ps, as_, pp, ap, mode, cnt, gate)
        if mode == 2:
            m[-1, ps:pp + 1] = gate
        return m

    def mode1_hides_prefix_row_too(rows, L, ps, as_, pp, ap, mode, cnt=0, gate=-8.0):
        m = O.talker_mask(rows, L, ps, as_, pp, ap, mode, cnt, gate)
        if mode == 1:
            m[:, ps:pp + 1] = FLOOR
        return m

    for planted in (gate_on_both_rows, audio_end_exclusive, count_not_normalised, mode1_hides_prefix_row_too):
        assert _kat_failures(planted), planted.__name__
