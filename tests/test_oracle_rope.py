"""Pins the RoPE-rebase oracle (oracle.kv_oracle.rope_rebase / rope_rotate /
rope_cos_sin) and the rollover / clone restatements of the logical cache.

* The rotation arithmetic is checked bit for bit against torch's own bf16
  elementwise ops on the CPU running the HF formula ``x * cos +
  rotate_half(x) * sin`` (each op rounds to bf16), which the reference kernel
  restates (gemma4_listener_kernels.cuh:318-330: "cos/sin in FP32, cast to
  BF16, then the two pointwise BF16 multiplies and BF16 add/subtract").
* The angle tables against torch's fp32 cos / sin cast to bf16.
* The reference's own test of the rebase kernel (gemma4_listener_test.cu:
  135-210): rope(x, 100) rebased by -60 is within 0.04 of rope(x, 40), for
  D 256 / base 1e4 and D 512 / base 1e6 with 64 rotated pairs, on its inputs
  ((token*31 + dim*7) % 101 - 50) / 64.
* Closed forms: delta 0 and unrotated pairs are the identity; composing two
  rebases approximates one; norms are kept within bf16 rounding.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O


def _bf16(rng, shape, scale=1.0):
    return O.round_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def _torch_hf_rotate(x: np.ndarray, c: np.ndarray, s: np.ndarray) -> np.ndarray:
    xb = torch.from_numpy(x).to(torch.bfloat16)
    cb = torch.from_numpy(np.concatenate([c, c])).to(torch.bfloat16)
    sb = torch.from_numpy(np.concatenate([s, s])).to(torch.bfloat16)
    half = x.shape[-1] // 2
    rot = torch.cat([-xb[..., half:], xb[..., :half]], dim=-1)
    return (xb * cb + rot * sb).float().numpy()


@pytest.mark.parametrize("d,base,pairs,delta", [(256, 1e4, None, -60), (512, 1e6, 64, -16000), (128, 1e6, None, 777)])
def test_rotation_is_hf_bf16_arithmetic_bit_for_bit(d, base, pairs, delta):
    rng = np.random.default_rng(d)
    x = _bf16(rng, (40, d), 3.0)
    c, s = O.rope_cos_sin(delta, O.gemma_inv_freq(d, base, pairs))
    got = O.rope_rotate(x, c, s)
    want = _torch_hf_rotate(x, c, s)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_angle_table_matches_torch_fp32_cos_sin_in_bf16():
    inv = O.gemma_inv_freq(256, 1e4)
    for delta in (-60, -4000, 12345, 1):
        c, s = O.rope_cos_sin(delta, inv)
        f = torch.tensor(np.float32(delta)) * torch.from_numpy(inv)
        tc = torch.cos(f).to(torch.bfloat16).float().numpy()
        ts = torch.sin(f).to(torch.bfloat16).float().numpy()
        # torch's fp32 cos/sin are within an ulp of the correctly rounded values;
        # after the bf16 cast the tables agree except at rare rounding ties
        assert np.mean(c != tc) <= 0.02 and np.mean(s != ts) <= 0.02
        assert np.max(np.abs(c - tc)) <= 2.0 ** -7 and np.max(np.abs(s - ts)) <= 2.0 ** -7


def _forward_rope(x: np.ndarray, inv_freq: np.ndarray, first_pos: int) -> np.ndarray:
    """kernel_rope_bf16 (gemma4_listener_kernels.cuh:294-331) per token at
    position first_pos + t."""
    out = np.empty_like(x)
    for t in range(x.shape[0]):
        c, s = O.rope_cos_sin(float(np.float32(first_pos + t)), inv_freq)
        out[t] = O.rope_rotate(x[t], c, s)
    return out


@pytest.mark.parametrize("d,base", [(256, 10000.0), (512, 1000000.0)])
def test_reference_rebase_test_bound(d, base):
    """gemma4_listener_test.cu:135-210: 8 tokens at position 100, delta -60,
    compared with a direct rotation to position 40: max diff <= 0.04."""
    tokens = 8
    x = np.array([[((t * 31 + j * 7) % 101 - 50) / 64.0 for j in range(d)] for t in range(tokens)], np.float32)
    x = O.round_bf16(x)
    # the test rotates every token of the block at the same position
    # (kernel_rope_bf16 with q_len tokens of one head: position = base + token)
    inv = np.array([1.0 / np.float32(base) ** (np.float32(2 * p) / np.float32(d)) if p < (64 if d == 512 else d // 2)
                    else 0.0 for p in range(d // 2)], np.float32)
    old = _forward_rope(x, inv, 100)
    rebased = np.stack([O.rope_rebase(old[t], inv, -60) for t in range(tokens)])
    direct = _forward_rope(x, inv, 40)
    assert float(np.max(np.abs(rebased - direct))) <= 0.04


def test_identity_cases():
    rng = np.random.default_rng(1)
    x = _bf16(rng, (16, 512))
    inv = O.gemma_inv_freq(512, 1e6, 64)
    assert np.array_equal(O.rope_rebase(x, inv, 0), x)
    y = O.rope_rebase(x, inv, -1234)
    assert np.array_equal(y[:, 64:256], x[:, 64:256]) and np.array_equal(y[:, 256 + 64:], x[:, 256 + 64:])
    assert not np.array_equal(y[:, :64], x[:, :64])


def test_rotation_keeps_norms_and_composes():
    rng = np.random.default_rng(2)
    x = _bf16(rng, (64, 256))
    inv = O.gemma_inv_freq(256, 1e4)
    y = O.rope_rebase(x, inv, -300)
    half = 128
    n0 = x[:, :half] ** 2 + x[:, half:] ** 2
    n1 = y[:, :half] ** 2 + y[:, half:] ** 2
    assert np.max(np.abs(n1 - n0) / np.maximum(n0, 1e-3)) < 0.05
    z = O.rope_rebase(O.rope_rebase(x, inv, -100), inv, -200)
    assert np.max(np.abs(z - y)) < 0.06
    # a plausible slip — swapping the sign of the sine term — fails the inverse test
    back = O.rope_rebase(y, inv, 300)
    assert np.max(np.abs(back - x)) < 0.06
    c, s = O.rope_cos_sin(300, inv)
    slip = O.rope_rotate(y, c, -s)
    assert np.max(np.abs(slip - x)) > 0.5


def test_rollover_and_copy_prefix_on_the_logical_cache():
    rng = np.random.default_rng(3)
    cache = O.OracleCache([O.OracleLayer(2, 128)], 2)
    k, v = _bf16(rng, (2, 50, 128)), _bf16(rng, (2, 50, 128))
    cache.append(0, 0, k, v)
    cache.copy_prefix(0, 1, 0, 30)
    k1, v1 = cache.values(1, 0)
    assert np.array_equal(k1, k[:, :30]) and np.array_equal(v1, v[:, :30])
    inv = O.gemma_inv_freq(128, 1e4)
    cache.rollover(0, 0, prefix_len=10, retained=8, inv_freq=inv)
    k0, v0 = cache.values(0, 0)
    assert k0.shape[1] == 18
    assert np.array_equal(k0[:, :10], k[:, :10]) and np.array_equal(v0[:, 10:], v[:, 42:])
    assert np.array_equal(k0[:, 10:], O.rope_rebase(k[:, 42:], inv, 10 - 42))
    with pytest.raises(ValueError):
        cache.rollover(0, 0, prefix_len=10, retained=8)  # L = 18 is not > 18
