#!/usr/bin/env python3
"""Writes the golden vectors of tests/golden/ (test infrastructure).

* ``attention_small.npz`` — tiny GQA decode-attention cases. Inputs are
  seeded N(0,1) draws rounded to bf16 (stored as uint16 bit patterns);
  expected outputs are float64 from the pure-Python brute force
  ``oracle.kv_oracle.attend_bruteforce`` (plain loops, math.exp), which is
  independent of the vectorised numpy oracle the tests check against it.
  head_dim is 64 so that the GPU kernel can run the same cases.
* ``attention_prefix_small.npz`` — the same kind of cases under a listener
  prefix-attention mask (key k < P visible only where mask[k] != 0): the
  canonical 34-position mask, a seeded random mask under a sliding window,
  and a mask that leaves a single visible key.
* ``int8_small.npz`` — per-row symmetric int8 quantisation worked out with
  Python's own ``round`` (round half to even) and explicit clamping, on rows
  that include exact ties, an all-zero row and a row with one huge value.
* ``reference_kats.json`` — the known answers the reference's own tests and
  static asserts hold for this path, as data (file:line of each source).

Run from the repo root: ``python tests/golden/make_golden.py``.
"""
from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.kv_oracle import attend_bruteforce  # noqa: E402

OUT = Path(__file__).resolve().parent

# (name, Hq, Hkv, D, L, Q, window, scale, seed)
ATTN_CASES = [
    ("gqa2_global_q1", 4, 2, 64, 37, 1, 0, 0.125, 101),
    ("gqa8_sliding_q2", 8, 1, 64, 40, 2, 16, 0.125, 102),
    ("mha_short_q2", 2, 2, 64, 5, 2, 0, 0.3, 103),
    ("single_key", 4, 1, 64, 1, 1, 0, 0.125, 104),
    ("gqa4_window1", 4, 1, 64, 9, 1, 1, 0.125, 105),
]


# (name, Hq, Hkv, D, L, Q, window, scale, seed, mask kind, P)
PREFIX_CASES = [
    ("canonical34_q2", 8, 1, 64, 40, 2, 0, 0.125, 201, "canonical", 34),
    ("canonical34_first_query", 4, 1, 64, 35, 1, 0, 0.125, 202, "canonical", 34),
    ("random40_sliding24_q2", 8, 2, 64, 60, 2, 24, 0.125, 203, "random", 40),
    ("single_prefix_key", 4, 1, 64, 12, 1, 0, 0.125, 204, "single5", 12),
]


def prefix_mask(kind: str, p: int, gen: torch.Generator) -> list[int]:
    if kind == "canonical":  # kernel_set_canonical_prefix_mask: positions 0 and p - 1
        return [1 if i in (0, p - 1) else 0 for i in range(p)]
    if kind == "random":
        return [int(x) for x in torch.randint(0, 2, (p,), generator=gen).tolist()]
    return [1 if i == 5 else 0 for i in range(p)]


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def make_attention() -> None:
    arrays = {}
    for name, hq, hkv, d, n_keys, qn, window, scale, seed in ATTN_CASES:
        gen = torch.Generator().manual_seed(seed)
        k = torch.randn((hkv, n_keys, d), generator=gen).to(torch.bfloat16)
        v = torch.randn((hkv, n_keys, d), generator=gen).to(torch.bfloat16)
        q = (0.5 * torch.randn((hq, qn, d), generator=gen)).to(torch.bfloat16)
        pos = list(range(n_keys - qn, n_keys))
        out = attend_bruteforce(q.float().tolist(), k.float().tolist(), v.float().tolist(), pos, scale, window)
        arrays[f"{name}.q"] = bf16_bits(q)
        arrays[f"{name}.k"] = bf16_bits(k)
        arrays[f"{name}.v"] = bf16_bits(v)
        arrays[f"{name}.out"] = np.asarray(out, dtype=np.float64)
        arrays[f"{name}.meta"] = np.asarray([hq, hkv, d, n_keys, qn, window], dtype=np.int64)
        arrays[f"{name}.scale"] = np.asarray([scale], dtype=np.float64)
    np.savez_compressed(OUT / "attention_small.npz", **arrays)


def make_attention_prefix() -> None:
    arrays = {}
    for name, hq, hkv, d, n_keys, qn, window, scale, seed, kind, plen in PREFIX_CASES:
        gen = torch.Generator().manual_seed(seed)
        k = torch.randn((hkv, n_keys, d), generator=gen).to(torch.bfloat16)
        v = torch.randn((hkv, n_keys, d), generator=gen).to(torch.bfloat16)
        q = (0.5 * torch.randn((hq, qn, d), generator=gen)).to(torch.bfloat16)
        mask = prefix_mask(kind, plen, gen)
        pos = list(range(n_keys - qn, n_keys))
        out = attend_bruteforce(q.float().tolist(), k.float().tolist(), v.float().tolist(), pos, scale, window,
                                prefix_attention=mask)
        arrays[f"{name}.q"] = bf16_bits(q)
        arrays[f"{name}.k"] = bf16_bits(k)
        arrays[f"{name}.v"] = bf16_bits(v)
        arrays[f"{name}.mask"] = np.asarray(mask, dtype=np.int64)
        arrays[f"{name}.out"] = np.asarray(out, dtype=np.float64)
        arrays[f"{name}.meta"] = np.asarray([hq, hkv, d, n_keys, qn, window], dtype=np.int64)
        arrays[f"{name}.scale"] = np.asarray([scale], dtype=np.float64)
    np.savez_compressed(OUT / "attention_prefix_small.npz", **arrays)


def quantise_row(row: list[float]) -> tuple[list[int], float]:
    amax = max(abs(x) for x in row)
    scale = float(np.float32(amax) / np.float32(127.0))
    if amax == 0.0:
        return [0] * len(row), scale
    out = []
    for x in row:
        r = round(float(np.float32(x) / np.float32(scale)))  # Python rounds half to even
        out.append(max(-127, min(127, r)))
    return out, scale


def make_int8() -> None:
    gen = torch.Generator().manual_seed(7)
    rows = torch.randn((6, 64), generator=gen).to(torch.bfloat16).float()
    rows[1] = 0.0
    rows[2, :] = 0.001
    rows[2, 0] = 1000.0          # one huge value: everything else rounds to 0
    rows[3] = torch.arange(64, dtype=torch.float32) - 31.5
    rows[3, 0] = 127.0            # amax 127 -> scale 1: every other x/scale is a .5 tie
    rows[4] = -rows[0]
    x = rows.to(torch.bfloat16)
    q, s = zip(*(quantise_row(r) for r in x.float().tolist()))
    np.savez_compressed(OUT / "int8_small.npz", x=bf16_bits(x), q=np.asarray(q, dtype=np.int8),
                        scale=np.asarray(s, dtype=np.float32))


REFERENCE_KATS = {
    "q_range_from_position": {
        "source": "native/gemma4_listener_microbatch/gemma4_listener_kernels.cuh:41-49",
        "cases": [
            {"base": 34, "q": 4, "capacity": 4096, "window": 0, "total": 38, "start": 0, "valid": True},
            {"base": 511, "q": 4, "capacity": 4096, "window": 512, "start": 0},
            {"base": 512, "q": 4, "capacity": 4096, "window": 512, "start": 1},
            {"base": 4093, "q": 4, "capacity": 4096, "window": 0, "valid": False},
        ],
    },
    "history_batch_visibility": {
        "source": "native/gemma4_listener_microbatch/test_history_batch_contract.cpp:88-103",
        "prefix": 265,
        "causal_key_limit": [[0, 266], [3, 269], [255, 521]],
        "sliding_window": 128,
        "sliding_start": [[0, 138], [255, 393]],
    },
    "sliding_capacity": {
        "source": "native/gemma4_listener/sliding_repeat_capacity_test.cpp:14-26",
        "cases": [
            {"window": 512, "max_q": 291, "max_seq_len": 16384, "capacity": 802},
            {"window": 512, "max_q": 291, "max_seq_len": 600, "capacity": 600},
        ],
    },
    "longest_common_prefix": {
        "source": "tests/kernel/test_thinker_cache_prefix.py:36-39",
        "cases": [[[11, 12, 13], [11, 12, 99, 13], 2], [[11, 12], [11, 12, 13], 2], [[], [11], 0]],
    },
    "static_prefix_copy": {
        "source": "tests/kernel/test_thinker_cache_prefix.py:14-66",
        "layers": 2, "kv_heads": 2, "head_dim": 4, "max_cache_len": 8, "source_len": 5, "copy": 3,
        "copied_bytes": 384, "dtype": "float32",
    },
    "thinker_bucket": {
        "source": "tests/kernel/test_thinker_cache_buckets.py:13-36",
        "cases": [[384, 128, 512], [385, 128, 1024], [896, 128, 1024], [897, 128, 2048], [1920, 128, 2048],
                  [1921, 128, 4096], [3968, 128, 4096]],
        "overflow": [4001, 128, 4129],
    },
    "audio_q1_counter": {
        "source": "tests/kernel/test_qwen_native_audio_q1.py:267-277",
        "start": 127, "frames": 40,
    },
    "canonical_prefix_mask": {
        "source": "native/gemma4_listener_microbatch/gemma4_listener_kernels.cuh:111-118 "
                  "(kernel_set_canonical_prefix_mask), generated_topology.h:22 (GEMMA4_CANONICAL_PREFIX_LEN), "
                  "duplex_kernel/listener.py:1983-1988 (BOS + 32 slots + BOA)",
        "length": 34, "visible": [0, 33],
    },
    "slot_kv_cache": {
        "source": "tests/kernel/test_future_prefix_slot_kv_cache.py:24-86",
        "joint_writes": [[[0, 1], 2], [[2, 4], 5], [[3, 5], 6]],
        "max_cache_len": 16,
        "out_of_range": [-1, 8], "out_of_range_capacity": 8,
    },
}


def main() -> None:
    make_attention()
    make_attention_prefix()
    make_int8()
    (OUT / "reference_kats.json").write_text(json.dumps(REFERENCE_KATS, indent=1) + "\n")
    print("golden vectors written to", OUT)


if __name__ == "__main__":
    main()
