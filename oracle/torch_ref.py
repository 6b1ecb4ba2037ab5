"""PyTorch-CPU restatement of the reference's Python KV path (baseline timing).

TEST INFRASTRUCTURE ONLY: imported by ``bench.py``'s ``cpu_baseline`` leg and
by tests, never by the product. It follows the calls the reference makes on
this path, on CPU tensors:

* append: HF ``DynamicLayer.update`` = ``torch.cat([keys, k], dim=-2)``
  (transformers cache_utils.py:127-146, reached from
  duplex_kernel/kv_cache.py:95-97); sliding layers keep the last ``W - 1``
  rows after an update and return the full states
  (``DynamicSlidingWindowLayer.update``, cache_utils.py:229-261);
* truncate: ``_slice_kv`` slice + ``.contiguous()`` (kv_cache.py:205-216);
* gather: zero buffer + copy + mask (shape_stable_listener.py:28-69);
* attend: ``F.scaled_dot_product_attention`` with GQA and an explicit
  causal / sliding-window boolean mask (shape_stable_listener.py:241-251 via
  transformers sdpa_attention_forward).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


class RefLayer:
    """One HF-style dynamic cache layer on the CPU."""

    def __init__(self, window: int = 0) -> None:
        self.window = int(window)
        self.keys: torch.Tensor | None = None
        self.values: torch.Tensor | None = None
        self.cumulative_length = 0

    def update(self, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        self.cumulative_length += k.shape[-2]
        if self.keys is None:
            full_k, full_v = k, v
        else:
            full_k = torch.cat([self.keys, k], dim=-2)
            full_v = torch.cat([self.values, v], dim=-2)
        if self.window > 0:
            self.keys = full_k[:, :, -self.window + 1:, :]
            self.values = full_v[:, :, -self.window + 1:, :]
        else:
            self.keys, self.values = full_k, full_v
        return full_k, full_v

    def truncate(self, keep_len: int) -> None:
        self.keys = self.keys[:, :, :keep_len, :].contiguous()
        self.values = self.values[:, :, :keep_len, :].contiguous()
        self.cumulative_length = keep_len


def decode_mask(q_len: int, k_len: int, first_key_pos: int, window: int) -> torch.Tensor:
    """Bool [q_len, k_len] visibility of the last q_len positions."""
    total = first_key_pos + k_len
    qpos = torch.arange(total - q_len, total).unsqueeze(1)
    kpos = torch.arange(first_key_pos, total).unsqueeze(0)
    vis = kpos <= qpos
    if window > 0:
        vis &= kpos >= qpos - window + 1
    return vis


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, window: int = 0,
           first_key_pos: int = 0) -> torch.Tensor:
    """q [B, Hq, Q, D]; k, v [B, Hkv, L, D] holding positions first_key_pos..."""
    mask = decode_mask(q.shape[2], k.shape[2], first_key_pos, window)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale,
                                          enable_gqa=q.shape[1] != k.shape[1])


def pad_gather(ks: list[torch.Tensor], target: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Zero-padded [N, H, target, D] batch + bool mask [N, target]."""
    n = len(ks)
    h, d = ks[0].shape[1], ks[0].shape[3]
    out = torch.zeros((n, h, target, d), dtype=ks[0].dtype)
    mask = torch.zeros((n, target), dtype=torch.bool)
    for i, k in enumerate(ks):
        m = k.shape[2]
        out[i, :, :m].copy_(k[0])
        mask[i, :m] = True
    return out, mask
