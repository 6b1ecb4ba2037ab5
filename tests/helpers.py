"""Shared helpers of the test suite: seeded inputs and tensor <-> oracle glue."""
from __future__ import annotations

import numpy as np
import torch


def randn_bf16(gen: torch.Generator, shape, scale: float = 1.0) -> torch.Tensor:
    """Seeded N(0,1)*scale drawn in fp32 on the CPU, rounded to bf16 (RNE)."""
    x = torch.randn(*shape, generator=gen, dtype=torch.float32) * scale
    return x.to(torch.bfloat16)


def to_np(t: torch.Tensor) -> np.ndarray:
    """Exact float32 copy of a (bf16 / fp32) tensor on the host."""
    return t.detach().to("cpu", torch.float32).numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bf16 bit patterns of a bf16 tensor."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def np_bf16_bits(x: np.ndarray) -> np.ndarray:
    from oracle.kv_oracle import f32_to_bf16_bits

    return f32_to_bf16_bits(x)
