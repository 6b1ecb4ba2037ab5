"""kvrt — MI355X-native (gfx950) KV-cache runtime for duplex decode loops.

Host side in Python on PyTorch-ROCm; compute in hand-written HIP kernels
behind the C ABI of include/kvrt.h (libkvrt.so, built in-tree).
"""
from .runtime import KVRTError, KVRuntime, LayerSpec, attend_tensors, copy_rows

__all__ = ["KVRTError", "KVRuntime", "LayerSpec", "attend_tensors", "copy_rows"]
