"""kvrt — MI355X-native (gfx950) KV-cache runtime for duplex decode loops.

Host side in Python on PyTorch-ROCm; compute in hand-written HIP kernels
behind the C ABI of include/kvrt.h (libkvrt.so, built in-tree).

* ``kvrt.runtime`` — ``KVRuntime``: the C-ABI context (slots x layers).
* ``kvrt.cache`` — ``KVRTCache``: one slot as a transformers Cache; gather/attend.
* ``kvrt.kv_cache`` / ``kvrt.thinker_cache`` — the reference's
  duplex_kernel/kv_cache.py and thinker_cache.py API over kvrt storage.
* ``kvrt.talker`` — HF talker cache import and the Q1 position counter.
"""
from .cache import KVRTCache, KVRTCacheLayer, append_attend, attend, attend_padded, gather
from .runtime import KVRTError, KVRuntime, LayerSpec, TalkerMask, attend_tensors, copy_rows

__all__ = ["KVRTCache", "KVRTCacheLayer", "KVRTError", "KVRuntime", "LayerSpec", "TalkerMask", "append_attend", "attend",
           "attend_padded", "attend_tensors", "copy_rows", "gather"]
