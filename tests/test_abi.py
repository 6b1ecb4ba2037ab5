"""The C ABI without a GPU: libkvrt.so loads, exports every function that
include/kvrt.h declares, and its ctypes mirror has the header's struct layout
(checked against a gcc-compiled probe, as the reference checks its binding's
struct offsets against the C header: tests/kernel/
test_native_listener_microbatch_binding.py:399-436). Argument validation
paths that fail before any HIP call are exercised; no kernel runs here."""
from __future__ import annotations

import ctypes
import json
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvrt.h"


def _lib():
    from kvrt import _lib as L

    if not L.LIB_PATH.exists():
        pytest.fail("libkvrt.so is not built; run __graft_entry__.build() first")
    return L, L.load()


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvrt_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_function_is_exported_and_bound():
    L, lib = _lib()
    declared = _declared_functions()
    assert len(declared) >= 20
    bound = {name for name, _, _ in L.SIGNATURES}
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in kvrt.h but not exported"
        assert name in bound, f"{name} declared in kvrt.h but missing from the ctypes table"
    assert bound <= set(declared)


def test_version_capabilities_and_error_strings():
    L, lib = _lib()
    assert lib.kvrt_abi_version() == L.KVRT_ABI_VERSION == 3
    caps = lib.kvrt_capabilities()
    for bit in (L.CAP_CONTIG, L.CAP_RING, L.CAP_PAGED, L.CAP_INT8, L.CAP_FUSED_APPEND_ATTEND, L.CAP_GATHER,
                L.CAP_DEVICE_LENGTHS, L.CAP_TENSOR_ATTEND, L.CAP_PREFILL_MFMA, L.CAP_TALKER_MASK,
                L.CAP_PREFIX_ATTENTION, L.CAP_SLOT_GENERATION, L.CAP_STREAM_CONFINED, L.CAP_ROLLBACK_POSITION):
        assert caps & bit
    assert L.strerror(0) == "ok"
    for code in range(-1, -7, -1):
        assert L.strerror(code) not in ("ok", "unknown error")
    assert L.strerror(-99) == "unknown error"


_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "kvrt.h"
#define F(S, m) printf("\"%s.%s\": [%zu, %zu],\n", #S, #m, offsetof(S, m), sizeof(((S *)0)->m))
int main(void) {
  printf("{\n");
  F(kvrt_tensor, data); F(kvrt_tensor, dtype); F(kvrt_tensor, ndim); F(kvrt_tensor, dims); F(kvrt_tensor, strides);
  F(kvrt_layer_spec, layout); F(kvrt_layer_spec, dtype); F(kvrt_layer_spec, kv_heads); F(kvrt_layer_spec, head_dim);
  F(kvrt_layer_spec, window); F(kvrt_layer_spec, ring_rows); F(kvrt_layer_spec, shared_src);
  F(kvrt_layer_spec, reserved);
  F(kvrt_config, struct_size); F(kvrt_config, n_layers); F(kvrt_config, n_slots); F(kvrt_config, capacity);
  F(kvrt_config, block_size); F(kvrt_config, pool_pages); F(kvrt_config, max_q); F(kvrt_config, pool_seed);
  F(kvrt_config, decode_wgs); F(kvrt_config, decode_kernel); F(kvrt_config, decode_merge);
  F(kvrt_storage, k); F(kvrt_storage, v); F(kvrt_storage, k_scale); F(kvrt_storage, v_scale);
  F(kvrt_counters, launches); F(kvrt_counters, appended_rows); F(kvrt_counters, appended_bytes);
  F(kvrt_counters, attended_keys); F(kvrt_counters, attended_bytes); F(kvrt_counters, gathered_bytes);
  F(kvrt_counters, truncations); F(kvrt_counters, truncated_rows); F(kvrt_counters, pages_in_use);
  F(kvrt_counters, pages_evicted); F(kvrt_counters, mfma_decodes);
  F(kvrt_talker_mask, prefix_start); F(kvrt_talker_mask, audio_start); F(kvrt_talker_mask, prefix_position);
  F(kvrt_talker_mask, audio_position); F(kvrt_talker_mask, prefix_attention_mode);
  F(kvrt_talker_mask, visible_prefix_count); F(kvrt_talker_mask, prefix_log_gate);
  F(kvrt_slot_info, generation); F(kvrt_slot_info, prefix_len); F(kvrt_slot_info, min_len);
  F(kvrt_slot_info, max_len); F(kvrt_slot_info, reserved);
  printf("\"const.KVRT_DECODE_AUTO\": [%d, 0], \"const.KVRT_DECODE_VALU\": [%d, 0], \"const.KVRT_DECODE_MFMA\": [%d, 0],\n",
         KVRT_DECODE_AUTO, KVRT_DECODE_VALU, KVRT_DECODE_MFMA);
  printf("\"const.KVRT_MERGE_AUTO\": [%d, 0], \"const.KVRT_MERGE_SEPARATE\": [%d, 0], \"const.KVRT_MERGE_LAST_WG\": [%d, 0],\n",
         KVRT_MERGE_AUTO, KVRT_MERGE_SEPARATE, KVRT_MERGE_LAST_WG);
  printf("\"const.KVRT_MAX_PREFIX_MASK\": [%d, 0], \"const.KVRT_ANY_GENERATION\": [%d, 0], \"const.DT_INT64\": [%d, 0],\n",
         KVRT_MAX_PREFIX_MASK, (int)KVRT_ANY_GENERATION, (int)KVRT_INT64);
  printf("\"sizeof.kvrt_tensor\": [%zu, 0], \"sizeof.kvrt_layer_spec\": [%zu, 0], \"sizeof.kvrt_config\": [%zu, 0],"
         " \"sizeof.kvrt_storage\": [%zu, 0], \"sizeof.kvrt_counters\": [%zu, 0],"
         " \"sizeof.kvrt_talker_mask\": [%zu, 0], \"sizeof.kvrt_slot_info\": [%zu, 0]\n}\n",
         sizeof(kvrt_tensor), sizeof(kvrt_layer_spec), sizeof(kvrt_config), sizeof(kvrt_storage),
         sizeof(kvrt_counters), sizeof(kvrt_talker_mask), sizeof(kvrt_slot_info));
  return 0;
}
"""


def test_ctypes_structs_match_the_c_header_layout(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    L, _ = _lib()
    src = tmp_path / "probe.c"
    src.write_text(_PROBE)
    exe = tmp_path / "probe"
    subprocess.run([gcc, "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    layout = json.loads(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout)
    structs = {"kvrt_tensor": L.KvrtTensor, "kvrt_layer_spec": L.KvrtLayerSpec, "kvrt_config": L.KvrtConfig,
               "kvrt_storage": L.KvrtStorage, "kvrt_counters": L.KvrtCounters, "kvrt_talker_mask": L.KvrtTalkerMask,
               "kvrt_slot_info": L.KvrtSlotInfo}
    for key, (off, size) in layout.items():
        sname, field = key.split(".")
        if sname == "const":
            assert getattr(L, field) == off, key
            continue
        if sname == "sizeof":
            assert ctypes.sizeof(structs[field]) == off, key
            continue
        desc = getattr(structs[sname], field)
        assert (desc.offset, desc.size) == (off, size), key


def _cfg(L, **kw):
    c = L.KvrtConfig()
    c.struct_size = ctypes.sizeof(L.KvrtConfig)
    c.n_layers, c.n_slots, c.capacity, c.block_size, c.pool_pages, c.max_q = 1, 2, 64, 16, 8, 2
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def _spec(L, **kw):
    s = L.KvrtLayerSpec()
    s.layout, s.dtype, s.kv_heads, s.head_dim, s.window, s.ring_rows, s.shared_src = 0, 0, 2, 128, 0, 0, -1
    for k, v in kw.items():
        setattr(s, k, v)
    return s


def test_layer_storage_bytes_per_layout():
    L, lib = _lib()
    kv, sc = ctypes.c_uint64(), ctypes.c_uint64()
    cfg = _cfg(L)
    assert lib.kvrt_layer_storage_bytes(ctypes.byref(cfg), ctypes.byref(_spec(L)), ctypes.byref(kv), ctypes.byref(sc)) == 0
    assert (kv.value, sc.value) == (2 * 2 * 64 * 128 * 2, 0)
    ring = _spec(L, layout=L.LAYOUT_RING, window=8, ring_rows=9)
    assert lib.kvrt_layer_storage_bytes(ctypes.byref(cfg), ctypes.byref(ring), ctypes.byref(kv), ctypes.byref(sc)) == 0
    assert kv.value == 2 * 2 * 9 * 128 * 2
    paged = _spec(L, layout=L.LAYOUT_PAGED, dtype=L.DT_INT8)
    assert lib.kvrt_layer_storage_bytes(ctypes.byref(cfg), ctypes.byref(paged), ctypes.byref(kv), ctypes.byref(sc)) == 0
    assert (kv.value, sc.value) == (8 * 2 * 16 * 128, 8 * 2 * 16 * 4)


@pytest.mark.parametrize("bad", [
    dict(cfg=dict(struct_size=4)),
    dict(cfg=dict(n_slots=0)),
    dict(cfg=dict(max_q=0)),
    dict(cfg=dict(decode_wgs=-1)),
    dict(cfg=dict(decode_kernel=3)),
    dict(cfg=dict(decode_kernel=-1)),
    dict(cfg=dict(decode_merge=3)),
    dict(cfg=dict(decode_merge=-1)),
    dict(spec=dict(head_dim=96)),
    dict(spec=dict(kv_heads=0)),
    dict(spec=dict(dtype=1)),                                   # int8 needs PAGED
    dict(spec=dict(layout=1, window=8, ring_rows=8)),          # ring rows < W + max_q - 1
    dict(spec=dict(layout=2), cfg=dict(block_size=12)),        # block size not a power of two
    dict(spec=dict(layout=2), cfg=dict(block_size=1, pool_pages=1 << 24)),  # pages past 24 bits
    dict(spec=dict(layout=2, kv_heads=64), cfg=dict(block_size=1024, pool_pages=1 << 15)),  # rows past 31 bits
    dict(spec=dict(shared_src=0)),                              # a layer cannot alias itself
])
def test_create_rejects_invalid_configs_before_touching_the_device(bad):
    L, lib = _lib()
    cfg = _cfg(L, **bad.get("cfg", {}))
    spec = _spec(L, **bad.get("spec", {}))
    ctx = ctypes.c_void_p()
    assert lib.kvrt_create(ctypes.byref(cfg), ctypes.byref(spec), ctypes.byref(ctx)) == L.KVRT_EINVAL
    assert not ctx.value


def test_null_context_calls_fail_with_einval():
    L, lib = _lib()
    slots = (ctypes.c_int32 * 1)(0)
    assert lib.kvrt_truncate(None, 0, 0, 0, 0, -1) == L.KVRT_EINVAL
    assert lib.kvrt_append_async(None, 0, 1, slots, None, None) == L.KVRT_EINVAL
    assert lib.kvrt_gather_async(None, 0, 1, slots, None, None, None, None) == L.KVRT_EINVAL
    assert lib.kvrt_append_gather_async(None, 0, 1, slots, None, None, None, None, None, None) == L.KVRT_EINVAL
    assert lib.kvrt_health(None) == L.KVRT_EINVAL
    assert lib.kvrt_destroy(None) == L.KVRT_EINVAL
    assert lib.kvrt_attend_tensors_async(None, None, None, None, None, None, 1.0, 0, None) == L.KVRT_EINVAL
    assert lib.kvrt_attend_talker_async(None, 0, 1, slots, None, None, 1.0, None) == L.KVRT_EINVAL
    assert lib.kvrt_set_prefix_attention_async(None, 0, None) == L.KVRT_EINVAL
    assert lib.kvrt_slot_info_get(None, 0, None) == L.KVRT_EINVAL
    assert lib.kvrt_copy_prefix_async(None, 0, 1, 4, 0) == L.KVRT_EINVAL
    assert lib.kvrt_rollover_async(None, 0, 4, 4, 0) == L.KVRT_EINVAL
    assert lib.kvrt_bind_stream(None, None) == L.KVRT_EINVAL


def test_runtime_refuses_to_start_without_a_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from kvrt import KVRuntime, LayerSpec

    with pytest.raises(RuntimeError, match="GPU"):
        KVRuntime([LayerSpec(kv_heads=1, head_dim=128)], n_slots=1, capacity=16)
