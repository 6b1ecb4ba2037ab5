"""ctypes binding of libkvrt.so (declarations in include/kvrt.h).

Loading fails loudly when the library is missing: there is no CPU or
PyTorch fallback behind any kvrt entry point.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int32, c_int64, c_uint32, c_uint64, c_void_p

from ._build import LIB_PATH

KVRT_ABI_VERSION = 3
KVRT_MAX_RANK = 4
KVRT_MAX_ROLLOVER_ROWS = 128
KVRT_MAX_ITEMS = 64
KVRT_MAX_PREFIX_MASK = 512
KVRT_ANY_GENERATION = 0
KVRT_NOALLOC_SCRATCH_BYTES = 16 << 20

KVRT_OK = 0
KVRT_EINVAL = -1
KVRT_ESTATE = -2
KVRT_EDEVICE = -3
KVRT_EPOISONED = -4
KVRT_ENOMEM = -5
KVRT_EFAULT = -6

LAYOUT_CONTIG = 0
LAYOUT_RING = 1
LAYOUT_PAGED = 2

DT_BF16 = 0
DT_INT8 = 1
DT_FP32 = 2
DT_BOOL = 3
DT_INT32 = 4
DT_INT64 = 5

CAP_CONTIG = 1 << 0
CAP_RING = 1 << 1
CAP_PAGED = 1 << 2
CAP_INT8 = 1 << 3
CAP_FUSED_APPEND_ATTEND = 1 << 4
CAP_GATHER = 1 << 5
CAP_DEVICE_LENGTHS = 1 << 6
CAP_TENSOR_ATTEND = 1 << 7
CAP_PREFILL_MFMA = 1 << 8
CAP_TALKER_MASK = 1 << 9
CAP_PREFIX_ATTENTION = 1 << 10
CAP_SLOT_GENERATION = 1 << 11
CAP_STREAM_CONFINED = 1 << 12
CAP_ROLLBACK_POSITION = 1 << 13


class KvrtTensor(ctypes.Structure):
    _fields_ = [
        ("data", c_void_p),
        ("dtype", c_int32),
        ("ndim", c_int32),
        ("dims", c_int64 * KVRT_MAX_RANK),
        ("strides", c_int64 * KVRT_MAX_RANK),
    ]


class KvrtLayerSpec(ctypes.Structure):
    _fields_ = [
        ("layout", c_int32),
        ("dtype", c_int32),
        ("kv_heads", c_int32),
        ("head_dim", c_int32),
        ("window", c_int32),
        ("ring_rows", c_int32),
        ("shared_src", c_int32),
        ("reserved", c_int32),
    ]


# kvrt_config.decode_kernel (kvrt.h KVRT_DECODE_*)
KVRT_DECODE_AUTO, KVRT_DECODE_VALU, KVRT_DECODE_MFMA = 0, 1, 2
DECODE_KERNELS = {"auto": KVRT_DECODE_AUTO, "valu": KVRT_DECODE_VALU, "mfma": KVRT_DECODE_MFMA}
# kvrt_config.decode_merge (kvrt.h KVRT_MERGE_*)
KVRT_MERGE_AUTO, KVRT_MERGE_SEPARATE, KVRT_MERGE_LAST_WG = 0, 1, 2
DECODE_MERGES = {"auto": KVRT_MERGE_AUTO, "separate": KVRT_MERGE_SEPARATE, "last_wg": KVRT_MERGE_LAST_WG}


class KvrtConfig(ctypes.Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("n_layers", c_int32),
        ("n_slots", c_int32),
        ("capacity", c_int32),
        ("block_size", c_int32),
        ("pool_pages", c_int32),
        ("max_q", c_int32),
        ("pool_seed", c_int32),
        ("decode_wgs", c_int32),
        ("decode_kernel", c_int32),
        ("decode_merge", c_int32),
    ]


class KvrtStorage(ctypes.Structure):
    _fields_ = [("k", c_void_p), ("v", c_void_p), ("k_scale", c_void_p), ("v_scale", c_void_p)]


class KvrtCounters(ctypes.Structure):
    _fields_ = [
        ("launches", c_uint64),
        ("appended_rows", c_uint64),
        ("appended_bytes", c_uint64),
        ("attended_keys", c_uint64),
        ("attended_bytes", c_uint64),
        ("gathered_bytes", c_uint64),
        ("truncations", c_uint64),
        ("truncated_rows", c_uint64),
        ("pages_in_use", c_uint64),
        ("pages_evicted", c_uint64),
        ("mfma_decodes", c_uint64),
    ]


class KvrtSlotInfo(ctypes.Structure):
    _fields_ = [
        ("generation", c_uint64),
        ("prefix_len", c_int32),
        ("min_len", c_int32),
        ("max_len", c_int32),
        ("reserved", c_int32),
    ]


class KvrtTalkerMask(ctypes.Structure):
    _fields_ = [
        ("prefix_start", c_int32),
        ("audio_start", c_int32),
        ("prefix_position", c_int32),
        ("audio_position", c_int32),
        ("prefix_attention_mode", c_int32),
        ("visible_prefix_count", c_int32),
        ("prefix_log_gate", c_float),
    ]


# (name, restype, argtypes) of every symbol declared in include/kvrt.h.
_T = POINTER(KvrtTensor)
_I32P = POINTER(c_int32)
SIGNATURES = [
    ("kvrt_abi_version", c_uint32, []),
    ("kvrt_capabilities", c_uint64, []),
    ("kvrt_strerror", ctypes.c_char_p, [c_int32]),
    ("kvrt_create", c_int32, [POINTER(KvrtConfig), POINTER(KvrtLayerSpec), POINTER(c_void_p)]),
    ("kvrt_create_with_storage", c_int32,
     [POINTER(KvrtConfig), POINTER(KvrtLayerSpec), POINTER(KvrtStorage), POINTER(c_void_p)]),
    ("kvrt_layer_storage_bytes", c_int32,
     [POINTER(KvrtConfig), POINTER(KvrtLayerSpec), POINTER(c_uint64), POINTER(c_uint64)]),
    ("kvrt_destroy", c_int32, [c_void_p]),
    ("kvrt_bind_stream", c_int32, [c_void_p, c_void_p]),
    ("kvrt_grow_slots", c_int32, [c_void_p, c_int32, POINTER(KvrtStorage)]),
    ("kvrt_layer_storage", c_int32, [c_void_p, c_int32, POINTER(KvrtStorage)]),
    ("kvrt_import_async", c_int32, [c_void_p, c_int32, c_int32, _T, _T, c_int32]),
    ("kvrt_append_async", c_int32, [c_void_p, c_int32, c_int32, _I32P, _T, _T]),
    ("kvrt_write_positions_async", c_int32, [c_void_p, c_int32, c_int32, _I32P, _I32P, _T, _T]),
    ("kvrt_reset_slot_async", c_int32, [c_void_p, c_int32]),
    ("kvrt_set_prefix_attention_async", c_int32, [c_void_p, c_int32, _T]),
    ("kvrt_slot_info_get", c_int32, [c_void_p, c_int32, POINTER(KvrtSlotInfo)]),
    ("kvrt_gather_async", c_int32, [c_void_p, c_int32, c_int32, _I32P, _I32P, _T, _T, _T]),
    ("kvrt_append_gather_async", c_int32, [c_void_p, c_int32, c_int32, _I32P, _T, _T, _I32P, _T, _T, _T]),
    ("kvrt_truncate", c_int32, [c_void_p, c_int32, c_int32, c_int32, c_uint64, c_int32]),
    ("kvrt_reserve_async", c_int32, [c_void_p, c_int32, c_int32]),
    ("kvrt_evict", c_int32, [c_void_p, c_int32, c_int32]),
    ("kvrt_copy_prefix_async", c_int32, [c_void_p, c_int32, c_int32, c_int32, c_uint64]),
    ("kvrt_copy_session_async", c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_int32, c_uint64]),
    ("kvrt_set_layer_rope", c_int32, [c_void_p, c_int32, POINTER(c_float), c_int32, c_float]),
    ("kvrt_rollover_async", c_int32, [c_void_p, c_int32, c_int32, c_int32, c_uint64]),
    ("kvrt_attend_decode_async", c_int32, [c_void_p, c_int32, c_int32, _I32P, _T, _T, c_float]),
    ("kvrt_append_attend_async", c_int32, [c_void_p, c_int32, c_int32, _I32P, _T, _T, _T, _T, c_float]),
    ("kvrt_attend_prefill_async", c_int32, [c_void_p, c_int32, c_int32, _I32P, _T, _T, c_float]),
    ("kvrt_attend_talker_async", c_int32,
     [c_void_p, c_int32, c_int32, _I32P, _T, _T, c_float, POINTER(KvrtTalkerMask)]),
    ("kvrt_attend_tensors_async", c_int32, [_T, _T, _T, c_void_p, _T, _T, c_float, c_int32, c_void_p]),
    ("kvrt_attend_tensors_noalloc_async", c_int32, [_T, _T, _T, c_void_p, _T, _T, c_float, c_int32, c_void_p]),
    ("kvrt_tensors_status", c_int32, [c_void_p]),
    ("kvrt_copy_rows_async", c_int32, [_T, _T, c_int64, c_void_p]),
    ("kvrt_session_state", c_int32, [c_void_p, c_int32, c_int32, _I32P]),
    ("kvrt_sync_lengths", c_int32, [c_void_p]),
    ("kvrt_get_counters", c_int32, [c_void_p, POINTER(KvrtCounters)]),
    ("kvrt_health", c_int32, [c_void_p]),
    ("kvrt_debug_inject_failure", c_int32, [c_void_p]),
]

_lib = None


def load() -> ctypes.CDLL:
    """Load libkvrt.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"libkvrt.so not found at {LIB_PATH}; build it first "
            "(python -c 'import __graft_entry__ as g; g.build()')"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.kvrt_abi_version() != KVRT_ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI {lib.kvrt_abi_version()}, this binding needs {KVRT_ABI_VERSION}; "
                           "rebuild it")
    _lib = lib
    return lib


def strerror(code: int) -> str:
    return load().kvrt_strerror(int(code)).decode()
