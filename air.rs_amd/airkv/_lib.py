"""ctypes binding of libairkv.so (the C ABI declared in include/air_kv.h).

This is the binding a Python caller of the drop-in boundary writes: plain
pointers and sizes, one declaration per exported symbol.  Loading fails loudly
when the library is missing; there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libairkv.so")
# AIRKV_HOST_LIB selects the host-only build of the C ABI (the allocator,
# sequence manager and swap manager compiled under AddressSanitizer + UBSan,
# `make -C air.rs_amd asan`) for the sanitizer test: it holds no device entry
# points, and calling one raises.
HOST_LIB_PATH = os.environ.get("AIRKV_HOST_LIB")

AIR_KV_OK = 0
AIR_KV_E_INVALID_ARG = -1
AIR_KV_E_OOM = -2
AIR_KV_E_NOT_FOUND = -3
AIR_KV_E_HIP = -4
AIR_KV_E_STATE = -5

F32, BF16, INT8, FP8 = 0, 1, 2, 3
LAYOUT_HEAD_MAJOR, LAYOUT_TOKEN_MAJOR = 0, 1


class AirKvError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class PoolDesc(ctypes.Structure):
    _fields_ = [("num_blocks", ctypes.c_int64), ("block_size", ctypes.c_int32),
                ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("scale_group", ctypes.c_int32)]


READ_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint8),
                           ctypes.c_size_t)
WRITE_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint8),
                            ctypes.c_size_t)

_P = ctypes.c_void_p
_i32, _i64, _u32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
_pi32, _pi64, _pu32 = ctypes.POINTER(_i32), ctypes.POINTER(_i64), ctypes.POINTER(_u32)
_SZ = ctypes.c_size_t
_int = ctypes.c_int

# symbol -> (restype, argtypes); every function declared in include/air_kv.h
SIGNATURES = {
    "air_kv_last_error": (_int, [ctypes.c_char_p, _SZ]),
    "air_block_allocator_create": (_int, [_i64, _i32, _pu32, ctypes.POINTER(_P)]),
    "air_block_allocator_destroy": (_int, [_P]),
    "air_block_allocator_allocate": (_int, [_P, _pu32]),
    "air_block_allocator_share": (_int, [_P, _u32]),
    "air_block_allocator_release": (_int, [_P, _u32]),
    "air_block_allocator_ref_count": (_int, [_P, _u32, _pu32]),
    "air_block_allocator_num_free": (_i64, [_P]),
    "air_block_allocator_num_used": (_i64, [_P]),
    "air_block_allocator_cow_write": (_int, [_P, _u32, _pu32]),
    "air_block_allocator_append_token": (_int, [_P, _u32, _pi32]),
    "air_block_allocator_block_info": (_int, [_P, _u32, _pi32, _pi32]),
    "air_block_allocator_can_allocate": (_int, [_P, _i64]),
    "air_block_allocator_utilization": (ctypes.c_float, [_P]),
    "air_num_blocks_for_tokens": (_i64, [_i64, _i32]),
    "air_seq_manager_create": (_int, [_i64, _i32, _pu32, ctypes.POINTER(_P)]),
    "air_seq_manager_destroy": (_int, [_P]),
    "air_seq_manager_allocator": (_P, [_P]),
    "air_seq_create": (_int, [_P, _pu32]),
    "air_seq_append_token": (_int, [_P, _u32, _pu32]),
    "air_seq_append_slots": (_int, [_P, _u32, _i32, _pi64, _pi32]),
    "air_seq_fork": (_int, [_P, _u32, _pu32]),
    "air_seq_free": (_int, [_P, _u32]),
    "air_seq_cow_last_block": (_int, [_P, _u32, _pu32, _pu32]),
    "air_seq_truncate": (_int, [_P, _u32, _i64]),
    "air_seq_cow_block": (_int, [_P, _u32, _i64, _pu32, _pu32]),
    "air_seq_table": (_int, [_P, _u32, _pu32, _i32, _pi32, _pi64]),
    "air_seq_export_tables": (_int, [_P, _pu32, _i32, _i32, _pi32, _pi32]),
    "air_seq_num_sequences": (_i64, [_P]),
    "air_seq_can_schedule": (_int, [_P]),
    "air_seq_swap_out": (_int, [_P, _u32, _pu32, _i32, _pi32]),
    "air_seq_swap_in": (_int, [_P, _u32, _i32, _pu32]),
    "air_kv_swap_create": (_int, [_i64, _i32, _SZ, ctypes.POINTER(_P)]),
    "air_kv_swap_destroy": (_int, [_P]),
    "air_kv_swap_seq_manager": (_P, [_P]),
    "air_kv_swap_evict": (_int, [_P, _u32, _P, _P, _pu32, _i32, _pi32]),
    "air_kv_swap_restore": (_int, [_P, _u32, _P, _P, _pu32, _i32, _pi32]),
    "air_kv_swap_is_evicted": (_int, [_P, _u32]),
    "air_kv_swap_evicted_count": (_i64, [_P]),
    "air_kv_swap_cpu_bytes_used": (_i64, [_P]),
    "air_kv_swap_maybe_evict": (_int, [_P, _u32, _i64, _P, _P, _pi32]),
    "air_kv_pool_create": (_int, [ctypes.POINTER(PoolDesc), ctypes.POINTER(_P)]),
    "air_kv_pool_destroy": (_int, [_P]),
    "air_kv_pool_info": (_int, [_P, ctypes.POINTER(PoolDesc), ctypes.POINTER(_P), ctypes.POINTER(_P),
                                ctypes.POINTER(_P), ctypes.POINTER(_P), ctypes.POINTER(_SZ)]),
    "air_kv_append": (_int, [_P, _P, _P, _P, _P, _i32]),
    "air_kv_gather": (_int, [_P, _P, _P, _P, _P, _i32, _i32, _P, _P, _i32, _i32]),
    "air_paged_decode_workspace_size": (_int, [_P, _i32, _i32, _i32, _i32, ctypes.POINTER(_SZ)]),
    "air_paged_decode": (_int, [_P, _P, _P, _i32, _i32, _P, _P, _i32, _i32, ctypes.c_float, _i32, _P,
                                _SZ, _P, _i32]),
    "air_paged_decode_append": (_int, [_P, _P, _P, _i32, _i32, _P, _P, _P, _P, _i32, _i32, ctypes.c_float,
                                       _i32, _P, _SZ, _P, _i32]),
    "air_paged_decode_noalloc": (_int, [_P, _P, _P, _i32, _i32, _P, _P, _i32, _i32, ctypes.c_float, _i32,
                                        _P, _i32]),
    "air_paged_prefill": (_int, [_P, _P, _P, _i32, _i32, _P, _i32, _i32, _P, _P, _i32, _i32,
                                 ctypes.c_float, _P, _SZ, _P, _i32]),
    "air_paged_prefill_workspace_size": (_int, [_P, _i32, _i32, _i32, ctypes.POINTER(_SZ)]),
    "air_kv_session_create": (_int, [_P, ctypes.POINTER(_P), _i32, ctypes.POINTER(_P)]),
    "air_kv_session_destroy": (_int, [_P]),
    "air_kv_session_fork": (_int, [_P, ctypes.POINTER(_P)]),
    "air_kv_session_seq_id": (_int, [_P, _pu32]),
    "air_kv_session_seq_len": (_int, [_P, _i32, _pi64]),
    "air_kv_session_append": (_int, [_P, _P, _i32, _P, _P, _i64]),
    "air_kv_session_save": (_int, [_P, _P, _i32, _P, _P, _i64]),
    "air_kv_session_load": (_int, [_P, _P, _i32, _P, _P, _i32]),
    "air_kv_session_clear": (_int, [_P]),
    "air_kv_session_truncate_to": (_int, [_P, _i64]),
    "air_kv_session_memory_usage": (_int, [_P, ctypes.POINTER(_SZ)]),
    "air_kv_block_wire_bytes": (_int, [_P, ctypes.POINTER(_SZ)]),
    "air_kv_pack_blocks": (_int, [_P, _P, _P, _i32, _P]),
    "air_kv_unpack_blocks": (_int, [_P, _P, _P, _i32, _P]),
    "air_kv_wire_int8_quantize": (_int, [_P, _P, _i32, _SZ, _P, _P]),
    "air_kv_pack_blocks_int8": (_int, [_P, _P, _P, _i32, _P, _P]),
    "air_kv_key_compress": (_int, [_P, _P, _i32, _i64, _i32, _P, _P, _P]),
    "air_kv_key_decompress": (_int, [_P, _P, _P, _P, _i64, _i32, _P]),
    "air_kv_value_compress": (_int, [_P, _P, _i32, _i64, _i32, _P, _P, _P]),
    "air_kv_value_decompress": (_int, [_P, _P, _P, _P, _i64, _i32, _P]),
    "air_kv_qjl_compress": (_int, [_P, _P, _i32, _i64, _i32, _P, _i32, _P, _P]),
    "air_kv_qjl_scores": (_int, [_P, _P, _P, _i64, _i32, _P, ctypes.c_float, _P, _P]),
    "air_kv_compress_blocks": (_int, [_P, _P, _P, _i32, _P, _P, _P, _P, _P, _P]),
    "air_kv_qjl_compress_blocks": (_int, [_P, _P, _P, _i32, _P, _i32, _P, _P]),
    "air_kv_block_frame_bytes": (_SZ, [_SZ]),
    "air_kv_block_serialise": (_int, [_u32, ctypes.c_uint16, _P, _SZ, _P, _SZ, ctypes.POINTER(_SZ)]),
    "air_kv_block_deserialise": (_int, [_P, _SZ, _pu32, ctypes.POINTER(ctypes.c_uint16), ctypes.POINTER(_P),
                                        ctypes.POINTER(_SZ)]),
    "air_kv_block_serialise_n": (_int, [_P, ctypes.c_uint16, _P, _SZ, _i32, _P]),
    "air_kv_int8_payload_bytes": (_SZ, [_SZ]),
    "air_kv_int8_payload_serialise": (_int, [_u32, ctypes.c_uint16, ctypes.c_float, _P, _SZ, _P, _SZ,
                                             ctypes.POINTER(_SZ)]),
    "air_kv_int8_payload_deserialise": (_int, [_P, _SZ, _pu32, ctypes.POINTER(ctypes.c_uint16),
                                               ctypes.POINTER(ctypes.c_float), ctypes.POINTER(_P),
                                               ctypes.POINTER(_SZ)]),
    "air_kv_int8_payload_serialise_n": (_int, [_P, ctypes.c_uint16, _P, _P, _SZ, _i32, _P]),
    "air_kv_copy_blocks": (_int, [_P, _P, _P, _P, _i32]),
    "air_kv_read_blocks": (_int, [_P, _P, _pi32, _i32, _P]),
    "air_kv_write_blocks": (_int, [_P, _P, _pi32, _i32, _P]),
    "air_kv_pool_read_cb": (_int, [_P, _u32, _P, _SZ]),
    "air_kv_pool_write_cb": (_int, [_P, _u32, _P, _SZ]),
    "air_kv_pool_error_count": (_int, [_P, _P, _pi64, _i32]),
}

_lib = None


def load(path: str = LIB_PATH):
    """Load libairkv.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    host_only = HOST_LIB_PATH is not None
    if host_only:
        path = HOST_LIB_PATH
    if not os.path.exists(path):
        raise ImportError(f"libairkv.so not built at {path}: run __graft_entry__.build() "
                          f"(make -C air.rs_amd)")
    L = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        if host_only and not hasattr(L, name):
            continue
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    load().air_kv_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int, what: str = "") -> int:
    if rc < 0:
        raise AirKvError(rc, f"{what}: {last_error()}" if what else last_error())
    return rc
