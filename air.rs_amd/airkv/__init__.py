"""airkv -- MI355X-native paged KV-cache path (host side of libairkv.so).

Mirrors the reference's paged-KV interface (src/paged_attention.rs,
src/kv_swap.rs, src/flash_decode.rs) over the C ABI in include/air_kv.h.  The
compute runs in hand-written gfx950 HIP kernels; importing this package does
not touch the GPU.
"""
from ._lib import (AIR_KV_E_HIP, AIR_KV_E_INVALID_ARG, AIR_KV_E_NOT_FOUND, AIR_KV_E_OOM,
                   AIR_KV_E_STATE, AIR_KV_OK, BF16, F32, FP8, INT8, LAYOUT_HEAD_MAJOR,
                   LAYOUT_TOKEN_MAJOR, LIB_PATH, SIGNATURES, AirKvError, last_error, load)
from . import kv_compress
from .kv_swap import KvSwapManager, pool_callbacks
from .paged_attention import (BLOCK_SIZE, MAX_BLOCKS, BlockAllocator, BlockTable,
                              SequenceManager, num_blocks_for_tokens)
from .pool import KvPool, wire_int8_quantize
from .session import PagedSessionCache
from . import pd_wire
from .pd_wire import KvBlock

__all__ = [
    "AIR_KV_OK", "AIR_KV_E_INVALID_ARG", "AIR_KV_E_OOM", "AIR_KV_E_NOT_FOUND", "AIR_KV_E_HIP",
    "AIR_KV_E_STATE", "F32", "BF16", "INT8", "FP8", "LAYOUT_HEAD_MAJOR", "LAYOUT_TOKEN_MAJOR",
    "LIB_PATH", "SIGNATURES", "AirKvError", "last_error", "load", "KvSwapManager",
    "pool_callbacks", "BLOCK_SIZE", "MAX_BLOCKS", "BlockAllocator", "BlockTable",
    "SequenceManager", "num_blocks_for_tokens", "KvPool", "PagedSessionCache", "wire_int8_quantize",
    "kv_compress", "pd_wire", "KvBlock",
]
