"""Python mirror of KvSwapManager (src/kv_swap.rs:22-121) over the C ABI.

``gpu_read(block, buf)`` / ``gpu_write(block, data)`` are Python callables,
exactly the reference's closures; ``pool_callbacks(pool)`` instead hands the C
library the pool-backed adapters so the copies never leave native code.
"""
from __future__ import annotations

import ctypes

from . import _lib
from ._lib import AIR_KV_E_HIP, AIR_KV_E_NOT_FOUND, AIR_KV_E_OOM, READ_FN, WRITE_FN
from .paged_attention import BLOCK_SIZE, SequenceManager


def pool_callbacks(pool):
    """(read_fn, write_fn, ctx) binding the swap seam to a device pool."""
    L = _lib.load()
    read = ctypes.cast(L.air_kv_pool_read_cb, ctypes.c_void_p)
    write = ctypes.cast(L.air_kv_pool_write_cb, ctypes.c_void_p)
    return read, write, pool.handle


class KvSwapManager:
    def __init__(self, capacity, block_bytes, block_size=BLOCK_SIZE):
        L = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(L.air_kv_swap_create(capacity, block_size, block_bytes, ctypes.byref(h)),
                   "KvSwapManager")
        self._h = h
        self.block_bytes = block_bytes
        self.seq_mgr = SequenceManager(capacity, block_size, _handle=L.air_kv_swap_seq_manager(h),
                                       _owner=self)

    def __del__(self):
        if getattr(self, "_h", None):
            _lib.load().air_kv_swap_destroy(self._h)
            self._h = None

    # A Python callable that raises makes the C callback return
    # AIR_KV_E_HIP (evict then stops before releasing anything, restore goes
    # back to the evicted state); the exception is raised again once the C
    # call has returned.
    @staticmethod
    def _read_cb(gpu_read, errors):
        if isinstance(gpu_read, tuple):          # (fnptr, ctx) from pool_callbacks
            return gpu_read[0], gpu_read[1], None

        def tramp(_ctx, block, dst, n):
            try:
                buf = (ctypes.c_uint8 * n).from_address(ctypes.addressof(dst.contents))
                gpu_read(block, memoryview(buf).cast("B"))
                return 0
            except BaseException as e:            # noqa: BLE001 -- re-raised after the call
                errors.append(e)
                return AIR_KV_E_HIP
        fn = READ_FN(tramp)
        return ctypes.cast(fn, ctypes.c_void_p), None, fn

    @staticmethod
    def _write_cb(gpu_write, errors):
        if isinstance(gpu_write, tuple):
            return gpu_write[0], gpu_write[1], None

        def tramp(_ctx, block, src, n):
            try:
                gpu_write(block, bytes((ctypes.c_uint8 * n).from_address(ctypes.addressof(src.contents))))
                return 0
            except BaseException as e:            # noqa: BLE001 -- re-raised after the call
                errors.append(e)
                return AIR_KV_E_HIP
        fn = WRITE_FN(tramp)
        return ctypes.cast(fn, ctypes.c_void_p), None, fn

    def evict(self, seq, gpu_read):
        t = self.seq_mgr.table(seq)
        if t is None:
            raise KeyError("sequence not found")
        errors = []
        fn, ctx, _keep = self._read_cb(gpu_read, errors)
        cap = max(len(t.physical_blocks), 1)
        arr = (ctypes.c_uint32 * cap)()
        n = ctypes.c_int32()
        rc = _lib.load().air_kv_swap_evict(self._h, seq, fn, ctx, arr, cap, ctypes.byref(n))
        if errors:
            raise errors[0]
        if rc == AIR_KV_E_NOT_FOUND:
            raise KeyError(_lib.last_error())
        _lib.check(rc, "evict")
        return list(arr)[:n.value]

    def restore(self, seq, gpu_write):
        errors = []
        fn, ctx, _keep = self._write_cb(gpu_write, errors)
        cap = 1 << 16
        arr = (ctypes.c_uint32 * cap)()
        n = ctypes.c_int32()
        rc = _lib.load().air_kv_swap_restore(self._h, seq, fn, ctx, arr, cap, ctypes.byref(n))
        if errors:
            raise errors[0]
        if rc == AIR_KV_E_NOT_FOUND:
            raise KeyError(_lib.last_error())
        if rc == AIR_KV_E_OOM:
            raise MemoryError(_lib.last_error())
        _lib.check(rc, "restore")
        return list(arr)[:n.value]

    def is_evicted(self, seq):
        return bool(_lib.check(_lib.load().air_kv_swap_is_evicted(self._h, seq)))

    def evicted_count(self):
        return _lib.check(_lib.load().air_kv_swap_evicted_count(self._h))

    @property
    def cpu_bytes_used(self):
        return _lib.check(_lib.load().air_kv_swap_cpu_bytes_used(self._h))

    def maybe_evict(self, seq, free_threshold, gpu_read):
        errors = []
        fn, ctx, _keep = self._read_cb(gpu_read, errors)
        out = ctypes.c_int32()
        rc = _lib.load().air_kv_swap_maybe_evict(self._h, seq, free_threshold, fn, ctx, ctypes.byref(out))
        if errors:
            raise errors[0]
        _lib.check(rc, "maybe_evict")
        return bool(out.value)
