"""PagedSessionCache: the SessionKvCache seam (src/kv_cache.rs:431-446) over
device pages.

One session is one sequence of a SequenceManager; layer l keeps its K/V in
pools[l] and every layer shares the sequence's block table.  The five trait
operations keep their meaning:

    seq_len(layer)      tokens stored for the layer (0 when empty)
    save(layer, k, v)   the layer's cache becomes the rows of k / v (f32
                        [n, n_kv_heads, head_dim]); rows already stored are
                        taken as unchanged (the decode loop grows a cache by
                        concatenation, src/model.rs:569), so only new rows are
                        written, and a shorter k shortens the layer
    load(layer)         the dense [seq, n_kv_heads, head_dim] view of
                        LayerCache::Attention (src/kv_cache.rs:121-122)
    clear()             every layer empty, every block released
    truncate_to(pos)    every layer keeps at most pos tokens (O(1) rollback,
                        src/kv_cache.rs:364-383); blocks past pos are released

plus append(layer, k_new, v_new) (the reshape-and-cache that replaces the
Tensor::cat) and fork() (fork_sequence with copy-on-write of shared blocks).
"""
from __future__ import annotations

import ctypes

from . import _lib
from .pool import _dev, _stream_ptr, _torch


class PagedSessionCache:
    def __init__(self, manager, pools, _handle=None):
        L = _lib.load()
        self.manager = manager
        self.pools = list(pools)
        if _handle is not None:
            self._h = _handle
            return
        arr = (ctypes.c_void_p * len(self.pools))(*[p.handle.value for p in self.pools])
        h = ctypes.c_void_p()
        _lib.check(L.air_kv_session_create(manager._h, arr, len(self.pools), ctypes.byref(h)),
                   "air_kv_session_create")
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            _lib.load().air_kv_session_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def seq_id(self):
        out = ctypes.c_uint32()
        _lib.check(_lib.load().air_kv_session_seq_id(self._h, ctypes.byref(out)))
        return out.value

    def seq_len(self, layer):
        out = ctypes.c_int64()
        _lib.check(_lib.load().air_kv_session_seq_len(self._h, layer, ctypes.byref(out)), "seq_len")
        return out.value

    def _rows(self, layer, k, v):
        torch = _torch()
        p = self.pools[layer]
        if k.dim() != 3 or k.shape[1:] != (p.n_kv_heads, p.head_dim) or v.shape != k.shape:
            raise ValueError("k / v must be [n, n_kv_heads, head_dim] of the layer's pool")
        _dev(k, torch.float32, "k")
        _dev(v, torch.float32, "v")
        return k.shape[0]

    def append(self, layer, k, v, stream=None):
        n = self._rows(layer, k, v)
        rc = _lib.load().air_kv_session_append(self._h, _stream_ptr(stream), layer,
                                               ctypes.c_void_p(k.data_ptr()),
                                               ctypes.c_void_p(v.data_ptr()), n)
        if rc == _lib.AIR_KV_E_OOM:
            raise MemoryError(_lib.last_error())
        _lib.check(rc, "append")

    def save(self, layer, k, v, stream=None):
        n = self._rows(layer, k, v)
        rc = _lib.load().air_kv_session_save(self._h, _stream_ptr(stream), layer,
                                             ctypes.c_void_p(k.data_ptr()),
                                             ctypes.c_void_p(v.data_ptr()), n)
        if rc == _lib.AIR_KV_E_OOM:
            raise MemoryError(_lib.last_error())
        _lib.check(rc, "save")

    def load(self, layer, dtype=None, stream=None):
        """(k, v) device tensors [seq, n_kv_heads, head_dim] (float32 for f32
        and 1-byte pools, bfloat16 for bf16 pools unless dtype is given)."""
        torch = _torch()
        p = self.pools[layer]
        if dtype is None:
            dtype = torch.bfloat16 if p.dtype == _lib.BF16 else torch.float32
        n = self.seq_len(layer)
        k = torch.empty(n, p.n_kv_heads, p.head_dim, dtype=dtype, device="cuda")
        v = torch.empty_like(k)
        odt = _lib.F32 if dtype == torch.float32 else _lib.BF16
        _lib.check(_lib.load().air_kv_session_load(self._h, _stream_ptr(stream), layer,
                                                   ctypes.c_void_p(k.data_ptr()),
                                                   ctypes.c_void_p(v.data_ptr()), odt), "load")
        return k, v

    def clear(self):
        _lib.check(_lib.load().air_kv_session_clear(self._h), "clear")

    def truncate_to(self, pos):
        _lib.check(_lib.load().air_kv_session_truncate_to(self._h, pos), "truncate_to")

    def fork(self):
        h = ctypes.c_void_p()
        rc = _lib.load().air_kv_session_fork(self._h, ctypes.byref(h))
        if rc == _lib.AIR_KV_E_OOM:
            raise MemoryError(_lib.last_error())
        _lib.check(rc, "fork")
        return PagedSessionCache(self.manager, self.pools, _handle=h)

    def memory_usage(self):
        out = ctypes.c_size_t()
        _lib.check(_lib.load().air_kv_session_memory_usage(self._h, ctypes.byref(out)))
        return out.value
