"""Python mirror of the reference's paged block manager over the C ABI.

Names and behaviour follow src/paged_attention.rs so that tests read like the
reference's own: ``BlockAllocator.allocate`` returns ``None`` when the pool
is exhausted (the reference's ``Option``), ``SequenceManager.append_token``
raises ``KeyError`` / ``MemoryError`` where the reference returns
``Err("sequence not found")`` / ``Err("out of memory ...")``.  Everything is
computed by the C++ allocator in libairkv.so.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import AIR_KV_E_NOT_FOUND, AIR_KV_E_OOM, AIR_KV_E_STATE, AirKvError

BLOCK_SIZE = 16    # src/paged_attention.rs:40
MAX_BLOCKS = 4096  # src/paged_attention.rs:45


def _order_ptr(free_order, capacity):
    if free_order is None:
        return None, None
    arr = np.ascontiguousarray(free_order, dtype=np.uint32)
    if arr.shape != (capacity,):
        raise ValueError("free_order must have one entry per block")
    return arr, arr.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def _raise_for(rc, what):
    if rc == AIR_KV_E_NOT_FOUND:
        raise KeyError(_lib.last_error())
    if rc == AIR_KV_E_OOM:
        raise MemoryError(_lib.last_error())
    _lib.check(rc, what)


def num_blocks_for_tokens(n_tokens: int, block_size: int = BLOCK_SIZE) -> int:
    return int(_lib.check(_lib.load().air_num_blocks_for_tokens(n_tokens, block_size)))


class BlockAllocator:
    """src/paged_attention.rs:89-196."""

    def __init__(self, capacity: int, block_size: int = BLOCK_SIZE, free_order=None, _handle=None,
                 _owner=None):
        L = _lib.load()
        self._owner = _owner
        if _handle is not None:
            self._h = _handle
            self._owned = False
            return
        h = ctypes.c_void_p()
        _keep, ptr = _order_ptr(free_order, capacity)
        _lib.check(L.air_block_allocator_create(capacity, block_size, ptr, ctypes.byref(h)),
                   "BlockAllocator")
        self._h = h
        self._owned = True

    def __del__(self):
        if getattr(self, "_owned", False) and self._h:
            _lib.load().air_block_allocator_destroy(self._h)
            self._h = None

    def allocate(self):
        out = ctypes.c_uint32()
        rc = _lib.load().air_block_allocator_allocate(self._h, ctypes.byref(out))
        if rc == AIR_KV_E_OOM:
            return None
        _lib.check(rc, "allocate")
        return out.value

    def share(self, block):
        _lib.check(_lib.load().air_block_allocator_share(self._h, block), "share")

    def release(self, block):
        _lib.check(_lib.load().air_block_allocator_release(self._h, block), "release")

    def ref_count(self, block):
        out = ctypes.c_uint32()
        _lib.check(_lib.load().air_block_allocator_ref_count(self._h, block, ctypes.byref(out)))
        return out.value

    def num_free_blocks(self):
        return _lib.check(_lib.load().air_block_allocator_num_free(self._h))

    def num_used_blocks(self):
        return _lib.check(_lib.load().air_block_allocator_num_used(self._h))

    def cow_write(self, block):
        out = ctypes.c_uint32()
        rc = _lib.load().air_block_allocator_cow_write(self._h, block, ctypes.byref(out))
        if rc == AIR_KV_E_OOM:
            return None
        _lib.check(rc, "cow_write")
        return out.value

    def append_token(self, block):
        full = ctypes.c_int32()
        rc = _lib.load().air_block_allocator_append_token(self._h, block, ctypes.byref(full))
        if rc == AIR_KV_E_STATE:
            raise AssertionError("cannot append to a full block")
        _lib.check(rc, "append_token")
        return bool(full.value)

    def block_info(self, block):
        n, f = ctypes.c_int32(), ctypes.c_int32()
        _lib.check(_lib.load().air_block_allocator_block_info(self._h, block, ctypes.byref(n),
                                                               ctypes.byref(f)))
        return n.value, bool(f.value)

    def can_allocate(self, n):
        return bool(_lib.check(_lib.load().air_block_allocator_can_allocate(self._h, n)))

    @staticmethod
    def num_blocks_for_tokens(n_tokens, block_size=BLOCK_SIZE):
        return num_blocks_for_tokens(n_tokens, block_size)

    def utilization(self):
        return float(_lib.load().air_block_allocator_utilization(self._h))


class BlockTable:
    """Snapshot of a sequence's table (src/paged_attention.rs:202-235)."""

    def __init__(self, seq_id, physical_blocks, num_tokens, block_size):
        self.seq_id = seq_id
        self.physical_blocks = list(physical_blocks)
        self.num_tokens = num_tokens
        self.block_size = block_size

    @staticmethod
    def logical_block_for_token(pos, block_size=BLOCK_SIZE):
        return pos // block_size

    def physical_block_for_token(self, pos):
        return self.physical_blocks[pos // self.block_size]

    def num_logical_blocks(self):
        return len(self.physical_blocks)

    def last_block_offset(self):
        return self.num_tokens % self.block_size


class SequenceManager:
    """src/paged_attention.rs:243-382."""

    def __init__(self, capacity, block_size=BLOCK_SIZE, free_order=None, _handle=None, _owner=None):
        L = _lib.load()
        self.block_size = block_size
        self._owner = _owner
        if _handle is not None:
            self._h = _handle
            self._owned = False
        else:
            h = ctypes.c_void_p()
            _keep, ptr = _order_ptr(free_order, capacity)
            _lib.check(L.air_seq_manager_create(capacity, block_size, ptr, ctypes.byref(h)),
                       "SequenceManager")
            self._h = h
            self._owned = True
        self.allocator = BlockAllocator(0, block_size, _handle=L.air_seq_manager_allocator(self._h),
                                        _owner=self)

    def __del__(self):
        if getattr(self, "_owned", False) and self._h:
            _lib.load().air_seq_manager_destroy(self._h)
            self._h = None

    def create_sequence(self):
        out = ctypes.c_uint32()
        _lib.check(_lib.load().air_seq_create(self._h, ctypes.byref(out)))
        return out.value

    def append_token(self, seq):
        out = ctypes.c_uint32()
        _raise_for(_lib.load().air_seq_append_token(self._h, seq, ctypes.byref(out)), "append_token")
        return out.value

    def append_slots(self, seq, n):
        """n append_token calls; returns the int64 slot of each new token."""
        slots = np.empty(n, np.int64)
        done = ctypes.c_int32()
        rc = _lib.load().air_seq_append_slots(self._h, seq, n,
                                              slots.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                              ctypes.byref(done))
        _raise_for(rc, "append_slots")
        return slots

    def fork_sequence(self, parent):
        out = ctypes.c_uint32()
        _raise_for(_lib.load().air_seq_fork(self._h, parent, ctypes.byref(out)), "fork_sequence")
        return out.value

    def free_sequence(self, seq):
        _lib.check(_lib.load().air_seq_free(self._h, seq))

    def table(self, seq):
        L = _lib.load()
        nb, nt = ctypes.c_int32(), ctypes.c_int64()
        rc = L.air_seq_table(self._h, seq, None, 0, ctypes.byref(nb), ctypes.byref(nt))
        if rc == AIR_KV_E_NOT_FOUND:
            return None
        _lib.check(rc)
        arr = (ctypes.c_uint32 * max(nb.value, 1))()
        _lib.check(L.air_seq_table(self._h, seq, arr, nb.value, ctypes.byref(nb), ctypes.byref(nt)))
        return BlockTable(seq, list(arr)[:nb.value], nt.value, self.block_size)

    def cow_last_block(self, seq):
        """Returns (old_block, new_block) or None (the reference's None)."""
        o, n = ctypes.c_uint32(), ctypes.c_uint32()
        rc = _lib.load().air_seq_cow_last_block(self._h, seq, ctypes.byref(o), ctypes.byref(n))
        if rc in (AIR_KV_E_NOT_FOUND, AIR_KV_E_OOM):
            return None
        _lib.check(rc)
        return o.value, n.value

    def truncate(self, seq, n_tokens):
        """Keep the first n_tokens tokens of seq and release the blocks past
        them (no counterpart in the reference; see air_seq_truncate)."""
        _raise_for(_lib.load().air_seq_truncate(self._h, seq, n_tokens), "truncate")

    def cow_block(self, seq, index):
        """cow_last_block for the block at table index `index`: returns
        (old_block, new_block); equal when the block was not shared."""
        o, n = ctypes.c_uint32(), ctypes.c_uint32()
        _raise_for(_lib.load().air_seq_cow_block(self._h, seq, index, ctypes.byref(o), ctypes.byref(n)),
                   "cow_block")
        return o.value, n.value

    def export_tables(self, seqs, max_blocks):
        seqs = np.ascontiguousarray(seqs, np.uint32)
        tables = np.empty((len(seqs), max_blocks), np.int32)
        lens = np.empty(len(seqs), np.int32)
        _raise_for(_lib.load().air_seq_export_tables(
            self._h, seqs.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(seqs), max_blocks,
            tables.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
            lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))), "export_tables")
        return tables, lens

    def num_sequences(self):
        return _lib.check(_lib.load().air_seq_num_sequences(self._h))

    def can_schedule(self):
        return bool(_lib.check(_lib.load().air_seq_can_schedule(self._h)))

    def swap_out(self, seq):
        t = self.table(seq)
        if t is None:
            raise KeyError("sequence not found")
        arr = (ctypes.c_uint32 * max(len(t.physical_blocks), 1))()
        n = ctypes.c_int32()
        _raise_for(_lib.load().air_seq_swap_out(self._h, seq, arr, len(t.physical_blocks),
                                                ctypes.byref(n)), "swap_out")
        return list(arr)[:n.value]

    def swap_in(self, seq, n_blocks):
        arr = (ctypes.c_uint32 * max(n_blocks, 1))()
        _raise_for(_lib.load().air_seq_swap_in(self._h, seq, n_blocks, arr), "swap_in")
        return list(arr)[:n_blocks]
