"""Restatement of the reference's paged block manager -- TEST INFRASTRUCTURE.

Pure-Python transcription of ``BlockAllocator`` / ``BlockTable`` /
``SequenceManager`` (src/paged_attention.rs:89-381) and ``KvSwapManager``
(src/kv_swap.rs:22-121), kept as literal as the language allows so that it
can serve as the checker for the product's C++ allocator.  The page size is
a constructor argument (the reference's ``BLOCK_SIZE = 16`` const,
src/paged_attention.rs:40, is the default).  Reference behaviour is kept,
including the two rough edges the product rejects instead:

* ``release`` of a block whose refcount is already 0 pushes it onto the free
  list again (src/paged_attention.rs:129-135: ``saturating_sub`` then
  ``push_back``), so the block can be handed out twice;
* ``append_token`` on a full block is an assertion (:172).
"""
from __future__ import annotations

from collections import deque

BLOCK_SIZE = 16     # src/paged_attention.rs:40
MAX_BLOCKS = 4096   # src/paged_attention.rs:45


class PhysicalBlock:
    """src/paged_attention.rs:61-80."""

    __slots__ = ("id", "num_tokens", "is_full")

    def __init__(self, bid: int):
        self.id, self.num_tokens, self.is_full = bid, 0, False


class BlockAllocator:
    """src/paged_attention.rs:89-196 (FIFO free list, refcounts, CoW metadata)."""

    def __init__(self, capacity: int, block_size: int = BLOCK_SIZE, free_order=None):
        self.block_size = block_size
        self.blocks = [PhysicalBlock(i) for i in range(capacity)]
        self.ref_counts = [0] * capacity
        # the reference initialises 0..capacity (:103-105); free_order is the
        # seeded-permutation constructor used by the configs' tests
        order = range(capacity) if free_order is None else list(free_order)
        self.free_blocks = deque(order)
        self.total_blocks = capacity

    def allocate(self):
        if not self.free_blocks:
            return None
        bid = self.free_blocks.popleft()
        self.ref_counts[bid] = 1
        self.blocks[bid].num_tokens = 0
        self.blocks[bid].is_full = False
        return bid

    def share(self, bid):
        self.ref_counts[bid] += 1

    def release(self, bid):
        self.ref_counts[bid] = max(self.ref_counts[bid] - 1, 0)
        if self.ref_counts[bid] == 0:
            self.free_blocks.append(bid)

    def ref_count(self, bid):
        return self.ref_counts[bid]

    def num_free_blocks(self):
        return len(self.free_blocks)

    def num_used_blocks(self):
        return self.total_blocks - len(self.free_blocks)

    def cow_write(self, bid):
        if self.ref_count(bid) <= 1:
            return bid
        new = self.allocate()
        if new is None:
            return None
        self.blocks[new].num_tokens = self.blocks[bid].num_tokens
        self.blocks[new].is_full = self.blocks[bid].is_full
        self.release(bid)
        return new

    def append_token(self, bid):
        blk = self.blocks[bid]
        assert not blk.is_full, "cannot append to a full block"
        blk.num_tokens += 1
        if blk.num_tokens == self.block_size:
            blk.is_full = True
        return blk.is_full

    def can_allocate(self, n):
        return len(self.free_blocks) >= n

    @staticmethod
    def num_blocks_for_tokens(n_tokens, block_size=BLOCK_SIZE):
        return -(-n_tokens // block_size)

    def utilization(self):
        return self.num_used_blocks() / self.total_blocks


class BlockTable:
    """src/paged_attention.rs:202-235."""

    def __init__(self, seq_id, block_size=BLOCK_SIZE):
        self.seq_id, self.block_size = seq_id, block_size
        self.physical_blocks = []
        self.num_tokens = 0

    def physical_block_for_token(self, pos):
        return self.physical_blocks[pos // self.block_size]

    def num_logical_blocks(self):
        return len(self.physical_blocks)

    def last_block_offset(self):
        return self.num_tokens % self.block_size


class SequenceManager:
    """src/paged_attention.rs:243-382."""

    def __init__(self, capacity, block_size=BLOCK_SIZE, free_order=None):
        self.block_size = block_size
        self.allocator = BlockAllocator(capacity, block_size, free_order)
        self.tables = {}
        self.next_seq_id = 0

    def create_sequence(self):
        sid = self.next_seq_id
        self.next_seq_id += 1
        self.tables[sid] = BlockTable(sid, self.block_size)
        return sid

    def append_token(self, sid):
        """Returns the physical block; raises KeyError / MemoryError like the
        reference's Err("sequence not found") / Err("out of memory ...")."""
        if sid not in self.tables:
            raise KeyError("sequence not found")
        t = self.tables[sid]
        needs_new = (not t.physical_blocks) or (t.last_block_offset() == 0 and t.num_tokens > 0)
        if needs_new:
            bid = self.allocator.allocate()
            if bid is None:
                raise MemoryError("out of memory — no free blocks")
            t.physical_blocks.append(bid)
        else:
            bid = t.physical_blocks[-1]
        self.allocator.append_token(bid)
        t.num_tokens += 1
        return bid

    def slot_for_append(self, sid):
        """The slot the next appended token lands in (slot arithmetic of
        :216-234): physical block of position num_tokens, times page size, plus
        its offset.  Performs the append."""
        pos = self.tables[sid].num_tokens
        bid = self.append_token(sid)
        return bid * self.block_size + pos % self.block_size

    def fork_sequence(self, parent):
        if parent not in self.tables:
            raise KeyError("parent sequence not found")
        blocks = list(self.tables[parent].physical_blocks)
        for b in blocks:
            self.allocator.share(b)
        cid = self.next_seq_id
        self.next_seq_id += 1
        t = BlockTable(cid, self.block_size)
        t.physical_blocks = blocks
        t.num_tokens = self.tables[parent].num_tokens
        self.tables[cid] = t
        return cid

    def free_sequence(self, sid):
        t = self.tables.pop(sid, None)
        if t is not None:
            for b in t.physical_blocks:
                self.allocator.release(b)

    def table(self, sid):
        return self.tables.get(sid)

    def cow_last_block(self, sid):
        t = self.tables.get(sid)
        if t is None or not t.physical_blocks:
            return None
        last = t.physical_blocks[-1]
        new = self.allocator.cow_write(last)
        if new is None:
            return None
        if new != last:
            t.physical_blocks[-1] = new
        return new

    def num_sequences(self):
        return len(self.tables)

    def can_schedule(self):
        return self.allocator.can_allocate(1)

    def swap_out(self, sid):
        if sid not in self.tables:
            raise KeyError("sequence not found")
        blocks = list(self.tables[sid].physical_blocks)
        for b in blocks:
            self.allocator.release(b)
        self.tables[sid].physical_blocks = []
        return blocks

    def swap_in(self, sid, n_blocks):
        if not self.allocator.can_allocate(n_blocks):
            raise MemoryError("out of memory — cannot swap in")
        if sid not in self.tables:
            raise KeyError("sequence not found")
        new = [self.allocator.allocate() for _ in range(n_blocks)]
        self.tables[sid].physical_blocks = list(new)
        return new


class KvSwapManager:
    """src/kv_swap.rs:22-121; the device copy is the caller's closure."""

    def __init__(self, capacity, block_bytes, block_size=BLOCK_SIZE):
        self.seq_mgr = SequenceManager(capacity, block_size)
        self.cpu_store = {}
        self.block_bytes = block_bytes
        self.cpu_bytes_used = 0

    def evict(self, sid, gpu_read):
        t = self.seq_mgr.table(sid)
        if t is None:
            raise KeyError("sequence not found")
        buf = bytearray(len(t.physical_blocks) * self.block_bytes)
        for i, b in enumerate(list(t.physical_blocks)):
            view = memoryview(buf)[i * self.block_bytes:(i + 1) * self.block_bytes]
            gpu_read(b, view)
        released = self.seq_mgr.swap_out(sid)
        self.cpu_bytes_used += len(buf)
        self.cpu_store[sid] = buf
        return released

    def restore(self, sid, gpu_write):
        if sid not in self.cpu_store:
            raise KeyError("no evicted data for sequence")
        # the reference removes the buffer before swap_in, so a failed
        # swap_in drops the evicted bytes (src/kv_swap.rs:87-89)
        buf = self.cpu_store.pop(sid)
        n = len(buf) // self.block_bytes
        new = self.seq_mgr.swap_in(sid, n)
        for i, b in enumerate(new):
            gpu_write(b, bytes(buf[i * self.block_bytes:(i + 1) * self.block_bytes]))
        self.cpu_bytes_used = max(self.cpu_bytes_used - len(buf), 0)
        return new

    def is_evicted(self, sid):
        return sid in self.cpu_store

    def evicted_count(self):
        return len(self.cpu_store)

    def maybe_evict(self, sid, free_threshold, gpu_read):
        if self.seq_mgr.allocator.num_free_blocks() < free_threshold and not self.is_evicted(sid):
            try:
                self.evict(sid, gpu_read)
                return True
            except Exception:
                return False
        return False
