"""Host-side block manager: the reference's own tests, run against both the
product (C++ via the C ABI) and the oracle restatement, plus a randomized
differential test that demands identical block tables.  CPU only.

Ported from src/paged_attention.rs:390-590 and src/kv_swap.rs:124-169.
"""
import random

import numpy as np
import pytest

import airkv
from oracle import paged_attention_ref as ref

IMPLS = {"product": airkv, "oracle": ref}
BS = 16


@pytest.fixture(params=sorted(IMPLS))
def m(request):
    return IMPLS[request.param]


def test_allocator_allocates_and_releases(m):
    a = m.BlockAllocator(4)
    b1, b2 = a.allocate(), a.allocate()
    assert a.num_free_blocks() == 2
    a.release(b1)
    assert a.num_free_blocks() == 3
    a.release(b2)
    assert a.num_free_blocks() == 4


def test_allocator_exhaustion_returns_none(m):
    a = m.BlockAllocator(2)
    assert a.allocate() is not None and a.allocate() is not None
    assert a.allocate() is None


def test_ref_count_tracks_sharing(m):
    a = m.BlockAllocator(4)
    b = a.allocate()
    assert a.ref_count(b) == 1
    a.share(b)
    assert a.ref_count(b) == 2
    a.release(b)
    assert a.ref_count(b) == 1
    a.release(b)
    assert a.ref_count(b) == 0


def test_cow_write_copies_on_shared_block(m):
    a = m.BlockAllocator(4)
    b = a.allocate()
    a.share(b)
    nb = a.cow_write(b)
    assert nb != b
    assert a.ref_count(b) == 1 and a.ref_count(nb) == 1


def test_cow_write_no_copy_on_sole_owner(m):
    a = m.BlockAllocator(4)
    b = a.allocate()
    assert a.cow_write(b) == b


def test_sequence_manager_create_and_append(m):
    mgr = m.SequenceManager(16)
    sid = mgr.create_sequence()
    for _ in range(BS):
        mgr.append_token(sid)
    t = mgr.table(sid)
    assert t.num_logical_blocks() == 1 and t.num_tokens == BS
    mgr.append_token(sid)
    assert mgr.table(sid).num_logical_blocks() == 2


def test_fork_shares_parent_blocks(m):
    mgr = m.SequenceManager(16)
    parent = mgr.create_sequence()
    for _ in range(BS):
        mgr.append_token(parent)
    child = mgr.fork_sequence(parent)
    assert mgr.table(parent).physical_blocks[0] == mgr.table(child).physical_blocks[0]
    assert mgr.allocator.ref_count(mgr.table(parent).physical_blocks[0]) == 2


def test_free_sequence_releases_blocks(m):
    mgr = m.SequenceManager(4)
    sid = mgr.create_sequence()
    mgr.append_token(sid)
    before = mgr.allocator.num_free_blocks()
    mgr.free_sequence(sid)
    assert mgr.allocator.num_free_blocks() == before + 1


def test_append_token_oom_error(m):
    mgr = m.SequenceManager(1)
    sid = mgr.create_sequence()
    for _ in range(BS):
        mgr.append_token(sid)
    with pytest.raises(MemoryError):
        mgr.append_token(sid)


def test_block_manager_is_send():
    # Rust compile-time Send check (src/paged_attention.rs:499-504); the C++
    # objects own no thread-affine state: a manager built on one thread is
    # used from another.
    import threading
    out = {}

    def make():
        out["mgr"] = airkv.SequenceManager(4)

    th = threading.Thread(target=make)
    th.start()
    th.join()
    sid = out["mgr"].create_sequence()
    assert out["mgr"].append_token(sid) == 0


def test_logical_block_for_token_correct():
    assert airkv.BlockTable.logical_block_for_token(0) == 0
    assert airkv.BlockTable.logical_block_for_token(BS - 1) == 0
    assert airkv.BlockTable.logical_block_for_token(BS) == 1


def test_can_allocate_checks_availability(m):
    a = m.BlockAllocator(4)
    assert a.can_allocate(4) and not a.can_allocate(5)
    a.allocate()
    assert a.can_allocate(3) and not a.can_allocate(4)


def test_num_blocks_for_tokens_rounds_up(m):
    f = m.BlockAllocator.num_blocks_for_tokens
    assert [f(0), f(1), f(BS), f(BS + 1), f(2 * BS)] == [0, 1, 1, 2, 2]


def test_utilization_tracks_usage(m):
    a = m.BlockAllocator(4)
    assert a.utilization() == 0.0
    a.allocate()
    assert abs(a.utilization() - 0.25) < 1e-6
    a.allocate()
    assert abs(a.utilization() - 0.5) < 1e-6


def test_swap_out_frees_blocks(m):
    mgr = m.SequenceManager(4)
    sid = mgr.create_sequence()
    for _ in range(BS):
        mgr.append_token(sid)
    before = mgr.allocator.num_free_blocks()
    assert len(mgr.swap_out(sid)) == 1
    assert mgr.allocator.num_free_blocks() == before + 1
    assert mgr.table(sid).physical_blocks == []


def test_swap_in_allocates_new_blocks(m):
    mgr = m.SequenceManager(4)
    sid = mgr.create_sequence()
    for _ in range(BS):
        mgr.append_token(sid)
    mgr.swap_out(sid)
    assert len(mgr.swap_in(sid, 1)) == 1
    assert len(mgr.table(sid).physical_blocks) == 1


def test_swap_in_oom_returns_error(m):
    mgr = m.SequenceManager(1)
    sid = mgr.create_sequence()
    mgr.append_token(sid)
    sid2 = mgr.create_sequence()
    with pytest.raises(MemoryError):
        mgr.swap_in(sid2, 1)


def test_can_schedule_reflects_pool_state(m):
    mgr = m.SequenceManager(1)
    assert mgr.can_schedule()
    sid = mgr.create_sequence()
    mgr.append_token(sid)
    assert not mgr.can_schedule()


# --- kv_swap.rs tests --------------------------------------------------------

def _noop_read(_block, buf):
    buf[:] = b"\xab" * len(buf)


def _noop_write(_block, _data):
    pass


def test_evict_and_restore_round_trip(m):
    mgr = m.KvSwapManager(8, 64)
    sid = mgr.seq_mgr.create_sequence()
    for _ in range(BS):
        mgr.seq_mgr.append_token(sid)
    before = mgr.seq_mgr.allocator.num_free_blocks()
    released = mgr.evict(sid, _noop_read)
    assert len(released) == 1
    assert mgr.seq_mgr.allocator.num_free_blocks() == before + 1
    assert mgr.is_evicted(sid)
    mgr.restore(sid, _noop_write)
    assert not mgr.is_evicted(sid)
    assert mgr.cpu_bytes_used == 0


def test_restore_fails_without_evict(m):
    mgr = m.KvSwapManager(4, 64)
    sid = mgr.seq_mgr.create_sequence()
    with pytest.raises(KeyError):
        mgr.restore(sid, _noop_write)


def test_maybe_evict_triggers_when_below_threshold(m):
    mgr = m.KvSwapManager(2, 64)
    sid = mgr.seq_mgr.create_sequence()
    for _ in range(BS):
        mgr.seq_mgr.append_token(sid)
    assert mgr.maybe_evict(sid, 2, _noop_read)
    assert mgr.is_evicted(sid)


def test_swap_bytes_round_trip_through_callbacks():
    """The bytes gpu_read produced come back to gpu_write unchanged, block
    by block, in table order (src/kv_swap.rs:61-68, :91-94)."""
    store = {}
    mgr = airkv.KvSwapManager(8, 32)
    sid = mgr.seq_mgr.create_sequence()
    for _ in range(3 * BS):
        mgr.seq_mgr.append_token(sid)
    blocks = mgr.seq_mgr.table(sid).physical_blocks

    def read(b, buf):
        buf[:] = bytes([(b * 7 + i) & 0xFF for i in range(len(buf))])

    mgr.evict(sid, read)
    got = []
    new = mgr.restore(sid, lambda b, data: got.append((b, data)))
    assert [b for b, _ in got] == new
    for (nb, data), ob in zip(got, blocks):
        assert data == bytes([(ob * 7 + i) & 0xFF for i in range(32)])


def _failing(_block, _buf):
    raise IOError("device copy failed")


def test_evict_stops_on_a_failed_read():
    """A read callback that fails leaves the sequence resident: nothing is
    released and nothing is stored."""
    mgr = airkv.KvSwapManager(8, 32)
    sid = mgr.seq_mgr.create_sequence()
    for _ in range(2 * BS):
        mgr.seq_mgr.append_token(sid)
    blocks = list(mgr.seq_mgr.table(sid).physical_blocks)
    free = mgr.seq_mgr.allocator.num_free_blocks()
    with pytest.raises(IOError):
        mgr.evict(sid, _failing)
    assert mgr.seq_mgr.table(sid).physical_blocks == blocks
    assert mgr.seq_mgr.allocator.num_free_blocks() == free
    assert not mgr.is_evicted(sid) and mgr.cpu_bytes_used == 0
    with pytest.raises(IOError):
        mgr.maybe_evict(sid, 100, _failing)
    assert not mgr.is_evicted(sid)


def test_restore_undoes_swap_in_on_a_failed_write():
    """A write callback that fails puts the sequence back into the evicted
    state with its bytes, so a second restore can succeed."""
    mgr = airkv.KvSwapManager(8, 32)
    sid = mgr.seq_mgr.create_sequence()
    for _ in range(2 * BS):
        mgr.seq_mgr.append_token(sid)

    def read(b, buf):
        buf[:] = bytes([(b + i) & 0xFF for i in range(len(buf))])

    old = list(mgr.seq_mgr.table(sid).physical_blocks)
    mgr.evict(sid, read)
    free = mgr.seq_mgr.allocator.num_free_blocks()
    used = mgr.cpu_bytes_used
    with pytest.raises(IOError):
        mgr.restore(sid, _failing)
    assert mgr.is_evicted(sid) and mgr.cpu_bytes_used == used
    assert mgr.seq_mgr.table(sid).physical_blocks == []
    assert mgr.seq_mgr.allocator.num_free_blocks() == free
    got = []
    mgr.restore(sid, lambda b, data: got.append(data))
    assert got == [bytes([(b + i) & 0xFF for i in range(32)]) for b in old]
    assert not mgr.is_evicted(sid)


# --- product-specific behaviour -----------------------------------------------

def test_product_rejects_double_release():
    a = airkv.BlockAllocator(2)
    b = a.allocate()
    a.release(b)
    with pytest.raises(airkv.AirKvError) as e:
        a.release(b)
    assert e.value.code == airkv.AIR_KV_E_STATE
    assert a.num_free_blocks() == 2          # no duplicate on the free list


def test_oracle_keeps_reference_double_release_quirk():
    a = ref.BlockAllocator(2)
    b = a.allocate()
    a.release(b)
    a.release(b)
    assert a.num_free_blocks() == 3          # the reference's duplicate push


def test_product_append_to_full_block_is_an_error():
    a = airkv.BlockAllocator(1)
    b = a.allocate()
    for _ in range(BS - 1):
        assert not a.append_token(b)
    assert a.append_token(b)
    with pytest.raises(AssertionError):
        a.append_token(b)


def test_unknown_sequence_errors():
    mgr = airkv.SequenceManager(4)
    with pytest.raises(KeyError):
        mgr.append_token(99)
    with pytest.raises(KeyError):
        mgr.fork_sequence(99)
    assert mgr.table(99) is None
    mgr.free_sequence(99)                    # ignored, as in the reference
    assert mgr.cow_last_block(99) is None


def test_free_order_permutation_and_validation():
    order = np.array([3, 1, 0, 2], np.uint32)
    a = airkv.BlockAllocator(4, free_order=order)
    assert [a.allocate() for _ in range(4)] == [3, 1, 0, 2]
    with pytest.raises(airkv.AirKvError):
        airkv.BlockAllocator(4, free_order=np.array([0, 0, 1, 2], np.uint32))


def test_append_slots_matches_slot_arithmetic():
    mgr = airkv.SequenceManager(8, block_size=16, free_order=np.array([5, 2, 7, 0, 1, 3, 4, 6], np.uint32))
    s = mgr.create_sequence()
    slots = mgr.append_slots(s, 40)
    blocks = mgr.table(s).physical_blocks
    assert blocks == [5, 2, 7]
    want = [blocks[p // 16] * 16 + p % 16 for p in range(40)]
    assert slots.tolist() == want


def test_export_tables_pads_with_minus_one():
    mgr = airkv.SequenceManager(16, block_size=16)
    a, b = mgr.create_sequence(), mgr.create_sequence()
    mgr.append_slots(a, 20)
    mgr.append_slots(b, 3)
    tables, lens = mgr.export_tables([a, b], 4)
    assert lens.tolist() == [20, 3]
    assert tables[0].tolist()[:2] == mgr.table(a).physical_blocks and tables[0, 2] == -1
    assert tables[1].tolist() == [mgr.table(b).physical_blocks[0], -1, -1, -1]
    with pytest.raises(airkv.AirKvError):
        mgr.export_tables([a], 1)            # 2 blocks do not fit a 1-wide table


@pytest.mark.parametrize("block_size", [16, 32])
def test_random_ops_match_oracle_tables(block_size):
    """Random create / append / fork / cow / free / swap sequences: the C++
    manager and the restatement must agree on every table, every refcount and
    the free-list length after every operation (FIFO order is therefore
    identical, since any difference would surface as a different block id)."""
    rng = random.Random(1234 + block_size)
    cap = 64
    order = list(range(cap))
    rng.shuffle(order)
    P = airkv.SequenceManager(cap, block_size, free_order=np.array(order, np.uint32))
    O = ref.SequenceManager(cap, block_size, free_order=order)
    live = []
    swapped = {}
    for step in range(3000):
        op = rng.random()
        if op < 0.08 or not live:
            sp, so = P.create_sequence(), O.create_sequence()
            assert sp == so
            live.append(sp)
        elif op < 0.70:
            s = rng.choice(live)
            if s in swapped:
                continue
            # writers copy a shared, partly filled last block first (the
            # protocol of src/paged_attention.rs:27-31, :326-335)
            to = O.table(s)
            if (to.physical_blocks and to.num_tokens % block_size
                    and O.allocator.ref_count(to.physical_blocks[-1]) > 1):
                r_o = O.cow_last_block(s)
                r_p = P.cow_last_block(s)
                assert (r_p is None) == (r_o is None)
                if r_o is None:
                    continue
                assert r_p[1] == r_o
            n = rng.randint(1, 40)
            for _ in range(n):
                try:
                    bo = O.append_token(s)
                except MemoryError:
                    with pytest.raises(MemoryError):
                        P.append_token(s)
                    break
                assert P.append_token(s) == bo
        elif op < 0.78:
            s = rng.choice(live)
            if s in swapped:
                continue
            c1, c2 = P.fork_sequence(s), O.fork_sequence(s)
            assert c1 == c2
            live.append(c1)
        elif op < 0.84:
            s = rng.choice(live)
            r_o = O.cow_last_block(s)
            r_p = P.cow_last_block(s)
            assert (r_p is None) == (r_o is None)
            if r_p is not None:
                assert r_p[1] == r_o
        elif op < 0.93:
            s = live.pop(rng.randrange(len(live)))
            swapped.pop(s, None)
            P.free_sequence(s)
            O.free_sequence(s)
        elif op < 0.97:
            s = rng.choice(live)
            if s in swapped:
                continue
            assert P.swap_out(s) == O.swap_out(s)
            swapped[s] = len(O.table(s).physical_blocks)
        else:
            if not swapped:
                continue
            s = rng.choice(list(swapped))
            n = block_size and -(-O.table(s).num_tokens // block_size)
            try:
                bo = O.swap_in(s, n)
            except MemoryError:
                with pytest.raises(MemoryError):
                    P.swap_in(s, n)
                continue
            assert P.swap_in(s, n) == bo
            swapped.pop(s)
        assert P.allocator.num_free_blocks() == O.allocator.num_free_blocks()
        for s in live:
            tp, to = P.table(s), O.table(s)
            assert tp.physical_blocks == to.physical_blocks and tp.num_tokens == to.num_tokens
    for b in range(cap):
        assert P.allocator.ref_count(b) == O.allocator.ref_count(b)


# ---- extensions without a reference counterpart (product only) -------------

def test_truncate_releases_trailing_blocks_fifo():
    """truncate keeps ceil(n/bs) blocks, pushes the others onto the back of
    the free list in table order, and leaves the front of the list alone."""
    order = np.array([5, 2, 7, 0, 1, 3, 4, 6], np.uint32)
    mgr = airkv.SequenceManager(8, block_size=16, free_order=order)
    s = mgr.create_sequence()
    mgr.append_slots(s, 40)                  # blocks 5, 2, 7
    mgr.truncate(s, 17)                      # keeps 5, 2; releases 7
    t = mgr.table(s)
    assert t.physical_blocks == [5, 2] and t.num_tokens == 17
    assert mgr.allocator.num_free_blocks() == 6
    # free list now 0 1 3 4 6 7: the next fresh sequence takes 0 first, 7 last
    o = mgr.create_sequence()
    assert [mgr.append_token(o) for _ in range(16 * 6)][::16] == [0, 1, 3, 4, 6, 7]


def test_truncate_sets_fill_and_appends_continue():
    mgr = airkv.SequenceManager(4, block_size=16)
    s = mgr.create_sequence()
    mgr.append_slots(s, 32)                  # two full blocks
    mgr.truncate(s, 20)
    last = mgr.table(s).physical_blocks[-1]
    assert mgr.allocator.block_info(last) == (4, False)
    slots = mgr.append_slots(s, 12)          # fills block 1 exactly, no new block
    assert len(mgr.table(s).physical_blocks) == 2
    assert slots.tolist() == [last * 16 + p for p in range(4, 16)]
    assert mgr.allocator.block_info(last) == (16, True)
    mgr.append_token(s)                      # next token opens a new block
    assert len(mgr.table(s).physical_blocks) == 3


def test_truncate_noop_zero_and_errors():
    mgr = airkv.SequenceManager(4, block_size=16)
    s = mgr.create_sequence()
    mgr.append_slots(s, 10)
    mgr.truncate(s, 10)
    mgr.truncate(s, 99)
    assert mgr.table(s).num_tokens == 10
    mgr.truncate(s, 0)
    assert mgr.table(s).physical_blocks == [] and mgr.allocator.num_free_blocks() == 4
    with pytest.raises(KeyError):
        mgr.truncate(77, 0)
    with pytest.raises(airkv.AirKvError):
        mgr.truncate(s, -1)


def test_truncate_into_shared_block_keeps_its_fill():
    """A block shared with a fork keeps the fill the other sequence gave it."""
    mgr = airkv.SequenceManager(8, block_size=16)
    s = mgr.create_sequence()
    mgr.append_slots(s, 30)
    c = mgr.fork_sequence(s)
    mgr.truncate(c, 5)
    first = mgr.table(s).physical_blocks[0]
    assert mgr.table(c).physical_blocks == [first]
    assert mgr.allocator.ref_count(first) == 2
    assert mgr.allocator.block_info(first) == (16, True)
    assert mgr.allocator.ref_count(mgr.table(s).physical_blocks[1]) == 1


def test_fork_truncate_cow_then_append():
    """A fork truncated into a block it shares: copy-on-write gives the
    private block the fork's own fill (5 of 16), so the fork keeps appending
    into it and the other owner's block is untouched."""
    mgr = airkv.SequenceManager(8, block_size=16)
    s = mgr.create_sequence()
    mgr.append_slots(s, 30)
    c = mgr.fork_sequence(s)
    mgr.truncate(c, 5)
    shared = mgr.table(s).physical_blocks[0]
    old, new = mgr.cow_last_block(c)
    assert old == shared and new != shared
    assert mgr.allocator.block_info(new) == (5, False)
    assert mgr.allocator.block_info(shared) == (16, True)
    slots = mgr.append_slots(c, 11)          # fills the private block exactly
    assert slots.tolist() == [new * 16 + p for p in range(5, 16)]
    assert mgr.allocator.block_info(new) == (16, True)
    nxt = mgr.append_token(c)                # then opens a fresh block
    assert nxt not in (new, shared) and len(mgr.table(c).physical_blocks) == 2
    assert mgr.allocator.ref_count(shared) == 1 and mgr.table(s).num_tokens == 30


def test_fork_truncate_cow_block_then_append():
    """The same through cow_block at an inner index: the private block holds
    the fork's tokens of it (a full block stays full)."""
    mgr = airkv.SequenceManager(8, block_size=16)
    s = mgr.create_sequence()
    mgr.append_slots(s, 40)
    c = mgr.fork_sequence(s)
    mgr.truncate(c, 20)                      # blocks 0 (full) and 1 (4 of 16), both shared
    _, n0 = mgr.cow_block(c, 0)
    _, n1 = mgr.cow_block(c, 1)
    assert mgr.allocator.block_info(n0) == (16, True)
    assert mgr.allocator.block_info(n1) == (4, False)
    assert mgr.append_slots(c, 12).tolist() == [n1 * 16 + p for p in range(4, 16)]


def test_cow_block_any_index():
    mgr = airkv.SequenceManager(8, block_size=16)
    s = mgr.create_sequence()
    mgr.append_slots(s, 40)
    c = mgr.fork_sequence(s)
    blocks = mgr.table(s).physical_blocks
    old, new = mgr.cow_block(c, 1)
    assert old == blocks[1] and new not in blocks
    assert mgr.table(c).physical_blocks == [blocks[0], new, blocks[2]]
    assert mgr.allocator.ref_count(old) == 1 and mgr.allocator.ref_count(new) == 1
    assert mgr.cow_block(c, 1) == (new, new)            # now private: no copy
    with pytest.raises(airkv.AirKvError):
        mgr.cow_block(c, 3)
