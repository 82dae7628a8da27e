"""Helpers shared by the GPU parity tests (test infrastructure)."""
import sys

import numpy as np

import airkv
import oracle
from airkv import workloads
from oracle import paged_attention_ref as ref


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def torch_mod():
    import torch
    return torch


def oracle_manager(w: workloads.Workload):
    """Replays the workload's sequence construction on the restated
    allocator; returns its seq ids and append batches."""
    cfg = w.cfg
    mgr = ref.SequenceManager(w.num_blocks, cfg.block_size, free_order=w.free_order.tolist())
    return mgr


def replay_batches_on_oracle(w, prefill_lens, decode_steps):
    mgr = oracle_manager(w)
    seqs = [mgr.create_sequence() for _ in prefill_lens]
    batches = []
    for s, L in zip(seqs, prefill_lens):
        if L:
            batches.append(np.array([mgr.slot_for_append(s) for _ in range(L)], np.int64))
    for _ in range(decode_steps):
        batches.append(np.array([mgr.slot_for_append(s) for s in seqs], np.int64))
    return mgr, seqs, batches


def run_appends(w, rows_k, rows_v, pool=None, host=None):
    """Append every batch of the workload to the device pool and/or the
    oracle host pool, consuming rows in order."""
    torch = torch_mod() if pool is not None else None
    off = 0
    for slots in w.batches:
        n = len(slots)
        k, v = rows_k[off:off + n], rows_v[off:off + n]
        if pool is not None:
            pool.append(torch.from_numpy(np.ascontiguousarray(k)).cuda(),
                        torch.from_numpy(np.ascontiguousarray(v)).cuda(),
                        torch.from_numpy(slots).cuda())
        if host is not None:
            assert host.append(k, v, slots) == 0
        off += n
    assert off == len(rows_k)


def host_pool_for(w, fill=0):
    c = w.cfg
    return oracle.HostPool(w.num_blocks, c.block_size, c.n_kv_heads, c.head_dim, c.dtype,
                           c.scale_group, fill=fill)


def device_pool_for(w):
    c = w.cfg
    return airkv.KvPool(w.num_blocks, c.block_size, c.n_kv_heads, c.head_dim, c.dtype,
                        c.scale_group)


def assert_bits_equal(a, b, what):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    av = a.view(np.uint8).reshape(-1)
    bv = b.view(np.uint8).reshape(-1)
    if not np.array_equal(av, bv):
        bad = np.nonzero(av != bv)[0]
        raise AssertionError(f"{what}: {bad.size} bytes differ, first at byte {bad[0]}")


def assert_floats_bit_equal(a, b, what):
    """f32 arrays equal bit for bit, except that any NaN matches any NaN: the
    sign and payload of a NaN produced by arithmetic are unspecified by IEEE
    754 and by Rust (its float docs call NaN bit patterns non-deterministic),
    so only NaN-ness is part of the contract."""
    a = np.array(a, np.float32, copy=True)
    b = np.array(b, np.float32, copy=True)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        bad = np.nonzero(na != nb)[0]
        raise AssertionError(f"{what}: NaN positions differ, first at {bad[0]}")
    a[na] = 0.0
    b[nb] = 0.0
    assert_bits_equal(a, b, what)


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def decode_pieces(workspace, seq_lens):
    """Pieces per sequence of the matrix-core decode that last used
    `workspace` (one launch: batch <= 4096).  The workspace starts with that
    launch's tile prefix (int32 [batch + 1], 16-token tiles per sequence) and
    the slice length in tiles; sequence b's tiles meet slices prefix[b] //
    chunk .. (prefix[b + 1] - 1) // chunk.  Also checks the prefix against
    seq_lens.  Empty sequences have 0 pieces."""
    import numpy as np
    torch = torch_mod()
    torch.cuda.synchronize()
    batch = len(seq_lens)
    head = workspace[:4 * (batch + 2)].cpu().numpy().view(np.int32)
    pre, chunk = head[:batch + 1].astype(np.int64), int(head[batch + 1])
    tiles = (np.asarray(seq_lens, np.int64) + 15) // 16
    assert np.array_equal(np.diff(pre), tiles), "tile prefix disagrees with seq_lens"
    assert chunk >= 1
    w0, w1 = pre[:-1] // chunk, (pre[1:] - 1) // chunk
    return np.where(tiles > 0, w1 - w0 + 1, 0)
