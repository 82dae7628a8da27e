"""GPU tests of PagedSessionCache, the paged SessionKvCache seam
(src/kv_cache.rs:431-446), through the C ABI.

Restates the reference's KvCacheManager tests that exercise the trait
(test_seq_len_tracking, test_clear, the save / load round trips,
src/kv_cache.rs:679-785) and the MockSessionKvCache truncate contract
(:508-531), with the stored bytes checked bit-exactly against the oracle's
codecs (bf16 RNE, Q8_0, reference fp8), plus the paged-only behaviour:
per-layer lengths, truncation releasing blocks, fork with copy-on-write, and
decode over a session's block table.
"""
import numpy as np
import pytest

import airkv
import oracle
from gpu_helpers import log, torch_mod

pytestmark = pytest.mark.gpu

NKV, D = 2, 128


def _rows(n, seed):
    torch = torch_mod()
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    k = torch.randn(n, NKV, D, generator=g, device="cuda")
    v = torch.randn(n, NKV, D, generator=g, device="cuda")
    return k, v


def _expected(rows, dtype):
    """What a pool of `dtype` returns for f32 rows (load converts back)."""
    x = rows.cpu().numpy().astype(np.float32)
    if dtype == airkv.F32:
        return x
    if dtype == airkv.BF16:
        return oracle.bf16_to_f32(oracle.bf16_from_f32(x.reshape(-1))).reshape(x.shape)
    flat = x.reshape(-1, 32)
    if dtype == airkv.INT8:
        out = np.stack([oracle.q8_dequantize(*oracle.q8_quantize(g)) for g in flat])
    else:
        out = []
        for g in flat:
            codes, scale = oracle.fp8_quantize_group(g)
            out.append(oracle.fp8_to_f32(codes) * np.float32(scale))
        out = np.stack(out).astype(np.float32)
    return out.reshape(x.shape)


def _session(n_layers=2, dtype=airkv.F32, capacity=32, bs=16):
    mgr = airkv.SequenceManager(capacity, block_size=bs)
    pools = [airkv.KvPool(capacity, bs, NKV, D, dtype) for _ in range(n_layers)]
    return mgr, pools, airkv.PagedSessionCache(mgr, pools)


def _load_np(s, layer):
    torch = torch_mod()
    k, v = s.load(layer, dtype=torch.float32)
    torch.cuda.synchronize()
    return k.cpu().numpy(), v.cpu().numpy()


def test_seq_len_tracking():
    """src/kv_cache.rs test_seq_len_tracking: layer 0 saved, layer 1 untouched."""
    _, _, s = _session()
    assert s.seq_len(0) == 0 and s.seq_len(1) == 0
    k, v = _rows(4, 1)
    s.save(0, k, v)
    assert s.seq_len(0) == 4 and s.seq_len(1) == 0


def test_clear_releases_everything():
    """src/kv_cache.rs test_clear: memory > 0 after saves, 0 after clear."""
    mgr, _, s = _session()
    k, v = _rows(40, 2)
    s.save(0, k, v)
    s.save(1, k, v)
    assert s.memory_usage() > 0
    free_before = mgr.allocator.num_free_blocks()
    s.clear()
    assert s.memory_usage() == 0 and s.seq_len(0) == 0 and s.seq_len(1) == 0
    assert mgr.allocator.num_free_blocks() == free_before + 3


@pytest.mark.parametrize("dtype", [airkv.F32, airkv.BF16, airkv.INT8, airkv.FP8])
def test_save_load_roundtrip_bitexact(dtype):
    """save then load returns the stored form of every row, bit for bit: f32
    as is, bf16 round-to-nearest-even, int8 / fp8 the dequantized Q8_0 /
    reference-fp8 groups."""
    _, _, s = _session(n_layers=1, dtype=dtype)
    k, v = _rows(37, 3)
    s.save(0, k, v)
    gk, gv = _load_np(s, 0)
    assert gk.shape == (37, NKV, D)
    assert np.array_equal(gk.view(np.uint32), _expected(k, dtype).view(np.uint32))
    assert np.array_equal(gv.view(np.uint32), _expected(v, dtype).view(np.uint32))


def test_decode_loop_saves_growing_cache():
    """The generator's pattern: each step saves the whole concatenated cache;
    only the new rows are written, and load returns every row."""
    torch = torch_mod()
    _, _, s = _session(n_layers=2)
    k, v = _rows(70, 4)
    for n in [5, 6, 7, 16, 17, 33, 70]:
        for layer in range(2):
            s.save(layer, k[:n].contiguous(), v[:n].contiguous())
        assert s.seq_len(0) == n and s.seq_len(1) == n
    for layer in range(2):
        gk, gv = _load_np(s, layer)
        assert np.array_equal(gk, k.cpu().numpy()) and np.array_equal(gv, v.cpu().numpy())
    del torch


def test_truncate_to_then_append():
    """truncate_to(pos) keeps pos tokens in every layer (MockSessionKvCache
    contract: seq_len == pos), releases the blocks past them, and later
    appends continue at pos."""
    mgr, _, s = _session(n_layers=2)
    k, v = _rows(40, 5)
    for layer in range(2):
        s.save(layer, k, v)
    free0 = mgr.allocator.num_free_blocks()
    s.truncate_to(21)
    assert s.seq_len(0) == 21 and s.seq_len(1) == 21
    assert mgr.allocator.num_free_blocks() == free0 + 1          # 3 blocks -> 2
    s.truncate_to(99)                                            # beyond: no change
    assert s.seq_len(0) == 21
    k2, v2 = _rows(13, 6)
    for layer in range(2):
        s.append(layer, k2, v2)
    want_k = np.concatenate([k.cpu().numpy()[:21], k2.cpu().numpy()])
    want_v = np.concatenate([v.cpu().numpy()[:21], v2.cpu().numpy()])
    for layer in range(2):
        gk, gv = _load_np(s, layer)
        assert np.array_equal(gk, want_k) and np.array_equal(gv, want_v)
    s.truncate_to(0)
    assert s.seq_len(0) == 0 and s.memory_usage() == 0


def test_per_layer_lengths_share_one_table():
    """Layers advance one at a time within a step: a lagging layer writes into
    blocks the leading layer allocated, and a shorter save shortens only that
    layer (blocks are released once no layer uses them)."""
    mgr, _, s = _session(n_layers=3)
    k, v = _rows(50, 7)
    s.save(0, k, v)
    s.save(1, k[:20].contiguous(), v[:20].contiguous())
    used = mgr.allocator.num_used_blocks()
    assert used == 4
    s.save(2, k, v)
    assert mgr.allocator.num_used_blocks() == 4                  # no new blocks
    s.save(0, k[:10].contiguous(), v[:10].contiguous())
    assert s.seq_len(0) == 10 and mgr.allocator.num_used_blocks() == 4
    s.save(2, k[:10].contiguous(), v[:10].contiguous())
    assert mgr.allocator.num_used_blocks() == 2                  # max len is layer 1's 20
    for layer, n in [(0, 10), (1, 20), (2, 10)]:
        gk, _ = _load_np(s, layer)
        assert np.array_equal(gk, k.cpu().numpy()[:n])


def test_fork_copy_on_write_isolation():
    """fork shares the parent's blocks; the first write into a shared block
    copies it (in every layer's pool), so neither session sees the other's
    new tokens."""
    mgr, _, parent = _session(n_layers=2)
    k, v = _rows(20, 8)
    for layer in range(2):
        parent.save(layer, k, v)
    child = parent.fork()
    assert child.seq_len(0) == 20 and child.seq_id != parent.seq_id
    shared = mgr.table(parent.seq_id).physical_blocks
    assert mgr.table(child.seq_id).physical_blocks == shared
    kc, vc = _rows(3, 9)
    kp, vp = _rows(5, 10)
    for layer in range(2):
        child.append(layer, kc, vc)
        parent.append(layer, kp, vp)
    assert mgr.table(child.seq_id).physical_blocks[0] == shared[0]      # full block still shared
    assert mgr.table(child.seq_id).physical_blocks[1] != shared[1]      # written block copied
    base_k, base_v = k.cpu().numpy(), v.cpu().numpy()
    for layer in range(2):
        ck, cv = _load_np(child, layer)
        pk, pv = _load_np(parent, layer)
        assert np.array_equal(ck, np.concatenate([base_k, kc.cpu().numpy()]))
        assert np.array_equal(cv, np.concatenate([base_v, vc.cpu().numpy()]))
        assert np.array_equal(pk, np.concatenate([base_k, kp.cpu().numpy()]))
        assert np.array_equal(pv, np.concatenate([base_v, vp.cpu().numpy()]))
    child.close()
    parent.close()
    assert mgr.allocator.num_free_blocks() == 32


@pytest.mark.parametrize("dtype", [airkv.BF16, airkv.INT8])
def test_fork_truncate_then_append(dtype):
    """A fork rolled back into a block it shares with its parent, then
    appended to: the shared block is copied with the fork's own fill, the
    fork keeps its first tokens and gets the new ones after them, and the
    parent is unchanged.  Repeated appends keep working."""
    mgr, _, parent = _session(n_layers=2, dtype=dtype)
    k, v = _rows(30, 30)
    for layer in range(2):
        parent.save(layer, k, v)
    child = parent.fork()
    child.truncate_to(5)
    assert child.seq_len(0) == 5 and mgr.table(child.seq_id).physical_blocks == \
        mgr.table(parent.seq_id).physical_blocks[:1]
    kc, vc = _rows(20, 31)
    for layer in range(2):
        child.append(layer, kc[:3].contiguous(), vc[:3].contiguous())
        child.append(layer, kc[3:].contiguous(), vc[3:].contiguous())
    assert child.seq_len(0) == 25
    t_child, t_parent = mgr.table(child.seq_id), mgr.table(parent.seq_id)
    assert t_child.physical_blocks[0] != t_parent.physical_blocks[0]
    assert len(t_child.physical_blocks) == 2
    want_c = _expected(torch_mod().cat([k[:5], kc]), dtype)
    want_cv = _expected(torch_mod().cat([v[:5], vc]), dtype)
    want_p, want_pv = _expected(k, dtype), _expected(v, dtype)
    for layer in range(2):
        ck, cv = _load_np(child, layer)
        pk, pv = _load_np(parent, layer)
        assert np.array_equal(ck, want_c) and np.array_equal(cv, want_cv)
        assert np.array_equal(pk, want_p) and np.array_equal(pv, want_pv)
    child.close()
    parent.close()
    assert mgr.allocator.num_free_blocks() == 32


def test_pool_callbacks_reject_a_foreign_block_size():
    """A swap manager whose block_bytes differ from the pool's: the pool
    callbacks refuse the copy, and evict stops before releasing anything."""
    pool = airkv.KvPool(16, 16, NKV, D, airkv.BF16)
    mgr = airkv.KvSwapManager(16, pool.block_bytes + 64, block_size=16)
    sid = mgr.seq_mgr.create_sequence()
    for _ in range(20):
        mgr.seq_mgr.append_token(sid)
    blocks = list(mgr.seq_mgr.table(sid).physical_blocks)
    read, _write, ctx = airkv.pool_callbacks(pool)
    with pytest.raises(airkv.AirKvError):
        mgr.evict(sid, (read, ctx))
    assert mgr.seq_mgr.table(sid).physical_blocks == blocks and not mgr.is_evicted(sid)


def test_out_of_blocks_leaves_state_unchanged():
    """An append that needs more blocks than are free raises MemoryError and
    changes nothing (the reference's "out of memory — no free blocks")."""
    mgr, _, s = _session(n_layers=1, capacity=3)
    k, v = _rows(40, 11)
    s.save(0, k, v)
    k2, v2 = _rows(9, 12)
    with pytest.raises(MemoryError):
        s.append(0, k2, v2)
    assert s.seq_len(0) == 40 and mgr.table(s.seq_id).num_tokens == 40
    gk, _ = _load_np(s, 0)
    assert np.array_equal(gk, k.cpu().numpy())
    s.append(0, k2[:8].contiguous(), v2[:8].contiguous())                # fits the last block
    assert s.seq_len(0) == 48


def test_decode_over_session_tables():
    """Sessions feed the decode kernel directly: their sequence ids export the
    block tables, and the output matches the oracle on the same rows."""
    torch = torch_mod()
    mgr = airkv.SequenceManager(64, block_size=16)
    pool = airkv.KvPool(64, 16, NKV, D, airkv.BF16)
    host = oracle.HostPool(64, 16, NKV, D, oracle.BF16)
    sessions, lens = [], [33, 5, 100]
    for i, n in enumerate(lens):
        s = airkv.PagedSessionCache(mgr, [pool])
        k, v = _rows(n, 20 + i)
        s.save(0, k, v)
        sessions.append(s)
    tables, seq_lens = mgr.export_tables([s.seq_id for s in sessions], 7)
    for s, n in zip(sessions, lens):
        t = mgr.table(s.seq_id)
        slots = np.array([t.physical_blocks[p // 16] * 16 + p % 16 for p in range(n)], np.int64)
        gk, gv = _load_np(s, 0)
        assert host.append(gk, gv, slots) == 0
    q = torch.randn(3, 4 * NKV, D, device="cuda")
    out = torch.empty_like(q)
    pool.paged_decode(q, torch.from_numpy(tables).cuda(), torch.from_numpy(seq_lens).cuda(), out)
    torch.cuda.synchronize()
    want = host.paged_decode(q.cpu().numpy(), tables, seq_lens)
    err = np.abs(out.cpu().numpy() - want).max() / np.abs(want).max()
    log(f"session decode rel err {err:.2e}")
    assert err <= 1e-3
