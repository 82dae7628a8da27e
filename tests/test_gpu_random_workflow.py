"""A seeded random workflow over one device pool, mirrored on the oracle:
sequences are created, grown by appends of 1 .. 48 tokens, forked (sharing
their blocks), copied on write before an append into a shared, partly filled
last block (air_seq_cow_last_block, then air_kv_copy_blocks of the page
bytes), freed, swapped out (the blocks' bytes read to the host with
air_kv_read_blocks, the blocks released) and swapped back in (new blocks,
the bytes written with air_kv_write_blocks).  The oracle runs the same
operations on its restated SequenceManager (oracle/paged_attention_ref.py,
src/paged_attention.rs) and on a host pool (block copies and swaps as plain
array copies).  Every few operations: the block tables and slots are equal,
every page, scale and table of the device pool equals the host pool bit for
bit, and the decode of every resident sequence is within tolerance of the
oracle's.  bf16 and int8 pools."""
import numpy as np
import pytest

import airkv
import oracle
from gpu_helpers import assert_bits_equal, log, rel_err, torch_mod
from oracle import paged_attention_ref as ref

pytestmark = pytest.mark.gpu

NB, BS, NKV, NQ, D = 192, 16, 4, 16, 128
TOL = {airkv.BF16: 1e-3, airkv.INT8: 2e-2}


def _dev(x):
    return torch_mod().from_numpy(np.ascontiguousarray(x)).cuda()


@pytest.mark.parametrize("dtype,seed", [(airkv.BF16, 1), (airkv.BF16, 2), (airkv.INT8, 3), (airkv.INT8, 4)])
def test_random_workflow(dtype, seed):
    torch = torch_mod()
    rng = np.random.default_rng(9000 + seed)
    order = rng.permutation(NB).astype(np.uint32)
    mgr = airkv.SequenceManager(NB, BS, free_order=order)
    orc = ref.SequenceManager(NB, BS, free_order=[int(b) for b in order])
    pool = airkv.KvPool(NB, BS, NKV, D, dtype)
    host = oracle.HostPool(NB, BS, NKV, D, dtype, pool.scale_group)
    live, swapped = [], {}                            # resident sequences; id -> saved bytes
    counts = {"create": 0, "append": 0, "fork": 0, "cow": 0, "free": 0, "swap_out": 0, "swap_in": 0}

    def host_blocks(ids):
        out = [host.k[ids].copy(), host.v[ids].copy()]
        if host.k_scales is not None:
            out += [host.k_scales[ids].copy(), host.v_scales[ids].copy()]
        return out

    def host_put(ids, arrays):
        host.k[ids], host.v[ids] = arrays[0], arrays[1]
        if host.k_scales is not None:
            host.k_scales[ids], host.v_scales[ids] = arrays[2], arrays[3]

    def check(tag):
        torch.cuda.synchronize()
        k, v, ks, vs = pool.snapshot()
        assert_bits_equal(k, host.k, f"{tag}: k pages")
        assert_bits_equal(v, host.v, f"{tag}: v pages")
        if ks is not None:
            assert_bits_equal(ks.view(np.uint32), host.k_scales.view(np.uint32), f"{tag}: k scales")
            assert_bits_equal(vs.view(np.uint32), host.v_scales.view(np.uint32), f"{tag}: v scales")
        seqs = [s for s in live if mgr.table(s).num_tokens > 0]
        for s in live:
            assert mgr.table(s).physical_blocks == orc.table(s).physical_blocks, f"{tag}: table of {s}"
            assert mgr.table(s).num_tokens == orc.table(s).num_tokens
        if not seqs:
            return
        mb = max(len(mgr.table(s).physical_blocks) for s in seqs)
        tables, lens = mgr.export_tables(seqs, mb)
        q = rng.standard_normal((len(seqs), NQ, D)).astype(np.float32)
        out = torch.empty(len(seqs), NQ, D, device="cuda")
        pool.paged_decode(_dev(q), _dev(tables), _dev(lens), out)
        got = out.cpu().numpy()
        want = host.paged_decode(q, tables, lens)
        err = rel_err(got, want)
        assert err <= TOL[dtype], f"{tag}: decode rel err {err:.2e}"

    for step in range(90):
        free_blocks = orc.allocator.num_free_blocks()
        op = rng.choice(["create", "append", "append", "append", "fork", "free", "swap_out", "swap_in"])
        if op == "create" or not live:
            s = mgr.create_sequence()
            assert s == orc.create_sequence()
            live.append(s)
            counts["create"] += 1
            op = "append"
        if op == "append":
            s = int(rng.choice(live))
            n = int(rng.integers(1, 49))
            if (n + BS - 1) // BS + 1 > free_blocks:
                continue
            t = orc.table(s)
            if t.physical_blocks and t.num_tokens % BS != 0 and orc.allocator.ref_count(t.physical_blocks[-1]) > 1:
                # copy on write before appending into a shared, partly filled block
                pair = mgr.cow_last_block(s)
                new = orc.cow_last_block(s)
                assert pair is not None and pair[1] == new
                old = pair[0]
                if new != old:
                    pool.copy_blocks(_dev(np.array([old], np.int32)), _dev(np.array([new], np.int32)))
                    host_put([new], host_blocks([old]))
                    counts["cow"] += 1
            slots = mgr.append_slots(s, n)
            want_slots = np.array([orc.slot_for_append(s) for _ in range(n)], np.int64)
            assert np.array_equal(slots, want_slots), f"step {step}: slots"
            k = rng.standard_normal((n, NKV, D)).astype(np.float32)
            v = rng.standard_normal((n, NKV, D)).astype(np.float32)
            pool.append(_dev(k), _dev(v), _dev(slots))
            assert host.append(k, v, slots) == 0
            counts["append"] += 1
        elif op == "fork":
            p = int(rng.choice(live))
            c = mgr.fork_sequence(p)
            assert c == orc.fork_sequence(p)
            live.append(c)
            counts["fork"] += 1
        elif op == "free" and len(live) > 1:
            s = int(rng.choice(live))
            mgr.free_sequence(s)
            orc.free_sequence(s)
            live.remove(s)
            counts["free"] += 1
        elif op == "swap_out" and len(live) > 1:
            s = int(rng.choice(live))
            blocks = list(mgr.table(s).physical_blocks)
            saved = (pool.read_blocks(blocks), host_blocks(blocks))
            assert mgr.swap_out(s) == orc.swap_out(s) == blocks
            swapped[s] = saved
            live.remove(s)
            counts["swap_out"] += 1
        elif op == "swap_in" and swapped:
            s = int(rng.choice(list(swapped)))
            dev_bytes, host_arrays = swapped[s]
            n = len(dev_bytes)
            if n > free_blocks:
                continue
            new = mgr.swap_in(s, n)
            assert new == orc.swap_in(s, n)
            if n:
                pool.write_blocks(new, dev_bytes)
                host_put(new, host_arrays)
            del swapped[s]
            live.append(s)
            counts["swap_in"] += 1
        if step % 10 == 9:
            check(f"step {step}")
    check("end")
    log(f"workflow dtype {dtype} seed {seed}: {counts}, {len(live)} live, {len(swapped)} swapped")
    assert counts["cow"] > 0 and counts["swap_in"] > 0 and counts["fork"] > 0
    assert pool.error_count() == 0
