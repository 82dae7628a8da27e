"""GPU parity on pools whose K and V slabs are each larger than 4 GiB, so
every page byte offset past the first 4 GiB needs 64-bit arithmetic in the
append, gather, fused append + decode, decode and prefill kernels.  The
sequences' block tables mix ids from the top of the pool (offsets beyond
2^32 bytes) with a few low ones.  The oracle runs on a small host pool that
mirrors only the touched blocks (each big block id mapped to a small one):
pages, group scales and gathered views bit-exact, attention within 1e-3
(bf16 pages) or 2e-2 (int8 / fp8 pages).  About 9.2 GB of device memory per
case; MI355X holds 288 GB."""
import numpy as np
import pytest

import airkv
import oracle
from gpu_helpers import assert_bits_equal, log, rel_err, torch_mod

pytestmark = pytest.mark.gpu

NKV, D, NQ = 8, 128, 32
TOL = {airkv.BF16: 1e-3, airkv.INT8: 2e-2, airkv.FP8: 2e-2}


@pytest.mark.parametrize("dtype,bs,n_blocks", [(airkv.BF16, 16, 140_000), (airkv.INT8, 16, 270_000),
                                               (airkv.FP8, 32, 140_000)])
def test_pool_beyond_4gib(dtype, bs, n_blocks):
    torch = torch_mod()
    log(f"large pool dtype={dtype} bs={bs} blocks={n_blocks}")
    pool = airkv.KvPool(n_blocks, bs, NKV, D, dtype)
    assert pool.num_blocks * pool.slab_bytes > (1 << 32)
    try:
        rng = np.random.default_rng(900 + dtype)
        lens = np.array([1, 100, 513, 1200], np.int64)        # context before the decode step
        final = lens + 1                                        # after the fused append
        nb = (final + bs - 1) // bs
        max_blocks = int(nb.max())
        total_blocks = int(nb.sum())
        # mostly ids above 2^32 / slab_bytes, a few low ones, no id twice
        high = rng.choice(np.arange(n_blocks - 4 * total_blocks, n_blocks), total_blocks - 4, replace=False)
        ids = rng.permutation(np.concatenate([high, [0, 1, 7, 1000]])).astype(np.int32)
        tables = np.full((len(lens), max_blocks), -1, np.int32)
        off = 0
        for b, n in enumerate(nb):
            tables[b, :n] = ids[off:off + n]
            off += n
        assert int(tables.max()) * pool.slab_bytes > (1 << 32)
        # the host mirror: block ids mapped to 0 .. total_blocks - 1
        small = {int(x): i for i, x in enumerate(ids)}
        tables_s = np.vectorize(lambda x: small.get(int(x), -1))(tables).astype(np.int32)
        host = oracle.HostPool(total_blocks, bs, NKV, D, dtype, 32)

        def slots_of(tbl, b, positions):
            return (tbl[b, positions // bs].astype(np.int64) * bs + positions % bs).astype(np.int64)

        # context rows
        n_ctx = int(lens.sum())
        k = rng.standard_normal((n_ctx, NKV, D)).astype(np.float32)
        v = rng.standard_normal((n_ctx, NKV, D)).astype(np.float32)
        big_slots = np.concatenate([slots_of(tables, b, np.arange(n)) for b, n in enumerate(lens)])
        small_slots = np.concatenate([slots_of(tables_s, b, np.arange(n)) for b, n in enumerate(lens)])
        pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), torch.from_numpy(big_slots).cuda())
        assert host.append(k, v, small_slots) == 0

        # the decode step: every sequence's new row appended by the decode launch
        kn = rng.standard_normal((len(lens), NKV, D)).astype(np.float32)
        vn = rng.standard_normal((len(lens), NKV, D)).astype(np.float32)
        q = torch.from_numpy(rng.standard_normal((len(lens), NQ, D)).astype(np.float32)).cuda().to(torch.bfloat16)
        out = torch.full((len(lens), NQ, D), float("nan"), device="cuda")
        tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(final.astype(np.int32)).cuda()
        pool.paged_decode_append(q, torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda(), tt, lt, out)
        torch.cuda.synchronize()
        assert host.append(kn, vn, np.array([slots_of(tables_s, b, np.array([n]))[0]
                                             for b, n in enumerate(lens)], np.int64)) == 0
        want = host.paged_decode(q.float().cpu().numpy(), tables_s, final.astype(np.int32))
        err = rel_err(out.cpu().numpy(), want)
        log(f"  fused append + decode rel err {err:.2e}")
        assert err <= TOL[dtype]

        # every touched page (and scale) against the mirror
        kb, vb, ksb, vsb = pool.split_blocks(pool.read_blocks(ids))
        order = np.array([small[int(x)] for x in ids])
        assert_bits_equal(kb, host.k[order], "k pages")
        assert_bits_equal(vb, host.v[order], "v pages")
        if ksb is not None:
            assert_bits_equal(ksb.view(np.uint32), host.k_scales[order].view(np.uint32), "k scales")
            assert_bits_equal(vsb.view(np.uint32), host.v_scales[order].view(np.uint32), "v scales")

        # decode alone, over the same pages
        out2 = torch.full_like(out, float("nan"))
        pool.paged_decode(q, tt, lt, out2)
        torch.cuda.synchronize()
        assert np.array_equal(out2.cpu().numpy().view(np.uint32), out.cpu().numpy().view(np.uint32))

        # gather (f32 views; quantized pages dequantized) against the oracle's
        per = final * NKV * D
        offs = np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)
        gk = torch.empty(int(per.sum()), device="cuda")
        gv = torch.empty_like(gk)
        pool.gather(tt, lt, torch.from_numpy(offs).cuda(), gk, gv, out_dtype=airkv.F32)
        wk, wv, _, bad = host.gather(tables_s, final.astype(np.int32), out_dtype=oracle.F32)
        assert bad == 0
        assert_bits_equal(gk.cpu().numpy().view(np.uint32), wk.view(np.uint32), "gathered k")
        assert_bits_equal(gv.cpu().numpy().view(np.uint32), wv.view(np.uint32), "gathered v")

        # prefill: the newest 64 tokens of the two longest sequences
        C = 64
        cu = np.array([0, C, 2 * C], np.int32)
        sel = [2, 3]
        qp = torch.from_numpy(rng.standard_normal((2 * C, NQ, D)).astype(np.float32)).cuda().to(torch.bfloat16)
        op = torch.full((2 * C, NQ, D), float("nan"), device="cuda")
        tsel = np.ascontiguousarray(tables[sel])
        pool.paged_prefill(qp, torch.from_numpy(cu).cuda(), torch.from_numpy(tsel).cuda(),
                           torch.from_numpy(final[sel].astype(np.int32)).cuda(), op, max_q_len=C)
        torch.cuda.synchronize()
        wantp = host.paged_prefill(qp.float().cpu().numpy(), cu, np.ascontiguousarray(tables_s[sel]),
                                   final[sel].astype(np.int32))
        errp = rel_err(op.cpu().numpy(), wantp)
        log(f"  prefill rel err {errp:.2e}")
        assert errp <= TOL[dtype]
        assert pool.error_count() == 0
    finally:
        pool.close()
