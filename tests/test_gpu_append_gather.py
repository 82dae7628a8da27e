"""GPU parity: append (reshape-and-cache, incl. quantize-on-append) and gather
against the oracle, bit-exact, through the C ABI."""
import numpy as np
import pytest

import airkv
import oracle
from airkv import workloads
from gpu_helpers import (assert_bits_equal, device_pool_for, host_pool_for, log,
                         replay_batches_on_oracle, run_appends, torch_mod)

pytestmark = pytest.mark.gpu

C1_PREFILL = [37, 128, 200, 511]


def _seq_rows(w, prefill, steps):
    """Source-row indices of each sequence, in append order."""
    n = len(prefill)
    rows = [[] for _ in range(n)]
    off = 0
    for i, L in enumerate(prefill):
        rows[i].extend(range(off, off + L))
        off += L
    for _ in range(steps):
        for i in range(n):
            rows[i].append(off + i)
        off += n
    return rows


def _gather(pool, tables, lens, out_dtype, layout):
    torch = torch_mod()
    per = lens.astype(np.int64) * pool.n_kv_heads * pool.head_dim
    offs = np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)
    tdt = torch.float32 if out_dtype == airkv.F32 else torch.bfloat16
    ok = torch.zeros(int(per.sum()), dtype=tdt, device="cuda")
    ov = torch.zeros_like(ok)
    pool.gather(torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda(),
                torch.from_numpy(offs).cuda(), ok, ov, out_dtype, layout)
    torch.cuda.synchronize()
    if out_dtype == airkv.F32:
        return ok.cpu().numpy(), ov.cpu().numpy(), offs
    return (ok.view(torch.int16).cpu().numpy().view(np.uint16),
            ov.view(torch.int16).cpu().numpy().view(np.uint16), offs)


@pytest.mark.parametrize("dtype", [airkv.F32, airkv.BF16, airkv.INT8, airkv.FP8])
def test_c1_append_gather_bitexact(dtype):
    log(f"c1 append/gather dtype={dtype}")
    w = workloads.c1_workload()
    w.cfg = workloads.Config(w.cfg.name, 8, 8, 64, 16, dtype, 4)
    # block tables / slot mappings identical to the restated allocator
    mgr_o, seqs_o, batches_o = replay_batches_on_oracle(w, C1_PREFILL, 16)
    assert len(batches_o) == len(w.batches)
    for a, b in zip(w.batches, batches_o):
        assert np.array_equal(a, b)
    k, v = next(workloads.kv_rows(w.n_rows, 8, 64, seed=11, chunk_rows=1 << 20))
    pool, host = device_pool_for(w), host_pool_for(w)
    run_appends(w, k, v, pool, host)
    pk, pv, pks, pvs = pool.snapshot()
    assert_bits_equal(pk, host.k, "k pages")
    assert_bits_equal(pv, host.v, "v pages")
    if dtype in (airkv.INT8, airkv.FP8):
        assert_bits_equal(pks, host.k_scales, "k scales")
        assert_bits_equal(pvs, host.v_scales, "v scales")
    assert pool.error_count() == 0

    tables, lens = w.tables()
    assert lens.tolist() == [53, 144, 216, 527]
    assert [int((t >= 0).sum()) for t in tables] == [4, 9, 14, 33]
    for s, so in zip(w.seqs, seqs_o):
        assert w.mgr.table(s).physical_blocks == mgr_o.table(so).physical_blocks
    outs = [airkv.F32] if dtype == airkv.F32 else [airkv.F32, airkv.BF16]
    rows = _seq_rows(w, C1_PREFILL, 16)
    for out_dtype in outs:
        for layout in (airkv.LAYOUT_HEAD_MAJOR, airkv.LAYOUT_TOKEN_MAJOR):
            gk, gv, offs = _gather(pool, tables, lens, out_dtype, layout)
            hk, hv, hoffs, bad = host.gather(tables, lens, out_dtype, layout)
            assert bad == 0 and np.array_equal(offs, hoffs)
            assert_bits_equal(gk, hk, f"gathered k out={out_dtype} layout={layout}")
            assert_bits_equal(gv, hv, f"gathered v out={out_dtype} layout={layout}")
            if dtype == airkv.F32 and layout == airkv.LAYOUT_TOKEN_MAJOR:
                # gather(append(x)) == x, bit for bit
                for b, r in enumerate(rows):
                    n = len(r) * 8 * 64
                    assert_bits_equal(gk[offs[b]:offs[b] + n].reshape(len(r), 8, 64), k[r], "roundtrip k")
                    assert_bits_equal(gv[offs[b]:offs[b] + n].reshape(len(r), 8, 64), v[r], "roundtrip v")
    if dtype == airkv.BF16:
        gk, _, offs = _gather(pool, tables, lens, airkv.BF16, airkv.LAYOUT_TOKEN_MAJOR)
        for b, r in enumerate(rows):
            n = len(r) * 8 * 64
            assert_bits_equal(gk[offs[b]:offs[b] + n].reshape(len(r), 8, 64),
                              oracle.bf16_from_f32(k[r]), "bf16 roundtrip == rne(x)")
    if dtype == airkv.INT8:
        # the direct pin: dequantized gather of sequence b equals the
        # reference Q8Tensor::quantize/dequantize of its dense [seq, heads,
        # dim] tensor flattened (src/kv_cache.rs:307-315, :54-92)
        gk, _, offs = _gather(pool, tables, lens, airkv.F32, airkv.LAYOUT_TOKEN_MAJOR)
        for b, r in enumerate(rows):
            q, s = oracle.q8_quantize(k[r].reshape(-1))
            n = len(r) * 8 * 64
            assert_bits_equal(gk[offs[b]:offs[b] + n], oracle.q8_dequantize(q, s), "Q8Tensor pin")


@pytest.mark.parametrize("dtype,head_dim,bs,scale_group", [
    (airkv.F32, 96, 16, 32), (airkv.BF16, 160, 32, 32), (airkv.INT8, 224, 16, 32), (airkv.FP8, 32, 32, 32),
    (airkv.BF16, 256, 16, 32), (airkv.INT8, 96, 32, 16), (airkv.FP8, 256, 16, 128), (airkv.BF16, 32, 16, 32),
    (airkv.INT8, 128, 16, 8), (airkv.FP8, 128, 32, 8), (airkv.INT8, 128, 32, 128), (airkv.FP8, 128, 16, 16)])
def test_append_gather_other_head_dims(dtype, head_dim, bs, scale_group):
    """head_dim 32 .. 256 beyond 64 and 128 (the pool takes any multiple of
    32), and 1-byte pages at head_dim 128 with scale groups of 8 .. 128
    elements (2 .. 32 lanes of the whole-line append): pages, scales and
    both gather layouts bit-exact with the oracle."""
    log(f"append/gather dtype={dtype} head_dim={head_dim} bs={bs} scale_group={scale_group}")
    cfg = workloads.Config("hd", 8, 4, head_dim, bs, dtype, 5, scale_group=scale_group)
    w = workloads.build_prefill_decode(cfg, [1, 33, 100, 257, 600], seed=120 + head_dim, decode_steps=3)
    k, v = next(workloads.kv_rows(w.n_rows, 4, head_dim, seed=121 + head_dim, chunk_rows=1 << 20))
    pool, host = device_pool_for(w), host_pool_for(w)
    run_appends(w, k, v, pool, host)
    pk, pv, pks, pvs = pool.snapshot()
    assert_bits_equal(pk, host.k, "k pages")
    assert_bits_equal(pv, host.v, "v pages")
    if dtype in (airkv.INT8, airkv.FP8):
        assert_bits_equal(pks, host.k_scales, "k scales")
        assert_bits_equal(pvs, host.v_scales, "v scales")
    tables, lens = w.tables()
    outs = [airkv.F32] if dtype == airkv.F32 else [airkv.F32, airkv.BF16]
    for out_dtype in outs:
        for layout in (airkv.LAYOUT_HEAD_MAJOR, airkv.LAYOUT_TOKEN_MAJOR):
            gk, gv, offs = _gather(pool, tables, lens, out_dtype, layout)
            hk, hv, hoffs, bad = host.gather(tables, lens, out_dtype, layout)
            assert bad == 0 and np.array_equal(offs, hoffs)
            assert_bits_equal(gk, hk, f"gathered k out={out_dtype} layout={layout}")
            assert_bits_equal(gv, hv, f"gathered v out={out_dtype} layout={layout}")
    assert pool.error_count() == 0


@pytest.mark.parametrize("name", ["f32", "bf16", "int8", "fp8"])
def test_c1_against_committed_digests(name):
    """The GPU's c1 pages, scales and gathered views hash to the digests the
    oracle committed in tests/golden/c1_digests.json (inputs from the
    reference LCG / Box-Muller streams), so an oracle and a kernel that
    drifted together across commits would still be caught."""
    import json
    import os
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import c1_digests as c1
    with open(c1.JSON_PATH) as f:
        doc = json.load(f)["digests"]
    log(f"c1 digests dtype={name}")
    w, batches, tables, lens, k, v = c1.workload()
    assert c1.sha(k) == doc["inputs"]["k_rows"] and c1.sha(v) == doc["inputs"]["v_rows"], \
        "input generator differs on this host"
    assert c1.sha(np.concatenate(batches)) == doc["inputs"]["slots"]
    assert c1.sha(tables) == doc["inputs"]["tables"] and c1.sha(lens) == doc["inputs"]["lens"]
    w.cfg = workloads.Config(w.cfg.name, 8, 8, 64, 16, c1.DTYPES[name], 4)
    pool = device_pool_for(w)
    run_appends(w, k, v, pool)
    want = doc[name]
    pk, pv, pks, pvs = pool.snapshot()
    assert c1.sha(pk) == want["k_pages"] and c1.sha(pv) == want["v_pages"]
    if "k_scales" in want:
        assert c1.sha(pks) == want["k_scales"] and c1.sha(pvs) == want["v_scales"]
    for od in c1.out_dtypes(name):
        for layout in (airkv.LAYOUT_HEAD_MAJOR, airkv.LAYOUT_TOKEN_MAJOR):
            gk, gv, _ = _gather(pool, tables, lens, c1.DTYPES[od], layout)
            assert [c1.sha(gk), c1.sha(gv)] == want[f"gather_{od}_layout{layout}"], (od, layout)
    assert pool.error_count() == 0


def test_untouched_slots_keep_their_contents():
    """Every appended slot is written exactly once; all other bytes of the
    pool are left alone (pages pre-filled with a sentinel via write_blocks)."""
    torch = torch_mod()
    w = workloads.c1_workload(seed=9)
    w.cfg = workloads.Config(w.cfg.name, 8, 8, 64, 16, airkv.BF16, 4)
    pool, host = device_pool_for(w), host_pool_for(w, fill=0x7BCD)
    sentinel = np.full((w.num_blocks, pool.block_bytes // 2), 0x7BCD, np.uint16).view(np.uint8)
    pool.write_blocks(np.arange(w.num_blocks, dtype=np.int32), sentinel)
    k, v = next(workloads.kv_rows(w.n_rows, 8, 64, seed=12, chunk_rows=1 << 20))
    run_appends(w, k, v, pool, host)
    pk, pv, _, _ = pool.snapshot()
    assert_bits_equal(pk, host.k, "k pages")
    assert_bits_equal(pv, host.v, "v pages")
    written = set()
    for slots in w.batches:
        for s in slots.tolist():
            assert s not in written
            written.add(s)
    assert len(written) == w.n_rows
    untouched = np.ones(w.num_blocks * 16, bool)
    untouched[list(written)] = False
    rows = pk.transpose(0, 2, 1, 3).reshape(w.num_blocks * 16, -1)
    assert np.all(rows[untouched] == 0x7BCD)
    torch.cuda.synchronize()


def _special_rows(n_rows, d, seed):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2 ** 32, size=(n_rows, d), dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32).copy()
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -1e-40, 1.4e-45, 448.0, -448.0,
                         256.0, 255.99998, 240.0, 1.0625, -1.0625, 1.9375, 2.5, -2.5, 0.5,
                         3.4e38, -3.4e38, 1e-8, 9e-9, 127.0], np.float32)
    for i in range(0, n_rows, 3):
        x[i, :len(specials)] = specials
        rng.shuffle(x[i])
    # some rows of small normal values (realistic magnitudes)
    x[1::3] = rng.standard_normal((len(x[1::3]), d)).astype(np.float32)
    # rows with one huge outlier per group
    x[2::3] = rng.standard_normal((len(x[2::3]), d)).astype(np.float32)
    x[2::3, ::32] *= 1e4
    return x


@pytest.mark.parametrize("dtype", [airkv.BF16, airkv.INT8, airkv.FP8])
def test_codec_edge_cases_bitexact(dtype):
    """Random bit patterns (NaN, inf, denormals, huge) plus hand-picked
    boundary values: codes and scales match the oracle bit for bit."""
    torch = torch_mod()
    log(f"codec edge cases dtype={dtype}")
    nkv, d, bs, nb = 4, 128, 16, 64
    n = nb * bs
    k = _special_rows(n * nkv, d, 21).reshape(n, nkv, d)
    v = _special_rows(n * nkv, d, 22).reshape(n, nkv, d)
    slots = workloads.lcg_permutation(n, 5).astype(np.int64)
    pool = airkv.KvPool(nb, bs, nkv, d, dtype, 32)
    host = oracle.HostPool(nb, bs, nkv, d, dtype, 32)
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), torch.from_numpy(slots).cuda())
    host.append(k, v, slots)
    pk, pv, pks, pvs = pool.snapshot()
    assert_bits_equal(pk, host.k, "k codes")
    assert_bits_equal(pv, host.v, "v codes")
    if dtype != airkv.BF16:
        assert_bits_equal(pks, host.k_scales, "k scales")
        assert_bits_equal(pvs, host.v_scales, "v scales")


def _q8_tie_groups(n_groups, seed):
    """Groups of 32 N(0,1) values in which some x * (1/scale) rounds (in f32)
    to an exact k + 0.5 while the exact product does not: f32::round must
    see the rounded product (half away from zero), not a fused one."""
    rng = np.random.default_rng(seed)
    found = []
    while len(found) < n_groups:
        x = rng.standard_normal((1 << 15, 32)).astype(np.float32)
        m = np.abs(x).max(1)
        scale = m / np.float32(127.0)
        inv = np.float32(1.0) / scale
        prod = x * inv[:, None]
        tie = (prod - np.trunc(prod) == np.float32(0.5)) | (prod - np.trunc(prod) == np.float32(-0.5))
        exact = x.astype(np.float64) * inv.astype(np.float64)[:, None]
        tie &= exact != prod.astype(np.float64)
        for i in np.nonzero(tie.any(1))[0][: n_groups - len(found)]:
            found.append(x[i])
    return np.stack(found)


def test_q8_rounding_ties_bitexact():
    torch = torch_mod()
    groups = _q8_tie_groups(64, 31)             # 64 groups -> 16 rows of 128
    rows = groups.reshape(16, 1, 128)
    pool = airkv.KvPool(1, 16, 1, 128, airkv.INT8, 32)
    host = oracle.HostPool(1, 16, 1, 128, airkv.INT8, 32)
    t = torch.from_numpy(rows).cuda()
    slots = np.arange(16, dtype=np.int64)
    pool.append(t, t, torch.from_numpy(slots).cuda())
    host.append(rows, rows, slots)
    pk, _, pks, _ = pool.snapshot()
    assert_bits_equal(pks, host.k_scales, "tie scales")
    assert_bits_equal(pk, host.k, "tie codes")


def test_fp8_encoder_sweep_all_high_halves():
    """The encoder's result depends only on the sign, exponent and the top
    four mantissa bits (plus NaN-ness), so every 16-bit high half with low
    halves {0x0000, 0x0001, 0xFFFF} exercises every branch and rounding
    case.  Groups carry 448.0 so the scale is exactly 1 and the code is
    F8E4M3::from_f32(x) itself."""
    torch = torch_mod()
    log("fp8 encoder sweep")
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    xs = np.concatenate([(hi | lo).view(np.float32) for lo in (0x0000, 0x0001, 0xFFFF)])
    a = np.abs(xs)
    xs = xs[~(a > 448.0)]                      # keeps NaNs and |x| <= 448
    per_group = 31
    ng = -(-len(xs) // per_group)
    pad = np.zeros(ng * per_group, np.float32)
    pad[:len(xs)] = xs
    groups = np.concatenate([np.full((ng, 1), 448.0, np.float32), pad.reshape(ng, per_group)], 1)
    d = 128
    nrows = -(-groups.shape[0] // 4)          # 4 groups of 32 per row
    full = np.zeros((nrows * 4, 32), np.float32)
    full[:, 0] = 448.0
    full[:groups.shape[0]] = groups
    rows = full.reshape(nrows, 1, d)
    bs = 16
    nb = -(-nrows // bs)
    pool = airkv.KvPool(nb, bs, 1, d, airkv.FP8, 32)
    slots = torch.arange(nrows, dtype=torch.int64, device="cuda")
    t = torch.from_numpy(rows).cuda()
    pool.append(t, t, slots)
    pk, _, pks, _ = pool.snapshot()
    codes = pk.reshape(-1, 32)[:full.shape[0]]
    scales = pks.reshape(-1)[:full.shape[0]]
    assert np.all(scales == 1.0)
    want = oracle.fp8_from_f32(full)
    assert_bits_equal(codes, want, "fp8 codes")


def test_invalid_slots_are_skipped_and_counted():
    torch = torch_mod()
    pool = airkv.KvPool(4, 16, 2, 64, airkv.BF16, 32)
    pool.error_count(reset=True)
    k = torch.randn(3, 2, 64, device="cuda")
    slots = torch.tensor([5, 64, -1], dtype=torch.int64, device="cuda")   # 64 == 4 * 16: out of range
    pool.append(k, k, slots)
    assert pool.error_count(reset=True) == 1
    pk, _, _, _ = pool.snapshot()
    rows = pk.transpose(0, 2, 1, 3).reshape(64, 2, 64)
    assert np.array_equal(rows[5], oracle.bf16_from_f32(k[0].cpu().numpy()))
    assert np.count_nonzero(np.delete(rows, 5, axis=0)) == 0
    # a table entry outside the pool within seq_len: skipped and counted
    tables = torch.tensor([[0, 99]], dtype=torch.int32, device="cuda")
    lens = torch.tensor([20], dtype=torch.int32, device="cuda")
    out = torch.zeros(20 * 2 * 64, dtype=torch.bfloat16, device="cuda")
    pool.gather(tables, lens, torch.zeros(1, dtype=torch.int64, device="cuda"), out, out.clone())
    assert pool.error_count(reset=True) >= 1


def test_copy_blocks_and_swap_roundtrip():
    """CoW page copy, and evict/restore through the pool-backed swap
    callbacks: restored pages hold the evicted bytes under new block ids."""
    torch = torch_mod()
    cfg = workloads.Config("swap", 8, 4, 128, 16, airkv.INT8, 2)
    pool = airkv.KvPool(32, 16, 4, 128, airkv.INT8, 32)
    swap = airkv.KvSwapManager(32, pool.block_bytes, 16)
    mgr = swap.seq_mgr
    s = mgr.create_sequence()
    slots = mgr.append_slots(s, 40)
    k = torch.randn(40, 4, 128, device="cuda")
    v = torch.randn(40, 4, 128, device="cuda")
    pool.append(k, v, torch.from_numpy(slots).cuda())
    before = pool.read_blocks(mgr.table(s).physical_blocks)
    # CoW: fork, copy the shared last block, compare
    c = mgr.fork_sequence(s)
    old, new = mgr.cow_last_block(c)
    assert old != new
    pool.copy_blocks(torch.tensor([old], dtype=torch.int32, device="cuda"),
                     torch.tensor([new], dtype=torch.int32, device="cuda"))
    assert np.array_equal(pool.read_blocks([new]), pool.read_blocks([old]))
    mgr.free_sequence(c)
    cb = airkv.pool_callbacks(pool)
    released = swap.evict(s, cb[0:1] + cb[2:3])
    assert len(released) == 3 and swap.is_evicted(s)
    # scribble over the released blocks
    pool.write_blocks(released, np.zeros((3, pool.block_bytes), np.uint8))
    new_blocks = swap.restore(s, cb[1:2] + cb[2:3])
    assert len(new_blocks) == 3
    assert np.array_equal(pool.read_blocks(new_blocks), before)


def test_bound_launchers_keep_their_tensors_alive():
    """bind_append / bind_gather / bind_decode / bind_prefill return launchers
    that call the C ABI with raw device addresses; each launcher must hold the
    tensors those addresses point into.  With the caller's references dropped
    and same-sized tensors allocated in between (which would take over freed
    memory), every tensor is still alive -- checked before any launch -- and
    each launch gives the direct call's pages and outputs bit for bit."""
    import gc
    import weakref
    torch = torch_mod()
    cfg = workloads.Config("bind", 32, 8, 128, 16, airkv.BF16, 2)
    w = workloads.build_prefill_decode(cfg, [40, 70], seed=191, decode_steps=0)
    slots_np = np.concatenate(w.batches)
    pa = airkv.KvPool(w.num_blocks, 16, 8, 128, airkv.BF16)
    pb = airkv.KvPool(w.num_blocks, 16, 8, 128, airkv.BF16)
    g = torch.Generator(device="cuda")
    g.manual_seed(192)
    k = torch.randn(len(slots_np), 8, 128, generator=g, device="cuda")
    v = torch.randn_like(k)
    st = torch.from_numpy(slots_np).cuda()
    pa.append(k, v, st)
    launch_append = pb.bind_append(k.clone(), v.clone(), st.clone())   # only the launcher holds these
    refs = [weakref.ref(t) for t in launch_append.keep if isinstance(t, torch.Tensor)]
    tables, lens = w.tables()
    per = lens.astype(np.int64) * 8 * 128
    offs = np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)
    want_k = torch.zeros(int(per.sum()), dtype=torch.bfloat16, device="cuda")
    want_v = torch.zeros_like(want_k)
    tt, lt, ot = (torch.from_numpy(x).cuda() for x in (tables, lens, offs))
    pa.gather(tt, lt, ot, want_k, want_v)
    gk, gv = torch.zeros_like(want_k), torch.zeros_like(want_v)
    launch_gather = pb.bind_gather(tt.clone(), lt.clone(), ot.clone(), gk, gv)
    refs += [weakref.ref(t) for t in launch_gather.keep if isinstance(t, torch.Tensor)]
    q = torch.randn(2, 32, 128, generator=g, device="cuda").to(torch.bfloat16)
    want_o = torch.empty(2, 32, 128, device="cuda")
    pa.paged_decode(q, tt, lt, want_o)
    out = torch.empty_like(want_o)
    launch_decode = pb.bind_decode(q.clone(), tt.clone(), lt.clone(), out, None)
    refs += [weakref.ref(t) for t in launch_decode.keep if isinstance(t, torch.Tensor)]
    cu = torch.tensor([0, 8, 24], dtype=torch.int32, device="cuda")
    qp = torch.randn(24, 32, 128, generator=g, device="cuda").to(torch.bfloat16)
    want_p = torch.empty(24, 32, 128, device="cuda")
    pa.paged_prefill(qp, cu, tt, lt, want_p)
    outp = torch.empty_like(want_p)
    launch_prefill = pb.bind_prefill(qp.clone(), cu.clone(), tt.clone(), lt.clone(), outp)
    refs += [weakref.ref(t) for t in launch_prefill.keep if isinstance(t, torch.Tensor)]
    torch.cuda.synchronize()
    gc.collect()
    # same-sized allocations that would reuse any memory the launchers lost
    filler = [torch.full_like(t, 7) for t in (k, v, q, qp)] + [torch.full_like(x, -1) for x in (st, tt, lt, ot, cu)]
    assert len(refs) >= 17 and all(r() is not None for r in refs), "a launcher lost a tensor it writes through"
    del filler
    gk.zero_()
    gv.zero_()
    out.zero_()
    outp.zero_()
    launch_append()
    launch_gather()
    launch_decode()
    launch_prefill()
    torch.cuda.synchronize()
    pka, pva, _, _ = pa.snapshot()
    pkb, pvb, _, _ = pb.snapshot()
    assert np.array_equal(pka, pkb) and np.array_equal(pva, pvb)
    assert torch.equal(gk.view(torch.int16), want_k.view(torch.int16))
    assert torch.equal(gv.view(torch.int16), want_v.view(torch.int16))
    assert torch.equal(out, want_o) and torch.equal(outp, want_p)
    assert pa.error_count() == 0 and pb.error_count() == 0


@pytest.mark.parametrize("dtype", [airkv.INT8, airkv.FP8])
def test_quantized_append_head_dim_128_partial_waves_and_invalid_slots(dtype):
    """head_dim 128 quantized appends load each wave's four tokens as whole
    source lines and hand them between lanes: token counts that leave a
    wave partly filled, several kv heads, a skipped slot (-1) and an
    out-of-range one must still give the oracle's pages and scales bit for
    bit and count the out-of-range slot once."""
    torch = torch_mod()
    nb, bs, nkv, d = 8, 16, 3, 128
    pool = airkv.KvPool(nb, bs, nkv, d, dtype)
    host = oracle.HostPool(nb, bs, nkv, d, dtype, pool.scale_group)
    pool.error_count(reset=True)
    rng = np.random.default_rng(77 + dtype)
    for n in (1, 2, 3, 5, 7, 13):
        log(f"quantized append dtype={dtype} tokens={n}")
        slots = rng.choice(nb * bs, size=n, replace=False).astype(np.int64)
        if n >= 5:
            slots[1] = -1
            slots[3] = nb * bs + 5                              # outside the pool
        k = (rng.standard_normal((n, nkv, d)) * rng.uniform(0.1, 30.0)).astype(np.float32)
        v = (rng.standard_normal((n, nkv, d)) * rng.uniform(0.1, 30.0)).astype(np.float32)
        pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), torch.from_numpy(slots).cuda())
        want_bad = host.append(k, v, slots)
        assert pool.error_count(reset=True) == want_bad == (1 if n >= 5 else 0)
    torch.cuda.synchronize()
    pk, pv, ks, vs = pool.snapshot()
    assert_bits_equal(pk, host.k, "k codes")
    assert_bits_equal(pv, host.v, "v codes")
    assert_bits_equal(ks.view(np.uint32), host.k_scales.view(np.uint32), "k scales")
    assert_bits_equal(vs.view(np.uint32), host.v_scales.view(np.uint32), "v scales")
