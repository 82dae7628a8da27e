"""GPU parity: split-K paged decode attention against the oracle (gather +
flash_decode with chunk 64, src/flash_decode.rs:153-173) through the C ABI.

Tolerances (relative to max |reference|): 1e-3 for f32/bf16 caches and 2e-2
for int8/fp8 caches, the oracle running on the same dequantized cache.
"""
import numpy as np
import pytest

import airkv
import oracle
from airkv import workloads
from gpu_helpers import (assert_floats_bit_equal, decode_pieces, device_pool_for, host_pool_for, log, rel_err, run_appends,
                         torch_mod)

pytestmark = pytest.mark.gpu

TOL = {airkv.F32: 1e-3, airkv.BF16: 1e-3, airkv.INT8: 2e-2, airkv.FP8: 2e-2}


def _decode_case(cfg, lens, seed, q_bf16=True, max_splits=64, outliers=None, out_bf16=False,
                 empty=(), workspace=None):
    """Decode of cfg with prefill `lens` (+1 decode token each) on the GPU and
    on the oracle; sequences listed in `empty` are decoded with length 0."""
    torch = torch_mod()
    w = workloads.build_prefill_decode(cfg, lens, seed, decode_steps=1)
    k, v = next(workloads.kv_rows(w.n_rows, cfg.n_kv_heads, cfg.head_dim, seed=seed + 100,
                                  outliers=outliers, chunk_rows=1 << 24))
    pool, host = device_pool_for(w), host_pool_for(w)
    run_appends(w, k, v, pool, host)
    tables, seq_lens = w.tables()
    seq_lens[list(empty)] = 0
    rng = np.random.default_rng(seed + 7)
    q = rng.standard_normal((cfg.batch, cfg.n_q_heads, cfg.head_dim)).astype(np.float32)
    qt = torch.from_numpy(q).cuda()
    if q_bf16:
        qt = qt.to(torch.bfloat16)
        q = qt.float().cpu().numpy()
    out = torch.zeros(q.shape, dtype=torch.bfloat16 if out_bf16 else torch.float32, device="cuda")
    if workspace == "new":
        workspace = pool.new_workspace(cfg.n_q_heads, cfg.batch, tables.shape[1], max_splits)
    pool.paged_decode(qt, torch.from_numpy(tables).cuda(), torch.from_numpy(seq_lens).cuda(), out,
                      max_splits=max_splits, workspace=workspace)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    want = host.paged_decode(q, tables, seq_lens, chunk=64)
    assert pool.error_count() == 0
    return got, want, (pool, host, tables, seq_lens, q, workspace)


@pytest.mark.parametrize("dtype", [airkv.F32, airkv.BF16, airkv.INT8, airkv.FP8])
@pytest.mark.parametrize("group", [1, 4, 6, 8, 16])
def test_decode_matches_oracle_small(dtype, group):
    """Groups of 1 .. 16 query heads per kv head (the matrix-core path takes
    any group up to 16; lanes of heads past the group read zeros), including
    one that is not a power of two."""
    log(f"decode small dtype={dtype} group={group}")
    nkv = 2 if group >= 8 else 4
    cfg = workloads.Config("small", nkv * group, nkv, 128, 16, dtype, 5)
    lens = [1, 17, 64, 300, 777]
    got, want, _ = _decode_case(cfg, lens, seed=30 + group)
    err = rel_err(got, want)
    log(f"  rel err {err:.2e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype,n_kv,group", [(airkv.F32, 2, 12), (airkv.BF16, 1, 32), (airkv.INT8, 2, 20),
                                              (airkv.FP8, 1, 24)])
def test_decode_groups_above_16(dtype, n_kv, group):
    """Query heads per kv head beyond the matrix-core kernel's 16 (multi-query
    attention: one kv head for all heads; the reference takes any ratio,
    src/chunked_attn.rs:65-72): the split kernel serves the group eight heads
    per workgroup, the last workgroup's heads past the group masked."""
    log(f"decode group {group} dtype={dtype}")
    cfg = workloads.Config("mqa", n_kv * group, n_kv, 128, 16, dtype, 4)
    got, want, _ = _decode_case(cfg, [5, 64, 333, 900], seed=90 + group)
    err = rel_err(got, want)
    log(f"  rel err {err:.2e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype,head_dim,group", [(airkv.F32, 96, 4), (airkv.BF16, 160, 2), (airkv.INT8, 32, 8),
                                                  (airkv.FP8, 224, 3), (airkv.BF16, 192, 16)])
def test_decode_other_head_dims(dtype, head_dim, group):
    """head_dim a multiple of 32 that is not 64, 128 or 256 (the pool takes any
    up to 256): the split kernel's lanes past head_dim idle."""
    log(f"decode head_dim {head_dim} dtype={dtype} group={group}")
    cfg = workloads.Config("hd", 2 * group, 2, head_dim, 16, dtype, 4)
    got, want, _ = _decode_case(cfg, [3, 70, 257, 640], seed=110 + head_dim)
    err = rel_err(got, want)
    log(f"  rel err {err:.2e}")
    assert err <= TOL[dtype]


def test_c2_shape_bf16_scaled():
    """configs[1] geometry (32 q / 8 kv, d 128, bs 16) at batch 8 and
    contexts U[512, 1500], q in bf16."""
    cfg = workloads.Config("c2s", 32, 8, 128, 16, airkv.BF16, 8)
    lens = workloads.c2_lengths(8, 512, 1500, seed=2)
    got, want, _ = _decode_case(cfg, lens, seed=41)
    err = rel_err(got, want)
    log(f"c2 scaled rel err {err:.2e}")
    assert err <= 1e-3


def test_c3_shape_int8_outliers_scaled():
    """configs[2] geometry (64 q / 8 kv, int8 Q8_0) with 1% outlier channels
    x20, batch 3, context 1000."""
    cfg = workloads.Config("c3s", 64, 8, 128, 16, airkv.INT8, 3)
    out_ch = workloads.outlier_channels(8, 128)
    got, want, _ = _decode_case(cfg, [1000, 1000, 1000], seed=43, outliers=out_ch)
    err = rel_err(got, want)
    log(f"c3 scaled rel err {err:.2e}")
    assert err <= 2e-2


def test_slices_span_and_share_sequences():
    """Matrix-core path (bf16, d 128): 300 short sequences (1..80 tokens, some
    decoded empty) and two long ones.  The balanced slices then end inside
    sequences, hold several sequences each, and the long sequences spread over
    many slices; every case must agree with the oracle."""
    cfg = workloads.Config("mix", 32, 8, 128, 16, airkv.BF16, 300)
    rng = np.random.default_rng(60)
    lens = rng.integers(0, 80, size=300)
    lens[7], lens[150] = 6000, 2500
    empty = [0, 1, 33, 34, 35, 299]
    got, want, _ = _decode_case(cfg, lens.tolist(), seed=61, empty=empty)
    assert np.count_nonzero(got[empty]) == 0
    err = rel_err(got, want)
    log(f"mixed slices rel err {err:.2e}")
    assert err <= 1e-3


@pytest.mark.parametrize("max_splits", [1, 3])
def test_slices_capped_by_max_splits(max_splits):
    """max_splits caps the slices per kv head at batch x max_splits (here far
    fewer than the GPU's waves): long slices, the same answers."""
    cfg = workloads.Config("cap", 32, 8, 128, 32, airkv.BF16, 4)
    got, want, _ = _decode_case(cfg, [3000, 17, 900, 4100], seed=62, max_splits=max_splits)
    err = rel_err(got, want)
    log(f"max_splits={max_splits} rel err {err:.2e}")
    assert err <= 1e-3


def test_batch_above_one_launch():
    """More sequences than one launch takes (4096): the host runs the batch
    in consecutive launches over the same workspace."""
    cfg = workloads.Config("wide", 8, 2, 128, 16, airkv.BF16, 4200)
    rng = np.random.default_rng(63)
    lens = rng.integers(1, 40, size=4200)
    got, want, _ = _decode_case(cfg, lens.tolist(), seed=64, empty=[4095, 4096])
    err = rel_err(got, want)
    log(f"batch 4200 rel err {err:.2e}")
    assert err <= 1e-3


def test_c4_shape_fp8_many_splits():
    """configs[3] geometry (fp8, bs 32) with contexts long enough that each
    sequence is spread over ~100 slices, merged by log-sum-exp."""
    cfg = workloads.Config("c4s", 64, 8, 128, 32, airkv.FP8, 2)
    got, want, _ = _decode_case(cfg, [20000, 9000], seed=44)
    err = rel_err(got, want)
    log(f"c4 scaled rel err {err:.2e}")
    assert err <= 2e-2


@pytest.mark.parametrize("dtype,max_splits", [(airkv.FP8, 2), (airkv.FP8, 8), (airkv.FP8, 64),
                                              (airkv.INT8, 5), (airkv.BF16, 3)])
def test_pieces_per_sequence_capped_by_max_splits(dtype, max_splits):
    """max_splits bounds the pieces of every sequence, not only the slice
    count: with one long and one shorter sequence (configs[3]'s geometry, fp8
    / int8 / bf16 pages) the balanced slices would cut the long one into
    ~100 pieces; the kernel widens the slices until it has at most
    max_splits.  The pieces come from the workspace's tile prefix and slice
    length; the output agrees with the oracle."""
    cfg = workloads.Config("c4cap", 64, 8, 128, 32, dtype, 3)
    got, want, ctx = _decode_case(cfg, [20000, 9000, 300], seed=45, max_splits=max_splits, workspace="new")
    pieces = decode_pieces(ctx[5], ctx[3])
    err = rel_err(got, want)
    log(f"dtype={dtype} max_splits={max_splits}: pieces {pieces.tolist()}, rel err {err:.2e}")
    assert pieces.max() <= max_splits
    if max_splits == 64:
        assert pieces[0] > 8          # the long sequence still spreads over many waves
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype", [airkv.INT8, airkv.FP8])
@pytest.mark.parametrize("head_dim,scale_group", [(64, 32), (128, 16), (128, 64), (256, 128)])
def test_quantized_pool_geometries(dtype, head_dim, scale_group):
    """1-byte pools of every geometry: head_dim 128 with scale groups of 32 or
    more takes the matrix-core kernel, the others (head_dim 64 / 256, groups
    of 16) the vector kernel; both against the oracle on the dequantized
    cache."""
    cfg = workloads.Config("qgeo", 16, 2, head_dim, 16, dtype, 4, scale_group=scale_group)
    got, want, _ = _decode_case(cfg, [5, 300, 1000, 64], seed=47 + head_dim + scale_group)
    err = rel_err(got, want)
    log(f"dtype={dtype} d={head_dim} sg={scale_group} rel err {err:.2e}")
    assert err <= 2e-2


def test_c5_shape_bf16_block32():
    """configs[4] geometry (bf16, block_size 32) with lognormal contexts."""
    cfg = workloads.Config("c5s", 32, 8, 128, 32, airkv.BF16, 6)
    lens = workloads.c5_lengths(6, median=300, lo=16, hi=2000, seed=8)
    got, want, _ = _decode_case(cfg, lens, seed=45)
    err = rel_err(got, want)
    log(f"c5 scaled rel err {err:.2e}")
    assert err <= 1e-3


@pytest.mark.parametrize("batch,lo,hi,dtype", [(300, 16, 700, airkv.BF16), (160, 300, 900, airkv.INT8),
                                                (3, 20000, 30000, airkv.BF16)])
def test_merge_modes(batch, lo, hi, dtype):
    """The merge kernel's modes, picked from slices per sequence: many short
    sequences (about two pieces each, four-piece batches), a middle case, and
    a few long sequences (four waves per query head), plus an empty sequence."""
    log(f"merge modes batch={batch} lens=[{lo}, {hi}) dtype={dtype}")
    cfg = workloads.Config("merge", 32, 8, 128, 16, dtype, batch)
    rng = np.random.default_rng(batch)
    lens = [int(x) for x in rng.integers(lo, hi, batch)]
    got, want, _ = _decode_case(cfg, lens, seed=60 + batch, empty=(batch // 2,))
    err = rel_err(got, want)
    log(f"  rel err {err:.2e}")
    assert err <= TOL[dtype]
    assert np.count_nonzero(got[batch // 2]) == 0


@pytest.mark.parametrize("q_bf16,out_bf16", [(False, False), (False, True), (True, True)])
def test_bf16_group16_query_and_output_dtypes(q_bf16, out_bf16):
    """GQA group 16 (32 q / 2 kv heads); f32 queries take the split hi/lo
    bf16 path, bf16 outputs are rounded once at the end."""
    cfg = workloads.Config("g16", 32, 2, 128, 16, airkv.BF16, 3)
    got, want, _ = _decode_case(cfg, [40, 513, 2100], seed=46, q_bf16=q_bf16, out_bf16=out_bf16)
    err = rel_err(got, want)
    log(f"g16 q_bf16={q_bf16} out_bf16={out_bf16} rel err {err:.2e}")
    assert err <= (4e-3 if out_bf16 else 1e-3)


@pytest.mark.parametrize("dtype,bs", [(airkv.INT8, 16), (airkv.FP8, 32)])
def test_one_byte_pages_f32_queries(dtype, bs):
    """1-byte pools round f32 queries to bf16 once: the output equals, bit for
    bit, that of the same queries given as bf16, and stays within the 2e-2
    tolerance of the oracle's f32-query attention (c3 / c4 head geometry,
    outlier channels)."""
    torch = torch_mod()
    cfg = workloads.Config("q32", 64, 8, 128, bs, dtype, 4)
    outl = workloads.outlier_channels(8, 128, seed=9)
    got, want, (pool, host, tables, lens, q, _) = _decode_case(cfg, [300, 1700, 4100, 9000], seed=48,
                                                           q_bf16=False, outliers=outl)
    err = rel_err(got, want)
    qb = torch.from_numpy(q).cuda().to(torch.bfloat16)
    out_b = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    pool.paged_decode(qb, torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda(), out_b)
    torch.cuda.synchronize()
    assert_floats_bit_equal(got, out_b.cpu().numpy(), "f32 queries against the same queries in bf16")
    log(f"1-byte dtype={dtype} f32 queries rel err {err:.2e}")
    assert err <= TOL[dtype]


def test_workspace_reuse_across_calls():
    """Calls that share one workspace give the same answers as fresh
    workspaces, for varying batches."""
    torch = torch_mod()
    cfg = workloads.Config("reuse", 32, 8, 128, 16, airkv.BF16, 6)
    w = workloads.build_prefill_decode(cfg, [700, 1500, 33, 2600, 260, 900], seed=47)
    k, v = next(workloads.kv_rows(w.n_rows, 8, 128, seed=48, chunk_rows=1 << 24))
    pool = device_pool_for(w)
    run_appends(w, k, v, pool)
    tables, lens = w.tables()
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
    ws = pool.new_workspace(32, 6, tables.shape[1], 64)
    for it in range(6):
        nb = [6, 3, 6, 1, 5, 6][it]
        q = torch.randn(nb, 32, 128, device="cuda").to(torch.bfloat16)
        out = torch.empty(nb, 32, 128, device="cuda")
        pool.paged_decode(q, tt[:nb].contiguous(), lt[:nb].contiguous(), out, workspace=ws)
        ref = torch.empty_like(out)
        pool.paged_decode(q, tt[:nb].contiguous(), lt[:nb].contiguous(), ref)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), it


@pytest.mark.parametrize("kv_len,seed_q,bound,chunk", [(128, 1, 1e-4, 32), (4096, 10, 1e-3, 64),
                                                       (32, 20, 1e-5, 32)])
def test_reference_flash_decode_inputs(kv_len, seed_q, bound, chunk):
    """The reference's own flash_decode tests (src/flash_decode.rs:232-275):
    the same LCG inputs (HD 64, one head) stored in an f32 paged pool; the
    GPU output must meet the reference's L-inf bound against
    reference_attention."""
    torch = torch_mod()
    hd = 64
    q = oracle.lcg_fill(seed_q, hd)
    k = oracle.lcg_fill(seed_q + 1, kv_len * hd).reshape(kv_len, 1, hd)
    v = oracle.lcg_fill(seed_q + 2, kv_len * hd).reshape(kv_len, 1, hd)
    nb = -(-kv_len // 16)
    pool = airkv.KvPool(nb, 16, 1, hd, airkv.F32, 32)
    slots = torch.from_numpy(workloads.lcg_permutation(nb, 77).astype(np.int64)).cuda()
    slots = (slots[:, None] * 16 + torch.arange(16, device="cuda")[None, :]).reshape(-1)[:kv_len]
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), slots.contiguous())
    table = (slots[::16] // 16).to(torch.int32).reshape(1, -1).contiguous()
    out = torch.zeros(1, 1, hd, device="cuda")
    pool.paged_decode(torch.from_numpy(q).cuda().reshape(1, 1, hd), table,
                      torch.tensor([kv_len], dtype=torch.int32, device="cuda"), out)
    got = out.cpu().numpy().reshape(hd)
    want = oracle.reference_attention(q, k.reshape(-1), v.reshape(-1), kv_len, hd)
    assert oracle.max_abs_error(got, want) < bound
    assert oracle.max_abs_error(got, oracle.flash_decode(q, k.reshape(-1), v.reshape(-1), kv_len, hd,
                                                         chunk)) < bound


def test_special_cases():
    """Closed forms: a single token returns its V row; identical keys give the
    mean of V; an empty sequence gives zeros; max_splits does not change the
    answer beyond rounding."""
    torch = torch_mod()
    d = 128
    pool = airkv.KvPool(64, 16, 1, d, airkv.F32, 32)
    k = torch.randn(1, d, device="cuda").repeat(200, 1).reshape(200, 1, d)
    v = torch.randn(200, 1, d, device="cuda")
    pool.append(k.contiguous(), v, torch.arange(200, dtype=torch.int64, device="cuda"))
    table = torch.arange(13, dtype=torch.int32, device="cuda").reshape(1, 13).repeat(3, 1).contiguous()
    lens = torch.tensor([1, 200, 0], dtype=torch.int32, device="cuda")
    q = torch.randn(3, 1, d, device="cuda")
    out = torch.full((3, 1, d), 7.0, device="cuda")
    pool.paged_decode(q, table, lens, out, max_splits=1)
    assert torch.equal(out[0, 0], v[0, 0])
    assert torch.allclose(out[1, 0], v.mean(0)[0], atol=1e-5)
    assert torch.count_nonzero(out[2]) == 0
    out2 = torch.empty_like(out)
    pool.paged_decode(q, table, lens, out2, max_splits=64)
    assert torch.allclose(out, out2, atol=1e-5)


def test_full_c2_against_torch_fp32():
    """configs[1] at full size (batch 64, contexts U[512, 4096], pool 1.25x):
    the paged decode agrees with a plain torch float32 attention over the
    gathered per-sequence K/V within 1e-3 relative."""
    torch = torch_mod()
    log("full c2")
    cfg = workloads.CONFIGS["c2"]
    lens = workloads.c2_lengths()
    w = workloads.build_prefill_decode(cfg, lens, seed=2)
    pool = device_pool_for(w)
    gen = workloads.kv_rows(w.n_rows, 8, 128, seed=5, device="cuda", chunk_rows=1 << 16)
    buf_k, buf_v, have = None, None, 0
    for slots in w.batches:
        n = len(slots)
        parts_k, parts_v = [], []
        while n > 0:
            if buf_k is None or have == buf_k.shape[0]:
                buf_k, buf_v = next(gen)
                have = 0
            take = min(n, buf_k.shape[0] - have)
            parts_k.append(buf_k[have:have + take])
            parts_v.append(buf_v[have:have + take])
            have += take
            n -= take
        pool.append(torch.cat(parts_k).contiguous(), torch.cat(parts_v).contiguous(),
                    torch.from_numpy(slots).cuda())
    tables, seq_lens = w.tables()
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(seq_lens).cuda()
    q = torch.randn(64, 32, 128, device="cuda").to(torch.bfloat16)
    out = torch.empty(64, 32, 128, device="cuda")
    pool.paged_decode(q, tt, lt, out)
    per = seq_lens.astype(np.int64) * 8 * 128
    offs = np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)
    gk = torch.empty(int(per.sum()), dtype=torch.bfloat16, device="cuda")
    gv = torch.empty_like(gk)
    pool.gather(tt, lt, torch.from_numpy(offs).cuda(), gk, gv)
    worst = 0.0
    for b in range(64):
        L = int(seq_lens[b])
        K = gk[offs[b]:offs[b] + L * 1024].view(8, L, 128).float()
        V = gv[offs[b]:offs[b] + L * 1024].view(8, L, 128).float()
        qb = q[b].float().view(8, 4, 128)
        s = torch.matmul(qb, K.transpose(1, 2).contiguous()) / np.sqrt(128.0)
        p = torch.softmax(s, dim=-1)
        ref = torch.matmul(p, V).reshape(32, 128)
        worst = max(worst, (out[b] - ref).abs().max().item() / ref.abs().max().item())
    log(f"full c2 worst rel err {worst:.2e}")
    assert worst <= 1e-3
    assert pool.error_count() == 0
