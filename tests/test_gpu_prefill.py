"""GPU parity: paged prefill attention (chunked, causal) against the oracle's
blockwise_attention_head per query head with q_offset = seq_len - q_len
(src/chunked_attn.rs:114-213), through the C ABI.

Tolerances (relative to max |reference|): 1e-3 for bf16 caches, 2e-2 for
int8 / fp8 caches, the oracle running on the same dequantized cache.
"""
import ctypes

import numpy as np
import pytest

import airkv
import oracle
from airkv import workloads
from gpu_helpers import device_pool_for, host_pool_for, log, rel_err, run_appends, torch_mod

pytestmark = pytest.mark.gpu

TOL = {airkv.BF16: 1e-3, airkv.INT8: 2e-2, airkv.FP8: 2e-2}


def _setup(cfg, ctx_lens, seed, outliers=None):
    w = workloads.build_prefill_decode(cfg, ctx_lens, seed, decode_steps=0)
    k, v = next(workloads.kv_rows(w.n_rows, cfg.n_kv_heads, cfg.head_dim, seed=seed + 100,
                                  outliers=outliers, chunk_rows=1 << 24))
    pool, host = device_pool_for(w), host_pool_for(w)
    run_appends(w, k, v, pool, host)
    tables, lens = w.tables()
    return pool, host, tables, lens


def _prefill_case(cfg, ctx_lens, q_lens, seed, q_bf16=True, out_bf16=False, max_q_len=None,
                  outliers=None, kv_block=512):
    torch = torch_mod()
    pool, host, tables, lens = _setup(cfg, ctx_lens, seed, outliers)
    cu = np.zeros(len(q_lens) + 1, np.int32)
    cu[1:] = np.cumsum(q_lens)
    total = int(cu[-1])
    rng = np.random.default_rng(seed + 7)
    q = rng.standard_normal((total, cfg.n_q_heads, cfg.head_dim)).astype(np.float32)
    qt = torch.from_numpy(q).cuda()
    if q_bf16:
        qt = qt.to(torch.bfloat16)
        q = qt.float().cpu().numpy()
    out = torch.full(q.shape, float("nan"), dtype=torch.bfloat16 if out_bf16 else torch.float32,
                     device="cuda")
    pool.paged_prefill(qt, torch.from_numpy(cu).cuda(), torch.from_numpy(tables).cuda(),
                       torch.from_numpy(lens).cuda(), out, max_q_len=max_q_len)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    want = host.paged_prefill(q, cu, tables, lens, kv_block=kv_block)
    assert pool.error_count() == 0
    assert np.all(np.isfinite(got))
    return got, want


@pytest.mark.parametrize("dtype", [airkv.BF16, airkv.INT8, airkv.FP8])
@pytest.mark.parametrize("group", [1, 2, 4, 6, 8, 16])
def test_prefill_matches_oracle_small(dtype, group):
    """Chunks of 1, 31, 32, 33 and 100 rows over prefixes of 0 .. 300 tokens
    (a whole-sequence prefill, partial token blocks, a single row), for GQA
    groups of 1 .. 16 query heads per kv head (6: work items of a token
    block that do not fill whole workgroups)."""
    log(f"prefill small dtype={dtype} group={group}")
    nkv = 1 if group >= 8 else 2
    cfg = workloads.Config("small", nkv * group, nkv, 128, 16, dtype, 5)
    q_lens = [1, 31, 32, 33, 100]
    ctx = [1, 31 + 17, 32 + 300, 33, 100 + 45]
    got, want = _prefill_case(cfg, ctx, q_lens, seed=60 + group)
    err = rel_err(got, want)
    log(f"  rel err {err:.2e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype,head_dim,n_kv,group,bs", [
    (airkv.F32, 128, 2, 4, 16), (airkv.F32, 64, 2, 2, 32), (airkv.F32, 96, 1, 6, 16),
    (airkv.BF16, 64, 2, 4, 16), (airkv.BF16, 96, 2, 2, 32), (airkv.BF16, 256, 1, 8, 16),
    (airkv.INT8, 160, 2, 2, 16), (airkv.FP8, 32, 4, 1, 32), (airkv.INT8, 224, 1, 12, 16)])
def test_prefill_vector_path_vs_oracle(dtype, head_dim, n_kv, group, bs):
    """Pools the matrix-core prefill does not take -- f32 pages (the
    reference's own cache dtype) and head_dim other than 128 -- run each
    query row on the split kernel over its causal keys: the oracle's
    blockwise attention, within the same tolerance."""
    cfg = workloads.Config("vec", n_kv * group, n_kv, head_dim, bs, dtype, 4)
    got, want = _prefill_case(cfg, [1, 37, 300, 700], [1, 37, 64, 100], seed=97 + head_dim)
    err = rel_err(got, want)
    log(f"prefill vector path dtype={dtype} d={head_dim} group={group}: rel err {err:.2e}")
    assert err <= TOL.get(dtype, 1e-3)


def test_prefill_vector_path_invalid_sequences():
    """The vector prefill keeps the matrix-core prefill's error handling: a
    chunk longer than its sequence and a seq_len beyond the table are each
    counted once with their rows zero-filled, the valid sequence matches the
    oracle, and an out-of-pool table entry inside a sequence is counted once
    and read as zero keys and values."""
    torch = torch_mod()
    cfg = workloads.Config("badvec", 8, 2, 128, 16, airkv.F32, 3)
    pool, host, tables, lens = _setup(cfg, [40, 50, 60], seed=79)
    q_lens = [10, 60, 5]
    lens_bad = lens.copy()
    lens_bad[2] = tables.shape[1] * 16 + 1
    cu = np.zeros(4, np.int32)
    cu[1:] = np.cumsum(q_lens)
    q = torch.randn((int(cu[-1]), 8, 128), device="cuda")
    out = torch.full((int(cu[-1]), 8, 128), 7.0, device="cuda")
    pool.error_count(reset=True)
    pool.paged_prefill(q, torch.from_numpy(cu).cuda(), torch.from_numpy(tables).cuda(),
                       torch.from_numpy(lens_bad).cuda(), out)
    torch.cuda.synchronize()
    assert pool.error_count(reset=True) == 2
    got = out.cpu().numpy()
    assert np.all(got[10:] == 0.0)
    want = host.paged_prefill(q.cpu().numpy()[:10], cu[:2], tables[:1], lens[:1])
    assert rel_err(got[:10], want) <= 1e-3
    t2 = tables.copy()
    t2[0, 1] = 1 << 30
    cu1 = np.array([0, 10], np.int32)
    out1 = torch.zeros((10, 8, 128), device="cuda")
    pool.paged_prefill(q[:10].contiguous(), torch.from_numpy(cu1).cuda(), torch.from_numpy(t2[:1]).cuda(),
                       torch.from_numpy(lens[:1]).cuda(), out1)
    torch.cuda.synchronize()
    assert pool.error_count(reset=True) == 1
    # the entry's tokens read as zero keys and values (as the matrix-core
    # prefill reads them): the oracle over a host pool with one more block,
    # all zeros, in the entry's place
    hz = oracle.HostPool(host.num_blocks + 1, 16, 2, 128, oracle.F32)
    hz.k[:-1], hz.v[:-1] = host.k, host.v
    hz.k[-1], hz.v[-1] = 0.0, 0.0
    tz = t2[:1].copy()
    tz[0, 1] = host.num_blocks
    want1 = hz.paged_prefill(q[:10].cpu().numpy(), cu1, tz, lens[:1])
    assert rel_err(out1.cpu().numpy(), want1) <= 1e-3
    assert pool.prefill_workspace_size(8, 3, 60) == 0


@pytest.mark.parametrize("dtype", [airkv.BF16, airkv.INT8])
def test_prefill_multi_query(dtype):
    """One kv head for 32 query heads (multi-query attention; the reference
    takes any ratio, src/chunked_attn.rs:65-72)."""
    cfg = workloads.Config("mqa", 32, 1, 128, 16, dtype, 3)
    got, want = _prefill_case(cfg, [40, 200, 530], [40, 64, 130], seed=95)
    err = rel_err(got, want)
    log(f"prefill multi-query dtype={dtype}: rel err {err:.2e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("bs", [16, 32])
def test_prefill_f32_queries_bf16_out(bs):
    cfg = workloads.Config("q32", 8, 2, 128, bs, airkv.BF16, 3)
    got, want = _prefill_case(cfg, [70, 129, 250], [70, 64, 97], seed=71, q_bf16=False,
                              out_bf16=True)
    err = rel_err(got, want)
    log(f"prefill f32 q / bf16 out bs={bs}: rel err {err:.2e}")
    assert err <= 1e-2          # bf16 output rounding (2^-9) dominates
    got, want = _prefill_case(cfg, [70, 129, 250], [70, 64, 97], seed=71, q_bf16=False)
    err = rel_err(got, want)
    log(f"prefill f32 q / f32 out bs={bs}: rel err {err:.2e}")
    assert err <= 1e-3


@pytest.mark.parametrize("dtype,bs", [(airkv.INT8, 16), (airkv.FP8, 32)])
def test_prefill_f32_queries_1byte_pages(dtype, bs):
    """f32 queries over int8 / fp8 pages: the f16 pass takes the queries as
    f16 hi + lo halves against f16 keys; within 2e-2 of the oracle on the
    same dequantized cache (f32 queries)."""
    cfg = workloads.Config("q32b", 8, 2, 128, bs, dtype, 3)
    got, want = _prefill_case(cfg, [70, 129, 250], [70, 64, 97], seed=72, q_bf16=False)
    err = rel_err(got, want)
    log(f"prefill f32 q dtype={dtype} bs={bs}: rel err {err:.2e}")
    assert err <= TOL[dtype]


def test_prefill_max_q_len_below_actual_still_complete():
    cfg = workloads.Config("mq", 8, 2, 128, 16, airkv.BF16, 2)
    got, want = _prefill_case(cfg, [300, 200], [300, 150], seed=73, max_q_len=40)
    assert rel_err(got, want) <= 1e-3


def test_prefill_ranked_dispatch_mixed_batch():
    """Workgroups start in decreasing order of the keys they need, ranked
    inside the kernel: a batch of 24 sequences with empty, single-row,
    whole-sequence and prefixed chunks must still cover every row once (the
    output starts as NaN, so a row that no workgroup serves fails)."""
    rng = np.random.default_rng(81)
    q_lens = [0, 1, 33, 64, 100, 0, 7, 96] + [int(x) for x in rng.integers(0, 90, 16)]
    ctx = [q + int(p) for q, p in zip(q_lens, rng.integers(0, 400, len(q_lens)))]
    ctx = [max(c, 1) for c in ctx]
    ctx[2] = 33                          # whole-sequence prefill
    cfg = workloads.Config("rank", 8, 2, 128, 16, airkv.BF16, len(q_lens))
    got, want = _prefill_case(cfg, ctx, q_lens, seed=83)
    err = rel_err(got, want)
    log(f"prefill ranked mixed batch of {len(q_lens)}: rel err {err:.2e}")
    assert err <= 1e-3


def test_prefill_unranked_orders_large_batch_and_many_slots():
    """Past 2048 sequences, or 16384 (sequence, slot) items, workgroups keep
    slot-major order without ranking; both fallbacks cover every row."""
    rng = np.random.default_rng(85)
    n = 2100
    q_lens = [int(x) for x in rng.integers(1, 4, n)]
    ctx = [q + int(p) for q, p in zip(q_lens, rng.integers(0, 30, n))]
    cfg = workloads.Config("big", 8, 2, 128, 16, airkv.BF16, n)
    got, want = _prefill_case(cfg, ctx, q_lens, seed=87)
    err = rel_err(got, want)
    log(f"prefill batch {n} (unranked): rel err {err:.2e}")
    assert err <= 1e-3
    # 130 sequences x 128 slots (max_q_len 4096, group 4) = 16640 items
    q_lens = [int(x) for x in rng.integers(0, 40, 130)]
    ctx = [max(q + int(p), 1) for q, p in zip(q_lens, rng.integers(0, 200, 130))]
    cfg = workloads.Config("slots", 8, 2, 128, 16, airkv.BF16, 130)
    got, want = _prefill_case(cfg, ctx, q_lens, seed=89, max_q_len=4096)
    err = rel_err(got, want)
    log(f"prefill 16640 items (unranked): rel err {err:.2e}")
    assert err <= 1e-3


def test_prefill_c5_chunks_scaled():
    """configs[4] prefill geometry: 512-token chunks (bs 32, 32 q / 8 kv,
    bf16) over prefixes from the lognormal context mix; two sequences and a
    reduced head count keep the scalar oracle within seconds."""
    cfg = workloads.Config("c5p", 8, 2, 128, 32, airkv.BF16, 2)
    prefix = workloads.c5_lengths(2, seed=5)
    got, want = _prefill_case(cfg, [p + 512 for p in prefix], [512, 512], seed=75)
    err = rel_err(got, want)
    log(f"prefill c5 chunks (prefix {prefix}): rel err {err:.2e}")
    assert err <= 1e-3


def test_prefill_c3_int8_outliers():
    cfg = workloads.Config("c3p", 16, 2, 128, 16, airkv.INT8, 2)
    out_ch = workloads.outlier_channels(2, 128)
    got, want = _prefill_case(cfg, [400, 257], [128, 257], seed=77, outliers=out_ch)
    err = rel_err(got, want)
    log(f"prefill int8 outliers: rel err {err:.2e}")
    assert err <= 2e-2


def test_prefill_full_c5_shape_vs_torch_fp32():
    """The full configs[4] head geometry (32 q / 8 kv, d 128, bs 32) with
    eight 512-token chunks, against a float32 torch attention over the
    gathered cache (causal mask of src/ops.rs:762-790)."""
    torch = torch_mod()
    cfg = workloads.Config("c5full", 32, 8, 128, 32, airkv.BF16, 8)
    prefix = workloads.c5_lengths(8, seed=9)
    ctx = [p + 512 for p in prefix]
    w = workloads.build_prefill_decode(cfg, ctx, 91, decode_steps=0)
    rows = workloads.kv_rows(w.n_rows, 8, 128, seed=92, device="cuda", chunk_rows=1 << 24)
    k, v = next(rows)
    pool = device_pool_for(w)
    off = 0
    for slots in w.batches:
        n = len(slots)
        pool.append(k[off:off + n].contiguous(), v[off:off + n].contiguous(),
                    torch.from_numpy(slots).cuda())
        off += n
    tables, lens = w.tables()
    cu = np.arange(9, dtype=np.int32) * 512
    g = torch.Generator(device="cuda")
    g.manual_seed(93)
    q = torch.randn((8 * 512, 32, 128), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((8 * 512, 32, 128), device="cuda")
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
    pool.paged_prefill(q, torch.from_numpy(cu).cuda(), tt, lt, out, max_q_len=512)
    # dense K/V of every sequence, token-major [t][h][d], f32
    offs = np.zeros(9, np.int64)
    offs[1:] = np.cumsum(np.array(lens, np.int64) * 8 * 128)
    gk = torch.empty(int(offs[-1]), device="cuda")
    gv = torch.empty_like(gk)
    pool.gather(tt, lt, torch.from_numpy(offs[:-1]).cuda(), gk, gv, out_dtype=airkv.F32,
                layout=airkv.LAYOUT_TOKEN_MAJOR)
    assert pool.error_count() == 0
    worst = 0.0
    for b in range(8):
        L = int(lens[b])
        kb = gk[offs[b]:offs[b + 1]].view(L, 8, 128).permute(1, 0, 2).contiguous()   # [kv][L][d]
        vb = gv[offs[b]:offs[b + 1]].view(L, 8, 128).permute(1, 0, 2).contiguous()
        qb = q[512 * b:512 * (b + 1)].float().permute(1, 0, 2).contiguous()          # [32][512][d]
        kr = kb.repeat_interleave(4, dim=0)
        vr = vb.repeat_interleave(4, dim=0)
        s = torch.bmm(qb, kr.transpose(1, 2).contiguous()) / np.sqrt(128.0)
        qpos = torch.arange(L - 512, L, device="cuda")[:, None]
        kpos = torch.arange(L, device="cuda")[None, :]
        s = s.masked_fill(kpos > qpos, float("-inf"))
        ref = torch.bmm(torch.softmax(s, dim=-1), vr).permute(1, 0, 2)               # [512][32][d]
        got = out[512 * b:512 * (b + 1)]
        e = float((got - ref).abs().max() / ref.abs().max())
        worst = max(worst, e)
    log(f"prefill full c5 shape vs torch fp32: worst rel err {worst:.2e}")
    assert worst <= 1e-3


@pytest.mark.parametrize("dtype,bs", [(airkv.INT8, 16), (airkv.FP8, 32)])
def test_prefill_full_70b_geometry_quantized_vs_torch_fp32(dtype, bs):
    """Quantized pages at the configs[2] / configs[3] head geometry (64 q /
    8 kv, d 128) with 1% of channels x20: eight sequences of 8192 cached
    tokens whose last 512 are the chunk, against a float32 torch causal
    attention over the dequantized cache (the D3 comparison), tolerance 2e-2."""
    torch = torch_mod()
    NQ, NKV, D, L, C = 64, 8, 128, 8192, 512
    cfg = workloads.Config("p70b", NQ, NKV, D, bs, dtype, 8)
    w = workloads.build_prefill_decode(cfg, [L] * 8, 95, decode_steps=0)
    outl = workloads.outlier_channels(NKV, D, seed=3)
    gen = workloads.kv_rows(10 ** 12, NKV, D, seed=96, device="cuda", chunk_rows=1 << 16, outliers=outl)
    pool = device_pool_for(w)
    for slots in w.batches:
        st = torch.from_numpy(slots).cuda()
        done = 0
        while done < len(slots):
            k, v = next(gen)
            n = min(len(slots) - done, k.shape[0])
            pool.append(k[:n].contiguous(), v[:n].contiguous(), st[done:done + n].contiguous())
            done += n
    tables, lens = w.tables()
    cu = np.arange(9, dtype=np.int32) * C
    g = torch.Generator(device="cuda")
    g.manual_seed(97)
    q = torch.randn((8 * C, NQ, D), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((8 * C, NQ, D), device="cuda")
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
    pool.paged_prefill(q, torch.from_numpy(cu).cuda(), tt, lt, out, max_q_len=C)
    offs = np.zeros(9, np.int64)
    offs[1:] = np.cumsum(np.array(lens, np.int64) * NKV * D)
    gk = torch.empty(int(offs[-1]), device="cuda")
    gv = torch.empty_like(gk)
    pool.gather(tt, lt, torch.from_numpy(offs[:-1]).cuda(), gk, gv, out_dtype=airkv.F32,
                layout=airkv.LAYOUT_TOKEN_MAJOR)
    assert pool.error_count() == 0
    torch.backends.cuda.matmul.allow_tf32 = False
    worst = 0.0
    grp = NQ // NKV
    for b in range(8):
        kb = gk[offs[b]:offs[b + 1]].view(L, NKV, D).permute(1, 0, 2).contiguous()
        vb = gv[offs[b]:offs[b + 1]].view(L, NKV, D).permute(1, 0, 2).contiguous()
        qb = q[C * b:C * (b + 1)].float().permute(1, 0, 2).contiguous()            # [NQ][C][D]
        kr = kb.repeat_interleave(grp, dim=0)
        vr = vb.repeat_interleave(grp, dim=0)
        s = torch.bmm(qb, kr.transpose(1, 2).contiguous()) / np.sqrt(float(D))
        qpos = torch.arange(L - C, L, device="cuda")[:, None]
        kpos = torch.arange(L, device="cuda")[None, :]
        s = s.masked_fill(kpos > qpos, float("-inf"))
        ref = torch.bmm(torch.softmax(s, dim=-1), vr).permute(1, 0, 2)
        got = out[C * b:C * (b + 1)]
        worst = max(worst, float((got - ref).abs().max() / ref.abs().max()))
    log(f"prefill 70B geometry dtype={dtype} bs={bs}: worst rel err {worst:.2e}")
    assert worst <= 2e-2


def test_prefill_invalid_sequences_counted_and_zeroed():
    """A chunk longer than its sequence and an out-of-range seq_len are
    counted and their rows zero-filled; the valid sequence is unaffected; an
    out-of-pool table entry inside a sequence is counted."""
    torch = torch_mod()
    cfg = workloads.Config("bad", 8, 2, 128, 16, airkv.BF16, 3)
    pool, host, tables, lens = _setup(cfg, [40, 50, 60], seed=79)
    q_lens = [10, 60, 5]                 # sequence 1: q_len 60 > seq_len 50
    lens_bad = lens.copy()
    lens_bad[2] = tables.shape[1] * 16 + 1   # beyond the table
    cu = np.zeros(4, np.int32)
    cu[1:] = np.cumsum(q_lens)
    q = torch.randn((int(cu[-1]), 8, 128), device="cuda").to(torch.bfloat16)
    out = torch.full((int(cu[-1]), 8, 128), 7.0, device="cuda")
    pool.error_count(reset=True)
    pool.paged_prefill(q, torch.from_numpy(cu).cuda(), torch.from_numpy(tables).cuda(),
                       torch.from_numpy(lens_bad).cuda(), out)
    torch.cuda.synchronize()
    assert pool.error_count(reset=True) == 2
    got = out.cpu().numpy()
    assert np.all(got[10:] == 0.0)
    want = host.paged_prefill(q.float().cpu().numpy()[:10], cu[:2], tables[:1], lens[:1])
    assert rel_err(got[:10], want) <= 1e-3
    # an out-of-pool block id inside sequence 0's length
    t2 = tables.copy()
    t2[0, 1] = 1 << 30
    cu1 = np.array([0, 10], np.int32)
    out1 = torch.zeros((10, 8, 128), device="cuda")
    pool.paged_prefill(q[:10].contiguous(), torch.from_numpy(cu1).cuda(), torch.from_numpy(t2[:1]).cuda(),
                       torch.from_numpy(lens[:1]).cuda(), out1)
    torch.cuda.synchronize()
    assert pool.error_count(reset=True) == 1
    assert torch.isfinite(out1).all()
    # its tokens read as zero keys and values: the oracle over a host pool
    # with one more block, all zeros, in the entry's place
    hz = oracle.HostPool(host.num_blocks + 1, 16, 2, 128, oracle.BF16)
    hz.k[:-1], hz.v[:-1] = host.k, host.v
    tz = t2[:1].copy()
    tz[0, 1] = host.num_blocks
    want1 = hz.paged_prefill(q[:10].float().cpu().numpy(), cu1, tz, lens[:1])
    assert rel_err(out1.cpu().numpy(), want1) <= 1e-3


def _long_split_pool(bs=16, L=12288, seed=161):
    torch = torch_mod()
    cfg = workloads.Config("split_bad", 32, 8, 128, bs, airkv.BF16, 1)
    w = workloads.build_prefill_decode(cfg, [L], seed, decode_steps=0)
    k, v = next(workloads.kv_rows(w.n_rows, 8, 128, seed=seed + 1, device="cuda", chunk_rows=1 << 24))
    pool = device_pool_for(w)
    off = 0
    for slots in w.batches:
        n = len(slots)
        pool.append(k[off:off + n].contiguous(), v[off:off + n].contiguous(), torch.from_numpy(slots).cuda())
        off += n
    tables, lens = w.tables()
    return pool, tables, lens


def test_prefill_key_split_skips_sequence_longer_than_its_table():
    """A 512-row chunk of one 12288-token sequence is a launch the key split
    cuts (fewer work groups than resident slots), but with seq_len one past
    its table the sequence is inconsistent: it must be counted once and its
    rows zero-filled, with no piece planned for it, so a workspace full of
    NaN bytes is never folded into its rows."""
    torch = torch_mod()
    C = 512
    pool, tables, lens = _long_split_pool()
    bad = lens.copy()
    bad[0] = tables.shape[1] * 16 + 1
    cu = torch.tensor([0, C], dtype=torch.int32, device="cuda")
    q = torch.randn((C, 32, 128), device="cuda").to(torch.bfloat16)
    ws = torch.full((pool.prefill_workspace_size(32, 1, C),), 0xFF, dtype=torch.uint8, device="cuda")
    assert ws.numel() > 0
    out = torch.full((C, 32, 128), 7.0, device="cuda")
    pool.error_count(reset=True)
    pool.paged_prefill(q, cu, torch.from_numpy(tables).cuda(), torch.from_numpy(bad).cuda(), out,
                       max_q_len=C, workspace=ws)
    torch.cuda.synchronize()
    assert pool.error_count(reset=True) == 1
    assert int(ws[:4].view(torch.int32).item()) == 0       # no split slot planned
    assert bool((out == 0.0).all())
    # the same launch with the true length is split and finite
    ws2 = torch.full_like(ws, 0xFF)
    pool.paged_prefill(q, cu, torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda(), out,
                       max_q_len=C, workspace=ws2)
    torch.cuda.synchronize()
    assert pool.error_count(reset=True) == 0
    assert int(ws2[:4].view(torch.int32).item()) > 0
    assert bool(torch.isfinite(out).all())


def test_prefill_key_split_rows_past_total_q_write_nothing():
    """cu_q = [0, 512] with only 448 query rows: the rows are inconsistent, so
    the sequence is counted, nothing is split, and nothing is written -- the
    guard rows that follow `out` in the same allocation keep their bytes."""
    torch = torch_mod()
    C, T = 512, 448
    pool, tables, lens = _long_split_pool(seed=171)
    cu = torch.tensor([0, C], dtype=torch.int32, device="cuda")
    q = torch.randn((T, 32, 128), device="cuda").to(torch.bfloat16)
    big = torch.full((C, 32, 128), 7.0, device="cuda")
    out = big[:T]
    ws = torch.full((pool.prefill_workspace_size(32, 1, C),), 0xFF, dtype=torch.uint8, device="cuda")
    pool.error_count(reset=True)
    pool.paged_prefill(q, cu, torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda(), out,
                       max_q_len=C, workspace=ws)
    torch.cuda.synchronize()
    assert pool.error_count(reset=True) == 1
    assert int(ws[:4].view(torch.int32).item()) == 0
    assert bool((big == 7.0).all())                      # rows inside and past `out` untouched


def test_prefill_rejects_bad_args():
    torch = torch_mod()
    L = airkv.load()
    q = torch.zeros((4, 8, 128), device="cuda")
    cu = torch.tensor([0, 4], dtype=torch.int32, device="cuda")
    tb = torch.zeros((1, 1), dtype=torch.int32, device="cuda")
    ln = torch.tensor([4], dtype=torch.int32, device="cuda")
    pb = airkv.KvPool(8, 16, 2, 128, airkv.BF16)
    rc = L.air_paged_prefill(pb.handle, None, ctypes.c_void_p(q.data_ptr()), airkv.F32, 7,
                             ctypes.c_void_p(cu.data_ptr()), 4, 4, ctypes.c_void_p(tb.data_ptr()),
                             ctypes.c_void_p(ln.data_ptr()), 1, 1, 0.1, None, 0, ctypes.c_void_p(q.data_ptr()),
                             airkv.F32)
    assert rc == airkv.AIR_KV_E_INVALID_ARG
    # the scale must be finite and > 0
    for bad in (0.0, -0.5, float("inf")):
        with pytest.raises(airkv.AirKvError):
            pb.paged_prefill(q, cu, tb, ln, torch.empty_like(q), scale=bad)


@pytest.mark.parametrize("dtype,bs,nq,qf32", [(airkv.BF16, 32, 32, False), (airkv.INT8, 16, 64, False),
                                              (airkv.BF16, 16, 32, True)])
def test_prefill_key_split_long_sequence_vs_torch_fp32(dtype, bs, nq, qf32):
    """One sequence of 12288 cached tokens whose last 512 are the chunk: far
    fewer work groups than resident workgroups, so the launch cuts long
    groups' keys over several workgroups and merges them by log-sum-exp.  The
    workspace header must report split slots; the split and the unsplit
    launch both match a float32 torch causal attention over the gathered
    cache (1e-3 for bf16 pages, 2e-2 for int8 pages)."""
    torch = torch_mod()
    NKV, D, L, C = 8, 128, 12288, 512
    cfg = workloads.Config("split", nq, NKV, D, bs, dtype, 1)
    w = workloads.build_prefill_decode(cfg, [L], 131, decode_steps=0)
    k, v = next(workloads.kv_rows(w.n_rows, NKV, D, seed=132, device="cuda", chunk_rows=1 << 24))
    pool = device_pool_for(w)
    off = 0
    for slots in w.batches:
        n = len(slots)
        pool.append(k[off:off + n].contiguous(), v[off:off + n].contiguous(), torch.from_numpy(slots).cuda())
        off += n
    tables, lens = w.tables()
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
    cu = torch.tensor([0, C], dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(133)
    q = torch.randn((C, nq, D), generator=g, device="cuda")
    if not qf32:
        q = q.to(torch.bfloat16)
    ws_bytes = pool.prefill_workspace_size(nq, 1, C)
    assert ws_bytes > 0
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device="cuda")
    out_split = torch.empty((C, nq, D), device="cuda")
    out_plain = torch.empty_like(out_split)
    pool.paged_prefill(q, cu, tt, lt, out_split, max_q_len=C, workspace=ws)
    pool.paged_prefill(q, cu, tt, lt, out_plain, max_q_len=C, split=False)
    n_split = int(ws[:4].view(torch.int32).item())
    offs = np.array([0, L * NKV * D], np.int64)
    gk = torch.empty(int(offs[-1]), device="cuda")
    gv = torch.empty_like(gk)
    pool.gather(tt, lt, torch.from_numpy(offs[:-1]).cuda(), gk, gv, out_dtype=airkv.F32,
                layout=airkv.LAYOUT_TOKEN_MAJOR)
    assert pool.error_count() == 0
    torch.backends.cuda.matmul.allow_tf32 = False
    kb = gk.view(L, NKV, D).permute(1, 0, 2).contiguous().repeat_interleave(nq // NKV, dim=0)
    vb = gv.view(L, NKV, D).permute(1, 0, 2).contiguous().repeat_interleave(nq // NKV, dim=0)
    qb = q.float().permute(1, 0, 2).contiguous()
    s = torch.bmm(qb, kb.transpose(1, 2).contiguous()) / np.sqrt(float(D))
    qpos = torch.arange(L - C, L, device="cuda")[:, None]
    kpos = torch.arange(L, device="cuda")[None, :]
    s = s.masked_fill(kpos > qpos, float("-inf"))
    ref = torch.bmm(torch.softmax(s, dim=-1), vb).permute(1, 0, 2)
    tol = 1e-3 if dtype == airkv.BF16 else 2e-2
    es = float((out_split - ref).abs().max() / ref.abs().max())
    ep = float((out_plain - ref).abs().max() / ref.abs().max())
    log(f"key split dtype={dtype} nq={nq} qf32={qf32}: {n_split} split slots, err split {es:.2e} plain {ep:.2e}")
    assert n_split > 0
    assert es <= tol and ep <= tol


@pytest.mark.parametrize("dtype,bs", [(airkv.BF16, 32), (airkv.INT8, 16), (airkv.FP8, 32)])
@pytest.mark.parametrize("case", ["unit", "tiny", "huge", "huge_k", "spikes", "split_tiny", "mixed_channels"])
def test_prefill_value_ranges_vs_torch_fp32(dtype, bs, case):
    """Every work item first runs with f16 operands (V as f16; 1-byte pages
    also keys and queries as f16) and runs again with the exact operands
    when that result is not finite or every output of a query row is below
    2^-14.  V at unit scale (the f16 pass only), scaled by 1e-6 (f16
    subnormals: the exact pass), by 1e5 (beyond f16's 65504: the exact pass),
    K scaled by 1e5 and Q by 1e-5 (1-byte keys beyond 65504 after
    dequantization, logits unchanged), a few
    2e5 spikes in otherwise unit values (only the work items that see a
    spike run again), and tiny values under the key split (pieces run again
    on their own): all within 1e-3 (bf16 pages) or 2e-2 (int8 / fp8 pages) of
    a float32 torch causal attention over the gathered cache.  mixed_channels
    scales 16 of each head's 128 value channels by 1e-6 and leaves the rest at
    unit scale: the rows' outputs are not small, so the f16 pass stands, and
    the documented per-channel bound holds -- channels at unit scale within
    the tolerance of their own largest output, the tiny channels within f16's
    subnormal spacing (2^-24) absolute."""
    torch = torch_mod()
    NKV, NQ, D, C = 8, 32, 128, 256
    split = case == "split_tiny"
    prefix = [6000] if split else [700, 1500, 90, 2600]
    cfg = workloads.Config("vrange", NQ, NKV, D, bs, dtype, len(prefix))
    ctx = [p + C for p in prefix]
    w = workloads.build_prefill_decode(cfg, ctx, 141, decode_steps=0)
    k, v = next(workloads.kv_rows(w.n_rows, NKV, D, seed=142, device="cuda", chunk_rows=1 << 24))
    if case in ("tiny", "split_tiny"):
        v = v * 1e-6
    elif case == "mixed_channels":
        v[:, :, :16] *= 1e-6
    elif case == "huge":
        v = v * 1e5
    elif case == "huge_k":
        k = k * 1e5
    elif case == "spikes":
        g0 = torch.Generator(device="cuda")
        g0.manual_seed(143)
        idx = torch.randint(0, v.numel(), (5,), generator=g0, device="cuda")
        v.view(-1)[idx] = 2e5
    pool = device_pool_for(w)
    off = 0
    for slots in w.batches:
        n = len(slots)
        pool.append(k[off:off + n].contiguous(), v[off:off + n].contiguous(), torch.from_numpy(slots).cuda())
        off += n
    tables, lens = w.tables()
    B = len(prefix)
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
    cu = torch.from_numpy(np.arange(B + 1, dtype=np.int32) * C).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(144)
    q = torch.randn((B * C, NQ, D), generator=g, device="cuda")
    if case == "huge_k":      # logits stay O(1): keys x 1e5, queries x 1e-5
        q = q * 1e-5
    q = q.to(torch.bfloat16)
    out = torch.full((B * C, NQ, D), float("nan"), device="cuda")
    if split:
        ws = torch.zeros(pool.prefill_workspace_size(NQ, B, C), dtype=torch.uint8, device="cuda")
        assert ws.numel() > 0
        pool.paged_prefill(q, cu, tt, lt, out, max_q_len=C, workspace=ws)
        assert int(ws[:4].view(torch.int32).item()) > 0
    else:
        pool.paged_prefill(q, cu, tt, lt, out, max_q_len=C)
    offs = np.zeros(B + 1, np.int64)
    offs[1:] = np.cumsum(np.array(lens, np.int64) * NKV * D)
    gk = torch.empty(int(offs[-1]), device="cuda")
    gv = torch.empty_like(gk)
    pool.gather(tt, lt, torch.from_numpy(offs[:-1]).cuda(), gk, gv, out_dtype=airkv.F32,
                layout=airkv.LAYOUT_TOKEN_MAJOR)
    assert pool.error_count() == 0
    torch.backends.cuda.matmul.allow_tf32 = False
    worst = 0.0
    for b in range(B):
        L = int(lens[b])
        kb = gk[offs[b]:offs[b + 1]].view(L, NKV, D).permute(1, 0, 2).contiguous().repeat_interleave(NQ // NKV, dim=0)
        vb = gv[offs[b]:offs[b + 1]].view(L, NKV, D).permute(1, 0, 2).contiguous().repeat_interleave(NQ // NKV, dim=0)
        qb = q[C * b:C * (b + 1)].float().permute(1, 0, 2).contiguous()
        s_ = torch.bmm(qb, kb.transpose(1, 2).contiguous()) / np.sqrt(float(D))
        qpos = torch.arange(L - C, L, device="cuda")[:, None]
        kpos = torch.arange(L, device="cuda")[None, :]
        s_ = s_.masked_fill(kpos > qpos, float("-inf"))
        ref = torch.bmm(torch.softmax(s_, dim=-1), vb).permute(1, 0, 2)
        got = out[C * b:C * (b + 1)]
        assert bool(torch.isfinite(got).all())
        worst = max(worst, float((got - ref).abs().max() / ref.abs().max()))
        if case == "mixed_channels":
            err = (got - ref).abs()
            tiny_abs = float(err[:, :, :16].max())
            unit_rel = float((err[:, :, 16:].amax(dim=(0, 1)) / ref[:, :, 16:].abs().amax(dim=(0, 1))).max())
            log(f"  seq {b}: tiny channels abs err {tiny_abs:.2e}, unit channels rel err {unit_rel:.2e}")
            assert tiny_abs <= 2.0 ** -24
            assert unit_rel <= TOL[dtype]
    log(f"prefill value range dtype={dtype} {case}: worst rel err {worst:.2e}")
    assert worst <= TOL[dtype]


def test_prefill_key_split_eight_pieces():
    """A 128-row chunk of one 12288-token sequence: 32 work groups against
    512 resident slots, so slots are cut into the maximum of eight pieces and
    the merge folds them in two batches of four.  The workspace descriptors
    must show eight pieces; the result matches a float32 torch causal
    attention within 1e-3."""
    torch = torch_mod()
    NKV, NQ, D, L, C = 8, 32, 128, 12288, 128
    cfg = workloads.Config("split8", NQ, NKV, D, 32, airkv.BF16, 1)
    w = workloads.build_prefill_decode(cfg, [L], 151, decode_steps=0)
    k, v = next(workloads.kv_rows(w.n_rows, NKV, D, seed=152, device="cuda", chunk_rows=1 << 24))
    pool = device_pool_for(w)
    off = 0
    for slots in w.batches:
        n = len(slots)
        pool.append(k[off:off + n].contiguous(), v[off:off + n].contiguous(), torch.from_numpy(slots).cuda())
        off += n
    tables, lens = w.tables()
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
    cu = torch.tensor([0, C], dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(153)
    q = torch.randn((C, NQ, D), generator=g, device="cuda").to(torch.bfloat16)
    ws = torch.zeros(pool.prefill_workspace_size(NQ, 1, C), dtype=torch.uint8, device="cuda")
    assert ws.numel() > 0
    out = torch.empty((C, NQ, D), device="cuda")
    pool.paged_prefill(q, cu, tt, lt, out, max_q_len=C, workspace=ws)
    hdr = ws[:64 + 16 * 64].view(torch.int32).cpu().numpy()
    n_split = int(hdr[0])
    pieces = [int(hdr[16 + 4 * i + 2]) for i in range(n_split)]
    offs = np.array([0, L * NKV * D], np.int64)
    gk = torch.empty(int(offs[-1]), device="cuda")
    gv = torch.empty_like(gk)
    pool.gather(tt, lt, torch.from_numpy(offs[:-1]).cuda(), gk, gv, out_dtype=airkv.F32,
                layout=airkv.LAYOUT_TOKEN_MAJOR)
    assert pool.error_count() == 0
    torch.backends.cuda.matmul.allow_tf32 = False
    kb = gk.view(L, NKV, D).permute(1, 0, 2).contiguous().repeat_interleave(NQ // NKV, dim=0)
    vb = gv.view(L, NKV, D).permute(1, 0, 2).contiguous().repeat_interleave(NQ // NKV, dim=0)
    qb = q.float().permute(1, 0, 2).contiguous()
    s_ = torch.bmm(qb, kb.transpose(1, 2).contiguous()) / np.sqrt(float(D))
    qpos = torch.arange(L - C, L, device="cuda")[:, None]
    kpos = torch.arange(L, device="cuda")[None, :]
    s_ = s_.masked_fill(kpos > qpos, float("-inf"))
    ref = torch.bmm(torch.softmax(s_, dim=-1), vb).permute(1, 0, 2)
    err = float((out - ref).abs().max() / ref.abs().max())
    log(f"key split eight pieces: {n_split} split slots, pieces {sorted(set(pieces))}, err {err:.2e}")
    assert n_split > 0 and max(pieces) == 8
    assert err <= 1e-3
