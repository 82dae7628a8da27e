"""GPU tests of air_paged_decode_append, the decode step that appends each
sequence's new K/V row and attends in one launch.  Through the C ABI, its
pages and outputs equal those of air_kv_append followed by air_paged_decode
(src/model.rs:577 appends, then src/ops.rs:333-357 attends) bit for bit, and
its outputs stay within the oracle tolerance of the restated append + decode.
Covered: sequences of 1 token and with full and partial last tiles,
sequences whose last tile sits in a later slice than their first, a batch
that takes two launches, GQA groups 1, 2, 4, 8 and 16, bf16 and f32 queries, page sizes
16 and 32, a sequence of length 0, a last block outside the pool, a sequence
longer than its table, repeated calls, int8 (Q8_0) and fp8 pools (the new
rows quantized in the launch: codes and scales bit-exact with air_kv_append
and with the oracle), and pools off the matrix-core decode (f32 pages, other
head dims, small scale groups, groups above 16: append, then decode)."""
import numpy as np
import pytest

import airkv
from airkv import workloads
from gpu_helpers import (assert_bits_equal, assert_floats_bit_equal, device_pool_for, host_pool_for, log,
                         rel_err, torch_mod)

pytestmark = pytest.mark.gpu

TOL_BF16 = 1e-3


def _to_dev(x):
    torch = torch_mod()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _setup(cfg, ctx_lens, seed):
    """Two device pools and the oracle pool holding every sequence's context;
    the decode step's slots and new rows are returned unappended."""
    w = workloads.build_prefill_decode(cfg, ctx_lens, seed=seed, decode_steps=1)
    k, v = next(workloads.kv_rows(w.n_rows, cfg.n_kv_heads, cfg.head_dim, seed=seed + 1, chunk_rows=1 << 24))
    pa, pb, host = device_pool_for(w), device_pool_for(w), host_pool_for(w)
    off = 0
    for slots in w.batches[:-1]:
        n = len(slots)
        for p in (pa, pb):
            p.append(_to_dev(k[off:off + n]), _to_dev(v[off:off + n]), _to_dev(slots))
        assert host.append(k[off:off + n], v[off:off + n], slots) == 0
        off += n
    k_new, v_new = k[off:], v[off:]
    assert len(k_new) == cfg.batch
    tables, lens = w.tables()
    return w, pa, pb, host, tables, lens, k_new, v_new


def _run_pair(cfg, pa, pb, host, tables, lens, k_new, v_new, q, q_f32, out_f32=True, append_mask=None):
    """Pool a: air_kv_append + air_paged_decode; pool b: air_paged_decode_append.
    append_mask[b] False: the reference path appends nothing for sequence b
    (length 0, last block outside the pool, longer than its table)."""
    torch = torch_mod()
    bs = cfg.block_size
    batch = len(lens)
    if append_mask is None:
        append_mask = np.ones(batch, bool)
    idx = np.nonzero(append_mask)[0]
    last = lens[idx] - 1
    slots = (tables[idx, last // bs].astype(np.int64) * bs + last % bs).astype(np.int64)
    qt = _to_dev(q)
    if not q_f32:
        qt = qt.to(torch.bfloat16)
        q = qt.float().cpu().numpy()
    odt = torch.float32 if out_f32 else torch.bfloat16
    t, sl = _to_dev(tables), _to_dev(lens)
    kn, vn = _to_dev(k_new), _to_dev(v_new)
    ws = pa.new_workspace(cfg.n_q_heads, batch, tables.shape[1], cfg.max_splits)
    out_a = torch.full((batch, cfg.n_q_heads, cfg.head_dim), float("nan"), dtype=odt, device="cuda")
    out_b = torch.full_like(out_a, float("nan"))
    if len(idx):
        pa.append(_to_dev(k_new[idx]), _to_dev(v_new[idx]), _to_dev(slots))
    pa.paged_decode(qt, t, sl, out_a, max_splits=cfg.max_splits, workspace=ws)
    pb.paged_decode_append(qt, kn, vn, t, sl, out_b, max_splits=cfg.max_splits, workspace=ws)
    torch.cuda.synchronize()
    ka, va, ksa, vsa = pa.snapshot()
    kb, vb, ksb, vsb = pb.snapshot()
    assert_bits_equal(kb, ka, "k pages")
    assert_bits_equal(vb, va, "v pages")
    if ksa is not None:                               # 1-byte pools: the group scales too
        assert_bits_equal(ksb.view(np.uint32), ksa.view(np.uint32), "k scales")
        assert_bits_equal(vsb.view(np.uint32), vsa.view(np.uint32), "v scales")
    got_a, got_b = out_a.float().cpu().numpy(), out_b.float().cpu().numpy()
    assert_floats_bit_equal(got_b, got_a, "decode output")
    if len(idx):
        assert host.append(k_new[idx], v_new[idx], slots) == 0
    # the fused pool against the oracle's append of the same rows
    assert_bits_equal(kb.reshape(host.k.shape), host.k, "k pages vs oracle")
    assert_bits_equal(vb.reshape(host.v.shape), host.v, "v pages vs oracle")
    if ksa is not None:
        assert_bits_equal(ksb.reshape(host.k_scales.shape).view(np.uint32), host.k_scales.view(np.uint32),
                          "k scales vs oracle")
        assert_bits_equal(vsb.reshape(host.v_scales.shape).view(np.uint32), host.v_scales.view(np.uint32),
                          "v scales vs oracle")
    return q, got_b


@pytest.mark.parametrize("n_q,bs,q_f32", [(32, 16, False), (64, 32, True), (32, 32, True), (64, 16, False),
                                          (8, 16, False), (128, 32, True), (16, 32, False)])
def test_decode_append_matches_append_then_decode(n_q, bs, q_f32):
    log(f"decode_append n_q={n_q} bs={bs} q_f32={q_f32}")
    # context lengths before the step: 0 (a one-token sequence), tiles that
    # the new token fills, starts or lands inside, and long sequences
    ctx = [0, 15, 16, 30, 31, 32, 47, 100, 700, 1500, 2200, 40, 4095]
    cfg = workloads.Config("decode_append", n_q, 8, 128, bs, airkv.BF16, len(ctx))
    w, pa, pb, host, tables, lens, k_new, v_new = _setup(cfg, ctx, seed=71 + bs + n_q)
    q = np.random.default_rng(73).standard_normal((cfg.batch, n_q, 128)).astype(np.float32)
    q, got = _run_pair(cfg, pa, pb, host, tables, lens, k_new, v_new, q, q_f32)
    want = host.paged_decode(q, tables, lens, chunk=64)
    err = rel_err(got, want)
    log(f"  identical to append + decode; rel err vs oracle {err:.2e}")
    assert err <= TOL_BF16
    assert pa.error_count() == 0 and pb.error_count() == 0


@pytest.mark.parametrize("dtype,n_q,bs,q_f32", [(airkv.INT8, 64, 16, False), (airkv.INT8, 32, 32, True),
                                                (airkv.FP8, 64, 32, False), (airkv.FP8, 32, 16, True),
                                                (airkv.INT8, 128, 16, False), (airkv.FP8, 8, 32, False)])
def test_decode_append_quantized_pools(dtype, n_q, bs, q_f32):
    """int8 (Q8_0) and fp8 pools: the fused launch quantizes each new K / V
    row into its page -- codes and group scales bit-exact with air_kv_append
    and with the oracle's append -- and its outputs are bit-exact with
    air_kv_append + air_paged_decode and within 2e-2 of the oracle.  The new
    rows carry outliers (channels x20) and a row of zeros, so scales of
    several magnitudes and the zero-group scale rule are exercised."""
    log(f"decode_append quantized dtype={dtype} n_q={n_q} bs={bs} q_f32={q_f32}")
    ctx = [0, 15, 16, 31, 32, 100, 700, 1500, 2200, 4095]
    cfg = workloads.Config("decode_append_q", n_q, 8, 128, bs, dtype, len(ctx))
    w, pa, pb, host, tables, lens, k_new, v_new = _setup(cfg, ctx, seed=171 + bs + n_q + dtype)
    k_new, v_new = k_new.copy(), v_new.copy()
    k_new[:, :, 5] *= 20.0
    v_new[:, :, 77] *= 20.0
    k_new[3] = 0.0                                     # an all-zero row: scale 1.0, codes 0
    v_new[4, 2, :40] = -0.0
    q = np.random.default_rng(173).standard_normal((cfg.batch, n_q, 128)).astype(np.float32)
    q, got = _run_pair(cfg, pa, pb, host, tables, lens, k_new, v_new, q, q_f32)
    want = host.paged_decode(q, tables, lens, chunk=64)   # (f32 queries: the device rounds them to bf16)
    err = rel_err(got, want)
    log(f"  identical to append + decode (pages, scales, outputs); rel err vs oracle {err:.2e}")
    assert err <= 2e-2
    assert pa.error_count() == 0 and pb.error_count() == 0


@pytest.mark.parametrize("dtype,group", [(airkv.INT8, 64), (airkv.FP8, 64), (airkv.INT8, 128), (airkv.FP8, 128)])
def test_decode_append_quantized_scale_groups(dtype, group):
    """1-byte pools whose scale groups span 64 or 128 elements (8 or 16 lanes
    of the fused quantizer per group, one or two scales per row): pages,
    scales and outputs bit-exact with air_kv_append + air_paged_decode and
    the pages and scales with the oracle's append."""
    log(f"decode_append quantized dtype={dtype} scale_group={group}")
    ctx = [0, 15, 31, 200, 1500]
    cfg = workloads.Config("decode_append_sg", 32, 8, 128, 16, dtype, len(ctx), scale_group=group)
    w, pa, pb, host, tables, lens, k_new, v_new = _setup(cfg, ctx, seed=191 + group + dtype)
    k_new, v_new = k_new.copy(), v_new.copy()
    k_new[:, :, 70] *= 30.0                            # one outlier channel in the second half of the row
    q = np.random.default_rng(192).standard_normal((cfg.batch, 32, 128)).astype(np.float32)
    q, got = _run_pair(cfg, pa, pb, host, tables, lens, k_new, v_new, q, q_f32=False)
    want = host.paged_decode(q, tables, lens, chunk=64)
    err = rel_err(got, want)
    log(f"  identical to append + decode; rel err vs oracle {err:.2e}")
    assert err <= 2e-2


@pytest.mark.parametrize("dtype", [airkv.INT8, airkv.FP8])
def test_decode_append_quantized_long_sequences(dtype):
    """1-byte pools with two long sequences spread over many slices: the last
    tile of each is computed by a later slice than the first, and pieces
    merge; pages, scales and outputs identical to the two-call path."""
    log(f"decode_append quantized multi-slice dtype={dtype}")
    ctx = [20000, 9000]
    cfg = workloads.Config("decode_append_qlong", 64, 8, 128, 32, dtype, len(ctx))
    w, pa, pb, host, tables, lens, k_new, v_new = _setup(cfg, ctx, seed=181 + dtype)
    q = np.random.default_rng(182).standard_normal((cfg.batch, 64, 128)).astype(np.float32)
    q, got = _run_pair(cfg, pa, pb, host, tables, lens, k_new, v_new, q, q_f32=False, out_f32=False)
    want = host.paged_decode(q, tables, lens, chunk=256)
    err = rel_err(got, want)
    log(f"  identical; rel err vs oracle {err:.2e}")
    assert err <= 2e-2 + 2 ** -8


def test_decode_append_multi_slice_sequences():
    """Two long sequences over every slice: each sequence's last tile is
    computed by a later slice than its first, and partial outputs merge."""
    log("decode_append multi-slice")
    ctx = [20000, 9000]
    cfg = workloads.Config("decode_append_long", 32, 8, 128, 16, airkv.BF16, len(ctx))
    w, pa, pb, host, tables, lens, k_new, v_new = _setup(cfg, ctx, seed=81)
    q = np.random.default_rng(82).standard_normal((cfg.batch, 32, 128)).astype(np.float32)
    q, got = _run_pair(cfg, pa, pb, host, tables, lens, k_new, v_new, q, q_f32=False, out_f32=False)
    want = host.paged_decode(q, tables, lens, chunk=256)
    err = rel_err(got, want)
    log(f"  identical; rel err vs oracle {err:.2e}")
    assert err <= TOL_BF16 + 2 ** -8       # bf16 output rounding


def test_decode_append_batch_above_one_launch():
    """4100 sequences: the host splits the batch over two launches, and the
    second launch's new rows start at sequence 4096."""
    log("decode_append batch 4100")
    ctx = np.random.default_rng(111).integers(0, 40, 4100).tolist()
    cfg = workloads.Config("decode_append_wide", 32, 8, 128, 16, airkv.BF16, len(ctx))
    w, pa, pb, host, tables, lens, k_new, v_new = _setup(cfg, ctx, seed=112)
    q = np.random.default_rng(113).standard_normal((cfg.batch, 32, 128)).astype(np.float32)
    _run_pair(cfg, pa, pb, host, tables, lens, k_new, v_new, q, q_f32=False)
    log("  identical to append + decode")


@pytest.mark.parametrize("dtype", [airkv.BF16, airkv.F32])
def test_decode_append_skips_invalid_sequences(dtype):
    """Length 0, a last block outside the pool and a sequence longer than its
    table append nothing, as the reference path appends nothing for them (the
    matrix-core step on bf16 pages, the vector path's slots on f32 pages)."""
    log(f"decode_append invalid sequences dtype={dtype}")
    ctx = [50, 63, 200, 17, 90]
    cfg = workloads.Config("decode_append_bad", 32, 8, 128, 16, dtype, len(ctx))
    w, pa, pb, host, tables, lens, k_new, v_new = _setup(cfg, ctx, seed=91)
    lens = lens.copy()
    tables = tables.copy()
    lens[1] = 0                                        # empty sequence
    tables[2, (lens[2] - 1) // 16] = w.num_blocks + 7  # last block outside the pool
    lens[3] = tables.shape[1] * 16 + 5                 # longer than its table
    mask = np.array([True, False, False, False, True])
    q = np.random.default_rng(92).standard_normal((cfg.batch, 32, 128)).astype(np.float32)
    _run_pair(cfg, pa, pb, host, tables, lens, k_new, v_new, q, q_f32=True, append_mask=mask)
    assert pb.error_count() > 0                        # the bad entries were counted
    log("  identical to append + decode, errors counted")


def test_decode_append_repeat_is_stable():
    """A second identical call rewrites the same rows with the same values:
    pages and outputs do not change (the bench loop relies on it)."""
    torch = torch_mod()
    log("decode_append repeat")
    ctx = [33, 300, 1000]
    cfg = workloads.Config("decode_append_rep", 64, 8, 128, 16, airkv.BF16, len(ctx))
    w, pa, pb, host, tables, lens, k_new, v_new = _setup(cfg, ctx, seed=101)
    q = _to_dev(np.random.default_rng(102).standard_normal((cfg.batch, 64, 128)).astype(np.float32))
    t, sl, kn, vn = _to_dev(tables), _to_dev(lens), _to_dev(k_new), _to_dev(v_new)
    ws = pb.new_workspace(64, cfg.batch, tables.shape[1])
    out = torch.empty((cfg.batch, 64, 128), device="cuda")
    launch = pb.bind_decode_append(q, kn, vn, t, sl, out, ws)
    torch.cuda.synchronize()
    first = out.cpu().numpy().copy()
    k1, v1, _, _ = pb.snapshot()
    for _ in range(3):
        launch()
    torch.cuda.synchronize()
    assert_floats_bit_equal(out.cpu().numpy(), first, "repeated output")
    k2, v2, _, _ = pb.snapshot()
    assert_bits_equal(k2, k1, "k pages")
    assert_bits_equal(v2, v1, "v pages")


@pytest.mark.parametrize("dtype,n_q,head_dim,bs,group", [(airkv.INT8, 32, 64, 16, 32), (airkv.FP8, 32, 128, 16, 16),
                                                          (airkv.BF16, 32, 64, 16, 32), (airkv.F32, 32, 128, 16, 32),
                                                          (airkv.BF16, 192, 128, 32, 32), (airkv.F32, 16, 96, 32, 32)])
def test_decode_append_vector_path_pools(dtype, n_q, head_dim, bs, group):
    """Pools off the matrix-core decode -- f32 pages, head_dim 64 or 96, 1-byte
    pages with scale groups of 16, 24 query heads per kv head -- take the
    same entry point: each sequence's slot from its table, the rows appended
    by air_kv_append's kernel, then the split decode.  Pages, scales and
    outputs equal air_kv_append + air_paged_decode bit for bit, the pages and
    scales the oracle's append."""
    log(f"decode_append vector path dtype={dtype} n_q={n_q} d={head_dim} bs={bs} scale_group={group}")
    ctx = [0, 15, 31, 200, 1500]
    cfg = workloads.Config("decode_append_vec", n_q, 8, head_dim, bs, dtype, len(ctx), scale_group=group)
    w, pa, pb, host, tables, lens, k_new, v_new = _setup(cfg, ctx, seed=201 + dtype + head_dim)
    q = np.random.default_rng(202).standard_normal((cfg.batch, n_q, head_dim)).astype(np.float32)
    q, got = _run_pair(cfg, pa, pb, host, tables, lens, k_new, v_new, q, q_f32=True)
    want = host.paged_decode(q, tables, lens, chunk=64)
    err = rel_err(got, want)
    log(f"  identical to append + decode; rel err vs oracle {err:.2e}")
    assert err <= (1e-3 if dtype in (airkv.F32, airkv.BF16) else 2e-2)
    assert pa.error_count() == 0 and pb.error_count() == 0
