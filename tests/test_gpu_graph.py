"""The decode step captured in a HIP graph (torch.cuda.CUDAGraph).  The
library's launches record no memset, host synchronisation or allocation, so
a captured air_paged_decode_append -- and a captured air_kv_append +
air_paged_decode pair -- replays like the eager calls.  Every replay is
checked bit for bit against the same eager calls on a twin pool (outputs,
pages and group scales), with new query / K / V values written in place
before each replay and other eager launches and synchronisations between
the replays.  bf16 pools (one matrix-core launch), int8 pools (the new rows
quantized in that launch) and f32 pools (the vector path: slots, append,
decode and merge kernels in the graph).  The paged prefill with its key
split (plan, main and merge kernels) and the gather replay the same way."""
import numpy as np
import pytest

import airkv
from airkv import workloads
from gpu_helpers import assert_bits_equal, assert_floats_bit_equal, device_pool_for, log, torch_mod

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _dev(x):
    return torch_mod().from_numpy(np.ascontiguousarray(x)).cuda()


def _pools(dtype, seed):
    cfg = workloads.Config("graph", 32, 8, 128, 16, dtype, 12)
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1, 700, cfg.batch).tolist()
    w = workloads.build_prefill_decode(cfg, ctx, seed=seed, decode_steps=1)
    k, v = next(workloads.kv_rows(w.n_rows, cfg.n_kv_heads, cfg.head_dim, seed=seed + 1, chunk_rows=1 << 24))
    pg, pe = device_pool_for(w), device_pool_for(w)
    off = 0
    for slots in w.batches[:-1]:
        n = len(slots)
        for p in (pg, pe):
            p.append(_dev(k[off:off + n]), _dev(v[off:off + n]), _dev(slots))
        off += n
    tables, lens = w.tables()
    last = lens - 1
    step_slots = (tables[np.arange(cfg.batch), last // cfg.block_size].astype(np.int64) * cfg.block_size
                  + last % cfg.block_size)
    return cfg, pg, pe, tables, lens, step_slots, rng


def _check(pg, pe, out_g, out_e, what):
    torch = torch_mod()
    torch.cuda.synchronize()
    assert_floats_bit_equal(out_g.float().cpu().numpy(), out_e.float().cpu().numpy(), f"{what} output")
    kg, vg, ksg, vsg = pg.snapshot()
    ke, ve, kse, vse = pe.snapshot()
    assert_bits_equal(kg, ke, f"{what} k pages")
    assert_bits_equal(vg, ve, f"{what} v pages")
    if ksg is not None:
        assert_bits_equal(ksg.view(np.uint32), kse.view(np.uint32), f"{what} k scales")
        assert_bits_equal(vsg.view(np.uint32), vse.view(np.uint32), f"{what} v scales")


@pytest.mark.parametrize("dtype", [airkv.BF16, airkv.INT8, airkv.F32])
@pytest.mark.parametrize("fused", [True, False])
def test_decode_step_graph_replays(dtype, fused):
    torch = torch_mod()
    cfg, pg, pe, tables, lens, step_slots, rng = _pools(dtype, 40 + 3 * dtype + int(fused))
    log(f"graph: dtype {dtype} fused {fused} lens {lens.tolist()}")
    B, nq, nkv, d = cfg.batch, cfg.n_q_heads, cfg.n_kv_heads, cfg.head_dim
    t, sl, st = _dev(tables), _dev(lens), _dev(step_slots)
    q = torch.randn(B, nq, d, device="cuda").to(torch.bfloat16)
    kn = torch.randn(B, nkv, d, device="cuda")
    vn = torch.randn(B, nkv, d, device="cuda")
    out_g = torch.full((B, nq, d), float("nan"), device="cuda")
    out_e = torch.full_like(out_g, float("nan"))
    ws_g = pg.new_workspace(nq, B, tables.shape[1], cfg.max_splits)
    ws_e = pe.new_workspace(nq, B, tables.shape[1], cfg.max_splits)

    def step(pool, out, ws):
        if fused:
            pool.paged_decode_append(q, kn, vn, t, sl, out, max_splits=cfg.max_splits, workspace=ws)
        else:
            pool.append(kn, vn, st)
            pool.paged_decode(q, t, sl, out, max_splits=cfg.max_splits, workspace=ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(pg, out_g, ws_g)                         # warm-up on the capturing stream
    torch.cuda.current_stream().wait_stream(s)
    step(pe, out_e, ws_e)
    _check(pg, pe, out_g, out_e, "warm-up")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(pg, out_g, ws_g)
    for r in range(REPLAYS):
        # new inputs in place; the graph reads them from the same buffers
        q.copy_(torch.randn(B, nq, d, device="cuda").to(torch.bfloat16))
        kn.copy_(torch.randn(B, nkv, d, device="cuda"))
        vn.copy_(torch.randn(B, nkv, d, device="cuda"))
        out_g.fill_(float("nan"))
        out_e.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        step(pe, out_e, ws_e)
        _check(pg, pe, out_g, out_e, f"replay {r}")
        # unrelated eager work between replays
        scratch = torch.empty_like(out_e)
        pe.paged_decode(q, t, sl, scratch, max_splits=cfg.max_splits, workspace=ws_e)
        torch.cuda.synchronize()
    assert pg.error_count() == 0 and pe.error_count() == 0


@pytest.mark.parametrize("dtype", [airkv.BF16, airkv.INT8])
def test_prefill_and_gather_graph_replays(dtype):
    """Paged prefill with the key split (plan, main and merge kernels: one long
    sequence and a short one) and the gather of both sequences, captured
    together; each replay, after new query values, equals the eager launches
    of the same calls bit for bit."""
    torch = torch_mod()
    bs = 32 if dtype == airkv.BF16 else 16
    cfg = workloads.Config("graph-prefill", 32, 8, 128, bs, dtype, 2)
    chunk = [256, 40]
    ctx = [3900, 300]
    w = workloads.build_prefill_decode(cfg, [c + q for c, q in zip(ctx, chunk)], seed=77, decode_steps=0)
    k, v = next(workloads.kv_rows(w.n_rows, cfg.n_kv_heads, cfg.head_dim, seed=78, chunk_rows=1 << 24))
    pool = device_pool_for(w)
    off = 0
    for slots in w.batches:
        n = len(slots)
        pool.append(_dev(k[off:off + n]), _dev(v[off:off + n]), _dev(slots))
        off += n
    tables, lens = w.tables()
    t, sl = _dev(tables), _dev(lens)
    cu = _dev(np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32))
    total = int(sum(chunk))
    q = torch.randn(total, 32, 128, device="cuda").to(torch.bfloat16)
    per = lens.astype(np.int64) * cfg.n_kv_heads * cfg.head_dim
    offs = _dev(np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64))

    def buffers():
        return (torch.full((total, 32, 128), float("nan"), dtype=torch.bfloat16, device="cuda"),
                torch.zeros(int(per.sum()), dtype=torch.bfloat16, device="cuda"),
                torch.zeros(int(per.sum()), dtype=torch.bfloat16, device="cuda"))

    out_g, gk_g, gv_g = buffers()
    out_e, gk_e, gv_e = buffers()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pre_g = pool.bind_prefill(q, cu, t, sl, out_g, max_q_len=max(chunk))
        gat_g = pool.bind_gather(t, sl, offs, gk_g, gv_g, out_dtype=airkv.BF16)
    torch.cuda.current_stream().wait_stream(s)
    assert pre_g.workspace is not None, "the long sequence should take the key split"
    pre_e = pool.bind_prefill(q, cu, t, sl, out_e, max_q_len=max(chunk))
    gat_e = pool.bind_gather(t, sl, offs, gk_e, gv_e, out_dtype=airkv.BF16)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        pre_g()
        gat_g()
    for r in range(REPLAYS):
        q.copy_(torch.randn(total, 32, 128, device="cuda").to(torch.bfloat16))
        for x in (out_g, out_e):
            x.fill_(float("nan"))
        for x in (gk_g, gv_g, gk_e, gv_e):
            x.zero_()
        torch.cuda.synchronize()
        g.replay()
        pre_e()
        gat_e()
        torch.cuda.synchronize()
        assert_floats_bit_equal(out_g.float().cpu().numpy(), out_e.float().cpu().numpy(), f"replay {r} prefill")
        for a, b, name in ((gk_g, gk_e, "k"), (gv_g, gv_e, "v")):
            assert_bits_equal(a.view(torch.int16).cpu().numpy(), b.view(torch.int16).cpu().numpy(),
                              f"replay {r} gathered {name}")
        assert np.isfinite(out_g.float().cpu().numpy()).all()
    assert pool.error_count() == 0
