"""GPU test of air_paged_decode_noalloc, the decode entry point that takes its
workspace from a library-owned device array: through the C ABI, its output
equals air_paged_decode's (same plan, same kernels: bit for bit) on two calls
in a row, the second with a smaller input, and stays within the oracle
tolerance.  A launch that needs more workspace than the array holds is
rejected before any device work."""
import ctypes

import numpy as np
import pytest

import airkv
from airkv import _lib, workloads
from gpu_helpers import device_pool_for, host_pool_for, log, rel_err, run_appends, torch_mod

pytestmark = pytest.mark.gpu

TOL = {airkv.BF16: 1e-3, airkv.INT8: 2e-2, airkv.FP8: 2e-2}
NOALLOC_SCRATCH_BYTES = 32 << 20       # AIR_KV_NOALLOC_SCRATCH_BYTES in include/air_kv.h


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _decode_both(pool, q, tables, lens, max_splits=64):
    """(workspace path, no-alloc path) outputs for the same launch."""
    torch = torch_mod()
    L = _lib.load()
    batch, n_q, d = q.shape
    max_blocks = tables.shape[1]
    qdt = airkv.F32 if q.dtype == torch.float32 else airkv.BF16
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    ws_bytes = ctypes.c_size_t()
    _lib.check(L.air_paged_decode_workspace_size(pool.handle, n_q, batch, max_blocks, max_splits,
                                                 ctypes.byref(ws_bytes)))
    assert ws_bytes.value <= NOALLOC_SCRATCH_BYTES
    ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device="cuda")
    out_ws = torch.full((batch, n_q, d), float("nan"), device="cuda")
    out_na = torch.full((batch, n_q, d), float("nan"), device="cuda")
    _lib.check(L.air_paged_decode(pool.handle, None, _p(q), qdt, n_q, _p(tables), _p(lens), batch, max_blocks,
                                  scale, max_splits, _p(ws), ws_bytes.value, _p(out_ws), airkv.F32),
               "air_paged_decode")
    _lib.check(L.air_paged_decode_noalloc(pool.handle, None, _p(q), qdt, n_q, _p(tables), _p(lens), batch,
                                          max_blocks, scale, max_splits, _p(out_na), airkv.F32),
               "air_paged_decode_noalloc")
    torch.cuda.synchronize()
    return out_ws.cpu().numpy(), out_na.cpu().numpy()


@pytest.mark.parametrize("dtype,q_f32", [(airkv.BF16, False), (airkv.INT8, True), (airkv.FP8, False)])
def test_noalloc_decode_matches_workspace_decode(dtype, q_f32):
    torch = torch_mod()
    log(f"noalloc decode dtype={dtype} q_f32={q_f32}")
    cfg = workloads.Config("noalloc", 32, 8, 128, 16, dtype, 6)
    lens = [3, 100, 700, 1500, 2200, 40]
    w = workloads.build_prefill_decode(cfg, lens, seed=61, decode_steps=1)
    k, v = next(workloads.kv_rows(w.n_rows, 8, 128, seed=62, chunk_rows=1 << 24))
    pool, host = device_pool_for(w), host_pool_for(w)
    run_appends(w, k, v, pool, host)
    tables, seq_lens = w.tables()
    rng = np.random.default_rng(63)
    q = rng.standard_normal((cfg.batch, cfg.n_q_heads, 128)).astype(np.float32)
    qt = torch.from_numpy(q).cuda()
    if not q_f32:
        qt = qt.to(torch.bfloat16)
        q = qt.float().cpu().numpy()
    # first call: the whole batch; second: a smaller batch (the first three
    # sequences, shorter table rows), on the array the first call used
    for n, mb in [(cfg.batch, tables.shape[1]), (3, 48)]:
        t = torch.from_numpy(np.ascontiguousarray(tables[:n, :mb])).cuda()
        sl = torch.from_numpy(np.ascontiguousarray(seq_lens[:n])).cuda()
        got_ws, got_na = _decode_both(pool, qt[:n].contiguous(), t, sl)
        assert np.array_equal(got_ws, got_na), "no-alloc decode differs from the workspace decode"
        want = host.paged_decode(q[:n], tables[:n, :mb], seq_lens[:n], chunk=64)
        err = rel_err(got_na, want)
        log(f"  batch {n}: identical to the workspace path, rel err vs oracle {err:.2e}")
        assert err <= TOL[dtype]
    assert pool.error_count() == 0


def test_noalloc_rejects_a_launch_above_the_array():
    """batch 4096 x 64 query heads needs ~150 MB of partials: rejected with
    AIR_KV_E_INVALID_ARG before anything is launched."""
    L = _lib.load()
    pool = airkv.KvPool(64, 16, 8, 128, airkv.BF16)
    ws_bytes = ctypes.c_size_t()
    _lib.check(L.air_paged_decode_workspace_size(pool.handle, 64, 4096, 4, 64, ctypes.byref(ws_bytes)))
    assert ws_bytes.value > NOALLOC_SCRATCH_BYTES
    rc = L.air_paged_decode_noalloc(pool.handle, None, None, airkv.BF16, 64, None, None, 4096, 4,
                                    0.088, 64, None, airkv.F32)
    assert rc == airkv.AIR_KV_E_INVALID_ARG
    assert "scratch" in airkv.last_error()


def test_noalloc_calls_on_two_streams_are_ordered():
    """Two no-alloc calls issued back to back on two streams share the GPU's
    scratch array: the second waits for the first (an event the library
    records after each call), so both outputs equal their workspace-path
    results, bit for bit, the larger call first."""
    torch = torch_mod()
    L = _lib.load()
    log("noalloc two streams")
    cfg = workloads.Config("noalloc2", 32, 8, 128, 16, airkv.BF16, 48)
    rng = np.random.default_rng(71)
    lens = rng.integers(500, 4000, size=48).tolist()
    w = workloads.build_prefill_decode(cfg, lens, seed=72, decode_steps=1)
    k, v = next(workloads.kv_rows(w.n_rows, 8, 128, seed=73, chunk_rows=1 << 24))
    pool = device_pool_for(w)
    run_appends(w, k, v, pool, None)
    tables, seq_lens = w.tables()
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(seq_lens).cuda()
    small = 8
    tt2, lt2 = tt[:small].contiguous(), lt[:small].contiguous()
    q = torch.randn(cfg.batch, 32, 128, device="cuda").to(torch.bfloat16)
    q2 = torch.randn(small, 32, 128, device="cuda").to(torch.bfloat16)
    want1, _ = _decode_both(pool, q, tt, lt)
    want2, _ = _decode_both(pool, q2, tt2, lt2)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    out1 = torch.full((cfg.batch, 32, 128), float("nan"), device="cuda")
    out2 = torch.full((small, 32, 128), float("nan"), device="cuda")
    torch.cuda.synchronize()
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    for _ in range(3):
        _lib.check(L.air_paged_decode_noalloc(pool.handle, ctypes.c_void_p(s1.cuda_stream), _p(q), airkv.BF16, 32,
                                              _p(tt), _p(lt), cfg.batch, tables.shape[1], scale, 64, _p(out1),
                                              airkv.F32), "air_paged_decode_noalloc (s1)")
        _lib.check(L.air_paged_decode_noalloc(pool.handle, ctypes.c_void_p(s2.cuda_stream), _p(q2), airkv.BF16,
                                              32, _p(tt2), _p(lt2), small, tables.shape[1], scale, 64, _p(out2),
                                              airkv.F32), "air_paged_decode_noalloc (s2)")
        torch.cuda.synchronize()
        assert np.array_equal(out1.cpu().numpy().view(np.uint32), want1.view(np.uint32))
        assert np.array_equal(out2.cpu().numpy().view(np.uint32), want2.view(np.uint32))
    assert pool.error_count() == 0



def test_noalloc_calls_allocate_no_device_memory():
    """After two warm-up calls (code objects loaded, the scratch array's
    address looked up, the ordering event created), further no-alloc calls of
    both sizes leave the device's free memory (hipMemGetInfo, which sees
    every allocation of the process, not only torch's) unchanged."""
    torch = torch_mod()
    L = _lib.load()
    log("noalloc allocates nothing")
    cfg = workloads.Config("noalloc3", 32, 8, 128, 16, airkv.BF16, 16)
    rng = np.random.default_rng(81)
    lens = rng.integers(200, 3000, size=16).tolist()
    w = workloads.build_prefill_decode(cfg, lens, seed=82, decode_steps=1)
    k, v = next(workloads.kv_rows(w.n_rows, 8, 128, seed=83, chunk_rows=1 << 24))
    pool = device_pool_for(w)
    run_appends(w, k, v, pool, None)
    tables, seq_lens = w.tables()
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(seq_lens).cuda()
    tt2, lt2 = tt[:4].contiguous(), lt[:4].contiguous()
    q = torch.randn(cfg.batch, 32, 128, device="cuda").to(torch.bfloat16)
    out = torch.empty((cfg.batch, 32, 128), device="cuda")
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))

    def call(n, t, sl):
        _lib.check(L.air_paged_decode_noalloc(pool.handle, None, _p(q), airkv.BF16, 32, _p(t), _p(sl), n,
                                              tables.shape[1], scale, 64, _p(out), airkv.F32),
                   "air_paged_decode_noalloc")

    call(cfg.batch, tt, lt)
    call(4, tt2, lt2)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        call(cfg.batch, tt, lt)
        call(4, tt2, lt2)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    log(f"  free device memory before {free0} after {free1}")
    assert free1 == free0
    assert pool.error_count() == 0
