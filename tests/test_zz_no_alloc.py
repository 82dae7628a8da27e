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
