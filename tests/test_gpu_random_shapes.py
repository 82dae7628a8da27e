"""GPU parity over seeded random shapes: page dtype, head_dim (32 .. 256),
block size, kv heads, GQA group (non-powers of two and groups above 16
included), scale group, batch, context lengths (one-token sequences
included), query and output dtypes.  Each case checks, through the C ABI:

  * the appended pages and scales, bit-exact with the oracle's append;
  * the decode step as one call (air_paged_decode_append) against the
    append + decode calls on a second pool: pages, scales and outputs bit
    for bit, and the outputs within tolerance of the oracle's decode;
  * the gather of every sequence (a random layout; f32, and bf16 for
    non-f32 pools), bit-exact with the oracle's;
  * the paged prefill of the newest rows of a few sequences (chunks of 0 ..
    32 rows) within tolerance of the oracle's blockwise attention.

Whichever kernels a shape selects (matrix-core or vector decode and
prefill, fused or appended step) must agree with the oracle."""
import numpy as np
import pytest

import airkv
from airkv import workloads
from gpu_helpers import (assert_bits_equal, assert_floats_bit_equal, device_pool_for, host_pool_for, log,
                         rel_err, torch_mod)

pytestmark = pytest.mark.gpu

TOL = {airkv.F32: 1e-3, airkv.BF16: 1e-3, airkv.INT8: 2e-2, airkv.FP8: 2e-2}
N_CASES = 64


def _shape(seed):
    rng = np.random.default_rng(5000 + seed)
    dtype = int(rng.choice([airkv.F32, airkv.BF16, airkv.INT8, airkv.FP8]))
    head_dim = int(rng.choice([32, 64, 96, 128, 128, 128, 160, 256]))
    bs = int(rng.choice([16, 32]))
    n_kv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 12, 16, 20, 32]))
    while n_kv * group > 64:                        # keeps the oracle's work small
        n_kv //= 2
        if n_kv == 0:
            n_kv, group = 1, 32
    sg = 32
    if dtype in (airkv.INT8, airkv.FP8):
        sg = int(rng.choice([g for g in (8, 16, 32, 64, 128) if head_dim % g == 0]))
    batch = int(rng.integers(1, 13))
    ctx = rng.integers(0, 1000, batch)
    ctx[rng.random(batch) < 0.2] = 0                # one-token sequences after the step
    return dict(dtype=dtype, head_dim=head_dim, bs=bs, n_kv=n_kv, group=group, sg=sg, ctx=ctx.tolist(),
                q_f32=bool(rng.random() < 0.5), out_bf16=bool(rng.random() < 0.3), rng=rng)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_shape(seed):
    torch = torch_mod()
    s = _shape(seed)
    dtype, d, bs, n_kv, group = s["dtype"], s["head_dim"], s["bs"], s["n_kv"], s["group"]
    n_q = n_kv * group
    rng = s["rng"]
    log(f"random shape {seed}: dtype={dtype} d={d} bs={bs} n_kv={n_kv} group={group} "
        f"scale_group={s['sg']} ctx={s['ctx']} q_f32={s['q_f32']} out_bf16={s['out_bf16']}")
    cfg = workloads.Config("rand", n_q, n_kv, d, bs, dtype, len(s["ctx"]), scale_group=s["sg"])
    w = workloads.build_prefill_decode(cfg, s["ctx"], seed=600 + seed, decode_steps=1)
    k, v = next(workloads.kv_rows(w.n_rows, n_kv, d, seed=700 + seed, chunk_rows=1 << 24))
    pa, pb, host = device_pool_for(w), device_pool_for(w), host_pool_for(w)

    def dev(x):
        return torch.from_numpy(np.ascontiguousarray(x)).cuda()

    # the context: every batch but the decode step's
    off = 0
    for slots in w.batches[:-1]:
        n = len(slots)
        for p in (pa, pb):
            p.append(dev(k[off:off + n]), dev(v[off:off + n]), dev(slots))
        assert host.append(k[off:off + n], v[off:off + n], slots) == 0
        off += n
    pk, pv, pks, pvs = pa.snapshot()
    assert_bits_equal(pk, host.k, "k pages")
    assert_bits_equal(pv, host.v, "v pages")
    if pks is not None:
        assert_bits_equal(pks, host.k_scales, "k scales")
        assert_bits_equal(pvs, host.v_scales, "v scales")

    # the decode step: append + decode on pool a, one call on pool b
    k_new, v_new, slots = k[off:], v[off:], w.batches[-1]
    tables, lens = w.tables()
    q = rng.standard_normal((len(lens), n_q, d)).astype(np.float32)
    qt = dev(q)
    if not s["q_f32"]:
        qt = qt.to(torch.bfloat16)
        q = qt.float().cpu().numpy()
    odt = torch.bfloat16 if s["out_bf16"] else torch.float32
    out_a = torch.full((len(lens), n_q, d), float("nan"), dtype=odt, device="cuda")
    out_b = torch.full_like(out_a, float("nan"))
    tt, lt = dev(tables), dev(lens)
    ws = pa.new_workspace(n_q, len(lens), tables.shape[1])
    pa.append(dev(k_new), dev(v_new), dev(slots))
    pa.paged_decode(qt, tt, lt, out_a, workspace=ws)
    pb.paged_decode_append(qt, dev(k_new), dev(v_new), tt, lt, out_b, workspace=ws)
    torch.cuda.synchronize()
    ka, va, ksa, vsa = pa.snapshot()
    kb, vb, ksb, vsb = pb.snapshot()
    assert_bits_equal(kb, ka, "fused step k pages")
    assert_bits_equal(vb, va, "fused step v pages")
    if ksa is not None:
        assert_bits_equal(ksb, ksa, "fused step k scales")
        assert_bits_equal(vsb, vsa, "fused step v scales")
    got_a, got_b = out_a.float().cpu().numpy(), out_b.float().cpu().numpy()
    assert_floats_bit_equal(got_b, got_a, "fused step output")
    assert host.append(k_new, v_new, slots) == 0
    tol = TOL[dtype] + (2 ** -8 if s["out_bf16"] else 0.0)
    want = host.paged_decode(q, tables, lens, chunk=64)
    err = rel_err(got_a, want)
    log(f"  decode rel err {err:.2e}")
    assert err <= tol

    # gather: both layouts, f32 views (quantized pages dequantized) and the
    # cache dtype's bf16 views, bit-exact with the oracle's
    per = lens.astype(np.int64) * n_kv * d
    offs = np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)
    for out_dtype in ([airkv.F32] if dtype == airkv.F32 else [airkv.F32, airkv.BF16]):
        layout = int(rng.choice([airkv.LAYOUT_HEAD_MAJOR, airkv.LAYOUT_TOKEN_MAJOR]))
        gdt = torch.float32 if out_dtype == airkv.F32 else torch.bfloat16
        gk = torch.zeros(int(per.sum()), dtype=gdt, device="cuda")
        gv = torch.zeros_like(gk)
        pa.gather(tt, lt, dev(offs), gk, gv, out_dtype, layout)
        torch.cuda.synchronize()
        hk, hv, hoffs, bad = host.gather(tables, lens, out_dtype, layout)
        assert bad == 0 and np.array_equal(offs, hoffs)
        view = np.uint32 if out_dtype == airkv.F32 else np.uint16
        assert_bits_equal(gk.cpu().view(torch.int32 if out_dtype == airkv.F32 else torch.int16).numpy().view(view),
                          hk.view(view), f"gathered k out={out_dtype} layout={layout}")
        assert_bits_equal(gv.cpu().view(torch.int32 if out_dtype == airkv.F32 else torch.int16).numpy().view(view),
                          hv.view(view), f"gathered v out={out_dtype} layout={layout}")

    # prefill: the newest rows of up to four sequences
    sel = rng.choice(len(lens), size=min(4, len(lens)), replace=False)
    q_lens = np.array([int(rng.integers(0, min(32, lens[b]) + 1)) for b in sel], np.int32)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    total = int(cu[-1])
    if total:
        qp = rng.standard_normal((total, n_q, d)).astype(np.float32)
        qpt = dev(qp)
        if not s["q_f32"]:
            qpt = qpt.to(torch.bfloat16)
            qp = qpt.float().cpu().numpy()
        op = torch.full((total, n_q, d), float("nan"), dtype=odt, device="cuda")
        ts, ls = np.ascontiguousarray(tables[sel]), np.ascontiguousarray(lens[sel])
        pa.paged_prefill(qpt, dev(cu), dev(ts), dev(ls), op, max_q_len=32)
        torch.cuda.synchronize()
        wantp = host.paged_prefill(qp, cu, ts, ls)
        errp = rel_err(op.float().cpu().numpy(), wantp)
        log(f"  prefill rows {q_lens.tolist()}: rel err {errp:.2e}")
        assert errp <= tol
    assert pa.error_count() == 0 and pb.error_count() == 0
