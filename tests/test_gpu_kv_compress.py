"""GPU parity: the warm-tier codecs of src/kv_compress.rs (1-bit sign keys,
affine u8 values, QJL sign projections and their scores) against the oracle's
scalar restatement, bit for bit, through the C ABI."""
import ctypes

import numpy as np
import pytest

import airkv
import oracle
from airkv import kv_compress as kc
from airkv import workloads
from gpu_helpers import (assert_bits_equal, assert_floats_bit_equal, device_pool_for, host_pool_for, log,
                         run_appends, torch_mod)

pytestmark = pytest.mark.gpu


def _edge_rows(d):
    """Rows that exercise the codecs' special cases."""
    rows = []
    rows.append(np.zeros(d, np.float32))
    rows.append(np.full(d, -0.0, np.float32))
    rows.append(np.full(d, 3.25, np.float32))                        # constant: range 0 -> scale 1
    r = np.arange(d, dtype=np.float32) * np.float32(0.5) - np.float32(d / 4)
    rows.append(r)                                                    # exact grid, many ties at the mean
    r = np.ones(d, np.float32); r[3] = np.nan
    rows.append(r)                                                    # NaN ignored by min / max
    r = np.linspace(-1, 1, d).astype(np.float32); r[0] = np.inf
    rows.append(r)
    r = np.linspace(-1, 1, d).astype(np.float32); r[1] = -np.inf
    rows.append(r)
    r = np.full(d, 3e38, np.float32); r[::2] = -3e38
    rows.append(r)                                                    # sums overflow to inf
    rows.append((np.arange(d, dtype=np.float32) + 1) * np.float32(1e-42))   # denormals
    r = np.zeros(d, np.float32); r[5] = np.nan; r[6] = -0.0
    rows.append(r)
    r = np.full(d, np.nan, np.float32)
    rows.append(r)                                                    # all NaN
    r = np.zeros(d, np.float32); r[::3] = 1.0; r[1::3] = -0.0
    rows.append(r)                                                    # +0 / -0 tie order in min / max
    r = np.zeros(d, np.float32); r[::3] = -1.0; r[1::3] = -0.0
    rows.append(r)                                                    # the same for max
    r = np.linspace(-2, 3, d).astype(np.float32)
    r.view(np.uint32)[2::7] = np.uint32(0x7F800001)                   # signalling NaNs are ignored too
    r.view(np.uint32)[4] = np.uint32(0xFFA00000)
    rows.append(r)
    r = np.full(d, -0.0, np.float32); r[d // 2:] = 0.0
    rows.append(r)                                                    # -0 then +0: the last zero wins
    r = np.zeros(d, np.float32); r[1] = 255.0                         # scale 1: codes round x itself
    r[2:6] = [np.nextafter(np.float32(0.5), np.float32(0)), 0.5, np.nextafter(np.float32(1.5), np.float32(0)), 1.5]
    rows.append(r)                                                    # just below / at the .5 ties
    return np.stack(rows)


def _rows(n, d, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, d)).astype(np.float32)
    x[: n // 4] *= np.float32(37.0)
    # magnitudes from 1e-38 to 1e36 (subnormal and huge scales), offsets far
    # larger than the spread (tiny ranges), and exact integer grids whose
    # quotients land on .5 ties
    mags = (10.0 ** rng.uniform(-38, 36, size=n // 4)).astype(np.float32)
    x[n // 4: n // 2] *= mags[:, None]
    x[n // 2: n // 2 + n // 8] += np.float32(1000.0)
    a, b = n // 2 + n // 8, n // 2 + n // 4
    x[a:b] = rng.integers(-300, 300, size=(b - a, d)).astype(np.float32) * np.float32(0.5)
    return np.concatenate([_edge_rows(d), x])


def _oracle_keys(x):
    w = (x.shape[1] + 63) // 64
    bits = np.zeros((len(x), w), np.uint64)
    mag = np.zeros(len(x), np.float32)
    mean = np.zeros(len(x), np.float32)
    for i, r in enumerate(x):
        bits[i], mag[i], mean[i] = oracle.key_compress(r)
    return bits, mag, mean


def _oracle_values(x):
    codes = np.zeros(x.shape, np.uint8)
    scale = np.zeros(len(x), np.float32)
    mn = np.zeros(len(x), np.float32)
    for i, r in enumerate(x):
        codes[i], scale[i], mn[i] = oracle.value_compress(r)
    return codes, scale, mn


@pytest.mark.parametrize("d", [32, 64, 128])
def test_key_and_value_compress_bit_exact(d):
    torch = torch_mod()
    x = _rows(3000, d, seed=d)
    xt = torch.from_numpy(x).cuda()
    bits, mag, mean = kc.key_compress(xt)
    codes, scale, mn = kc.value_compress(xt)
    torch.cuda.synchronize()
    ob, om, omean = _oracle_keys(x)
    assert_bits_equal(kc.as_u64(bits), ob, "key bits")
    assert_bits_equal(mag.cpu().numpy(), om, "key magnitude")
    assert_bits_equal(mean.cpu().numpy(), omean, "key mean")
    oc, osc, omn = _oracle_values(x)
    assert_bits_equal(codes.cpu().numpy(), oc, "value codes")
    assert_bits_equal(scale.cpu().numpy(), osc, "value scale")
    assert_bits_equal(mn.cpu().numpy(), omn, "value min")
    log(f"key/value compress d={d}: {len(x)} rows bit-exact")


def test_bf16_rows_compress_as_their_f32_values():
    torch = torch_mod()
    x = _rows(1000, 128, seed=5)
    xb = torch.from_numpy(x).cuda().to(torch.bfloat16)
    xf = xb.float().cpu().numpy()
    bits, mag, mean = kc.key_compress(xb)
    codes, scale, mn = kc.value_compress(xb)
    ob, om, omean = _oracle_keys(xf)
    oc, osc, omn = _oracle_values(xf)
    assert_bits_equal(kc.as_u64(bits), ob, "bf16 key bits")
    assert_bits_equal(mag.cpu().numpy(), om, "bf16 magnitude")
    assert_bits_equal(mean.cpu().numpy(), omean, "bf16 mean")
    assert_bits_equal(codes.cpu().numpy(), oc, "bf16 codes")
    assert_bits_equal(scale.cpu().numpy(), osc, "bf16 scale")
    assert_bits_equal(mn.cpu().numpy(), omn, "bf16 min")


@pytest.mark.parametrize("d", [64, 128])
def test_decompress_bit_exact(d):
    torch = torch_mod()
    x = _rows(800, d, seed=9)
    xt = torch.from_numpy(x).cuda()
    bits, mag, mean = kc.key_compress(xt)
    codes, scale, mn = kc.value_compress(xt)
    kd = kc.key_decompress(bits, mag, mean, d).cpu().numpy()
    vd = kc.value_decompress(codes, scale, mn).cpu().numpy()
    hb, hm, hmean = kc.as_u64(bits), mag.cpu().numpy(), mean.cpu().numpy()
    hc, hs, hmn = codes.cpu().numpy(), scale.cpu().numpy(), mn.cpu().numpy()
    for i in range(len(x)):
        assert_floats_bit_equal(kd[i], oracle.key_decompress(hb[i], hm[i], hmean[i], d), f"key row {i}")
        assert_floats_bit_equal(vd[i], oracle.value_decompress(hc[i], hs[i], hmn[i]), f"value row {i}")


@pytest.mark.parametrize("proj_dim", [64, 100, 256])
def test_qjl_compress_and_scores_bit_exact(proj_dim):
    torch = torch_mod()
    d = 128
    proj = oracle.qjl_projection_matrix(proj_dim, d, seed=42)
    x = _rows(1500, d, seed=proj_dim)
    xt = torch.from_numpy(x).cuda()
    pt = torch.from_numpy(proj).cuda()
    bits, mag = kc.qjl_compress(xt, pt, proj_dim)
    hb, hm = kc.as_u64(bits), mag.cpu().numpy()
    for i in range(len(x)):
        ob, om = oracle.qjl_compress(x[i], proj, proj_dim)
        assert_bits_equal(hb[i], ob, f"qjl bits row {i}")
        assert_bits_equal(hm[i:i + 1], np.array([om], np.float32), f"qjl magnitude row {i}")
    # one query against every key
    q = np.random.default_rng(1).standard_normal(d).astype(np.float32)
    qb, qm = oracle.qjl_compress(q, proj, proj_dim)
    cos, dot = kc.qjl_scores(bits, mag, torch.from_numpy(qb.view(np.int64)).cuda(), qm, proj_dim)
    cos, dot = cos.cpu().numpy(), dot.cpu().numpy()
    for i in range(len(x)):
        c = oracle.qjl_cos_sim(hb[i], qb, proj_dim)
        assert_bits_equal(cos[i:i + 1], np.array([c], np.float32), f"cos row {i}")
        want = np.float32(np.float32(c) * hm[i]) * np.float32(qm)
        assert_floats_bit_equal(dot[i:i + 1], np.array([want], np.float32), f"dot row {i}")
    log(f"qjl m={proj_dim}: {len(x)} keys bit-exact, scores bit-exact")


def _pool_rows_f32(host, dtype, which):
    pages = host.k if which == "k" else host.v
    if dtype == airkv.F32:
        return pages.reshape(-1, host.head_dim).copy()
    if dtype == airkv.BF16:
        return oracle.bf16_to_f32(pages).reshape(-1, host.head_dim)
    sc = host.k_scales if which == "k" else host.v_scales
    vals = pages.astype(np.float32) if dtype == airkv.INT8 else oracle.fp8_to_f32(pages)
    vals = vals.reshape(sc.shape[:3] + (-1, host.group))
    return (vals * sc[..., None]).reshape(-1, host.head_dim)


@pytest.mark.parametrize("dtype,d,sg", [(airkv.F32, 128, 32), (airkv.BF16, 128, 32), (airkv.INT8, 128, 32),
                                        (airkv.FP8, 128, 32), (airkv.INT8, 64, 8), (airkv.FP8, 64, 16),
                                        (airkv.INT8, 32, 16), (airkv.FP8, 32, 32), (airkv.BF16, 32, 32),
                                        (airkv.F32, 64, 32)])
def test_compress_blocks_matches_oracle(dtype, d, sg):
    """Codecs straight from pool blocks of every page dtype, head_dim 32 .. 128
    and scale groups of 8 .. 32 elements (1-byte rows of 32 take the per-row
    loader, the others the staged loads)."""
    torch = torch_mod()
    cfg = workloads.Config("cb", 8, 4, d, 16, dtype, 3, scale_group=sg)
    w = workloads.build_prefill_decode(cfg, [40, 70, 33], seed=13, decode_steps=0)
    k, v = next(workloads.kv_rows(w.n_rows, 4, d, seed=14, chunk_rows=1 << 20))
    pool, host = device_pool_for(w), host_pool_for(w)
    run_appends(w, k, v, pool, host)
    ids = np.array([3, 0, w.num_blocks - 1, 7], np.int32)
    out = kc.compress_blocks(pool, torch.from_numpy(ids).cuda())
    proj = oracle.qjl_projection_matrix(64, d, seed=3)
    qbits, qmag = kc.qjl_compress_blocks(pool, torch.from_numpy(ids).cuda(), torch.from_numpy(proj).cuda(), 64)
    kr = _pool_rows_f32(host, dtype, "k").reshape(w.num_blocks, -1, d)[ids].reshape(-1, d)
    vr = _pool_rows_f32(host, dtype, "v").reshape(w.num_blocks, -1, d)[ids].reshape(-1, d)
    ob, om, omean = _oracle_keys(kr)
    oc, osc, omn = _oracle_values(vr)
    assert_bits_equal(kc.as_u64(out["key_bits"]), ob, "block key bits")
    assert_bits_equal(out["key_magnitude"].cpu().numpy(), om, "block key magnitude")
    assert_bits_equal(out["key_mean"].cpu().numpy(), omean, "block key mean")
    assert_bits_equal(out["value_codes"].cpu().numpy(), oc, "block value codes")
    assert_bits_equal(out["value_scale"].cpu().numpy(), osc, "block value scale")
    assert_bits_equal(out["value_min"].cpu().numpy(), omn, "block value min")
    hq = kc.as_u64(qbits)
    for i in range(0, len(kr), 7):
        b, m = oracle.qjl_compress(kr[i], proj, 64)
        assert_bits_equal(hq[i], b, f"block qjl row {i}")
    assert pool.error_count() == 0


@pytest.mark.parametrize("n_kv", [2, 4])
def test_compress_blocks_out_of_pool_ids_counted_and_zeroed(n_kv):
    """32-row blocks take the row-by-row key codec, 64-row blocks the staged
    one; out-of-pool ids are counted once and their rows come out zero."""
    torch = torch_mod()
    pool = airkv.KvPool(8, 16, n_kv, 64, airkv.BF16)
    pool.append(torch.randn(8 * 16, n_kv, 64, device="cuda"), torch.randn(8 * 16, n_kv, 64, device="cuda"),
                torch.arange(8 * 16, dtype=torch.int64, device="cuda"))
    ids = torch.tensor([1, 99, -1], dtype=torch.int32, device="cuda")
    out = kc.compress_blocks(pool, ids)
    assert pool.error_count(reset=True) == 2
    rows = n_kv * 16
    assert torch.all(out["key_magnitude"][rows:] == 0) and torch.all(out["value_codes"][rows:] == 0)
    assert torch.all(out["value_scale"][rows:] == 0) and torch.all(out["key_mean"][rows:] == 0)
    assert torch.all(out["value_min"][rows:] == 0)
    assert torch.all(out["key_magnitude"][:rows] > 0)


def test_codec_argument_errors():
    torch = torch_mod()
    L = airkv.load()
    x = torch.zeros((4, 96), device="cuda")
    with pytest.raises(airkv.AirKvError):
        kc.key_compress(x)
    x = torch.zeros((4, 64), device="cuda")
    with pytest.raises(airkv.AirKvError):
        kc.qjl_compress(x, torch.zeros(513 * 64, device="cuda"), 513)
    assert L.air_kv_qjl_compress(None, ctypes.c_void_p(x.data_ptr()), airkv.F32, 4, 64, None, 64, None,
                                 None) == airkv.AIR_KV_E_INVALID_ARG
