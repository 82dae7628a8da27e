"""GPU parity of the KvBlock wire kernels (src/pd_disagg.rs:39-83): pack,
unpack and the int8 transfer quantization, bit-exact against the oracle.

pack: every wire element is bf16_from_f32 of the page element as f32 (bf16
pages copy their bits; int8 / fp8 pages dequantize q * scale first), laid
out [block_size][n_kv_heads][head_dim][K|V].  int8: KvBlock::int8_quantize of
that wire block (oracle.pd_int8_quantize, pinned on the CPU).  unpack: the
pages that the oracle's append writes for the wire values at the block's
slots.
"""
import numpy as np
import pytest

import airkv
import oracle
from gpu_helpers import assert_bits_equal, log, torch_mod

pytestmark = pytest.mark.gpu

BS, NKV, D = 16, 8, 128


def _filled_pool(dtype, nb=24, seed=0):
    torch = torch_mod()
    pool = airkv.KvPool(nb, BS, NKV, D, dtype)
    rng = np.random.default_rng(seed)
    k = (rng.standard_normal((nb * BS, NKV, D)) * rng.uniform(0.1, 5.0)).astype(np.float32)
    v = (rng.standard_normal((nb * BS, NKV, D)) * rng.uniform(0.1, 5.0)).astype(np.float32)
    slots = np.arange(nb * BS, dtype=np.int64)
    pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), torch.from_numpy(slots).cuda())
    return pool


def _page_values(pool, ids):
    """f32 values of the pages of `ids`, [n][NKV][BS][D] for K and V."""
    k, v, ks, vs = pool.split_blocks(pool.read_blocks(ids))
    if pool.dtype == airkv.F32:
        return k, v
    if pool.dtype == airkv.BF16:
        return (oracle.bf16_to_f32(k.reshape(-1)).reshape(k.shape),
                oracle.bf16_to_f32(v.reshape(-1)).reshape(v.shape))
    g = pool.scale_group

    def deq(c, s):
        if pool.dtype == airkv.INT8:
            x = c.astype(np.int8).astype(np.float32)
        else:
            x = oracle.fp8_to_f32(c.reshape(-1)).reshape(c.shape)
        return (x.reshape(*c.shape[:3], D // g, g) * s[..., None]).astype(np.float32).reshape(c.shape)
    return deq(k, ks), deq(v, vs)


def _expected_wire(pool, ids):
    k, v = _page_values(pool, ids)                               # [n][h][t][d]
    kv = np.stack([k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3)], axis=-1)   # [n][t][h][d][2]
    return oracle.bf16_from_f32(kv.reshape(-1)).reshape(len(ids), -1)


@pytest.mark.parametrize("dtype", [airkv.F32, airkv.BF16, airkv.INT8, airkv.FP8])
def test_pack_blocks_bitexact(dtype):
    torch = torch_mod()
    pool = _filled_pool(dtype, seed=int(dtype))
    ids = np.array([5, 0, 23, 11, 11, 7], np.int32)
    wire = pool.pack_blocks(torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    assert pool.wire_bytes == 4 * BS * NKV * D
    got = wire.cpu().numpy().view(np.uint16).reshape(len(ids), -1)
    assert_bits_equal(got, _expected_wire(pool, ids), f"pack dtype={dtype}")


@pytest.mark.parametrize("dtype", [airkv.F32, airkv.BF16, airkv.INT8, airkv.FP8])
def test_pack_blocks_int8_bitexact(dtype):
    """Fused pack + KvBlock::int8_quantize equals the oracle's int8_quantize
    of the packed wire block: codes and scale."""
    torch = torch_mod()
    pool = _filled_pool(dtype, seed=10 + int(dtype))
    ids = np.array([3, 9, 0, 22], np.int32)
    codes, scales = pool.pack_blocks_int8(torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    want_wire = _expected_wire(pool, ids)
    for i in range(len(ids)):
        want_q, want_s = oracle.pd_int8_quantize(want_wire[i])
        assert np.float32(scales[i].item()).view(np.uint32) == np.float32(want_s).view(np.uint32)
        assert np.array_equal(codes[i].cpu().numpy(), want_q)


def test_pack_blocks_int8_bf16_special_blocks():
    """The fused int8 pack of a bf16 pool on blocks with the edge cases of
    KvBlock::int8_quantize: all zeros, NaN elements, an infinity, a subnormal
    absmax, .5 ties of x * inv, signed zeros, and random blocks, taken by more
    blocks than the kernel's persistent workgroups so each one runs several
    blocks in a row.  Codes and scales equal the oracle's quantization of the
    expected wire blocks."""
    torch = torch_mod()
    nb = 600
    pool = airkv.KvPool(nb, BS, NKV, D, airkv.BF16)
    rng = np.random.default_rng(61)
    f = (rng.standard_normal((nb, 2, NKV, BS, D)) * 3).astype(np.float32)
    f[1] = 0.0
    f[2].reshape(-1)[::97] = np.nan
    f[3].reshape(-1)[1234] = np.inf
    f[4] = f[4] * np.float32(1e-39)                             # subnormal absmax
    f[5] = (np.float32(127.0) * np.linspace(-1, 1, f[5].size, dtype=np.float32)).reshape(f[5].shape)
    f[6] = -0.0
    f[7].reshape(-1)[::5] = -np.inf
    raw = oracle.bf16_from_f32(f.reshape(-1)).reshape(nb, -1)
    pool.write_blocks(np.arange(nb, dtype=np.int32), raw.view(np.uint8))
    ids = np.concatenate([np.arange(1, 8), rng.permutation(nb)]).astype(np.int32)
    codes, scales = pool.pack_blocks_int8(torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    want_wire = _expected_wire(pool, ids)
    got_c, got_s = codes.cpu().numpy(), scales.cpu().numpy()
    for i in range(len(ids)):
        want_q, want_s = oracle.pd_int8_quantize(want_wire[i])
        assert got_s[i].view(np.uint32) == np.float32(want_s).view(np.uint32), (i, ids[i])
        assert np.array_equal(got_c[i], want_q), (i, ids[i])
    assert pool.error_count() == 0


def test_wire_int8_quantize_special_blocks():
    """Whole wire buffers with the edge cases of the reference arithmetic:
    an all-zero block (scale 1.0, codes 0), NaN elements (ignored by the
    absmax, code 0), infinities (scale inf), subnormal maxima (1/scale
    overflows), values at exact .5 ties of x * inv, and random blocks."""
    torch = torch_mod()
    n, e = 7, 4096
    rng = np.random.default_rng(5)
    f = (rng.standard_normal((n, e)) * 3).astype(np.float32)
    f[0] = 0.0
    f[1, ::97] = np.nan
    f[2, 17] = np.inf
    f[3] = f[3] * np.float32(1e-40)                  # subnormal range
    f[4] = np.float32(127.0) * np.linspace(-1, 1, e, dtype=np.float32)   # ties after * inv
    bits = oracle.bf16_from_f32(f.reshape(-1)).reshape(n, e)
    wire = torch.from_numpy(bits.view(np.uint8).copy()).cuda()
    codes, scales = airkv.wire_int8_quantize(wire)
    torch.cuda.synchronize()
    for i in range(n):
        want_q, want_s = oracle.pd_int8_quantize(bits[i])
        got_s = np.float32(scales[i].item())
        assert got_s.view(np.uint32) == np.float32(want_s).view(np.uint32), i
        assert np.array_equal(codes[i].cpu().numpy(), want_q), i
    assert scales[0].item() == 1.0 and int(codes[0].abs().max()) == 0


@pytest.mark.parametrize("dtype", [airkv.F32, airkv.BF16, airkv.INT8, airkv.FP8])
def test_unpack_blocks_matches_oracle_append(dtype):
    """unpack writes the pages the oracle's append writes for the wire
    values (as f32) at the block's slots; other blocks stay untouched."""
    torch = torch_mod()
    nb = 12
    pool = airkv.KvPool(nb, BS, NKV, D, dtype)
    host = oracle.HostPool(nb, BS, NKV, D, dtype)
    ids = np.array([4, 10, 0], np.int32)
    rng = np.random.default_rng(20 + int(dtype))
    vals = (rng.standard_normal((len(ids), BS, NKV, D, 2)) * 2).astype(np.float32)
    wire_bits = oracle.bf16_from_f32(vals.reshape(-1)).reshape(len(ids), -1)
    pool.unpack_blocks(torch.from_numpy(ids).cuda(),
                       torch.from_numpy(wire_bits.view(np.uint8).reshape(len(ids), -1).copy()).cuda())
    torch.cuda.synchronize()
    wf = oracle.bf16_to_f32(wire_bits.reshape(-1)).reshape(len(ids), BS, NKV, D, 2)
    k = wf[..., 0].reshape(-1, NKV, D)
    v = wf[..., 1].reshape(-1, NKV, D)
    slots = (ids[:, None].astype(np.int64) * BS + np.arange(BS)[None, :]).reshape(-1)
    assert host.append(k, v, slots) == 0
    gk, gv, gks, gvs = pool.snapshot()
    assert_bits_equal(gk, host.k, "unpack K pages")
    assert_bits_equal(gv, host.v, "unpack V pages")
    if host.k_scales is not None:
        assert_bits_equal(gks, host.k_scales, "unpack K scales")
        assert_bits_equal(gvs, host.v_scales, "unpack V scales")


@pytest.mark.parametrize("geom", [(16, 8, 128), (32, 3, 64), (16, 5, 32), (16, 4, 96), (32, 2, 256)])
def test_bf16_special_bits_and_geometries(geom):
    """bf16 pools of several geometries (head counts that are not powers of
    two, head_dim 32..128) whose pages hold the special bit patterns:
    signalling and quiet NaNs of both signs, infinities, signed zeros,
    subnormals and the largest finite values.  pack gives bf16_from_f32 of
    each page element (a signalling NaN gains its quiet bit, everything else
    keeps its bits) in the wire layout; unpack of that wire into other blocks
    gives the same bits back in the pages."""
    torch = torch_mod()
    bs, nkv, d = geom
    nb = 12
    pool = airkv.KvPool(nb, bs, nkv, d, airkv.BF16)
    rng = np.random.default_rng(40 + nkv)
    raw = rng.integers(0, 1 << 16, size=(nb, 2, nkv, bs, d), dtype=np.uint16)
    special = np.array([0x7F81, 0xFF81, 0x7FC1, 0xFFC0, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x0001, 0x807F,
                        0x7F7F, 0xFF7F, 0x7FFF, 0xFFFF], np.uint16)
    flat = raw.reshape(-1)
    flat[rng.choice(flat.size, size=4 * special.size, replace=False)] = np.tile(special, 4)
    pool.write_blocks(np.arange(nb, dtype=np.int32), raw.reshape(nb, -1).view(np.uint8))
    src = np.array([3, 0, 7, 11], np.int32)
    wire = pool.pack_blocks(torch.from_numpy(src).cuda())
    torch.cuda.synchronize()
    k, v = raw[src, 0], raw[src, 1]                                     # [n][h][t][d]
    kv = np.stack([k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3)], axis=-1)
    want = oracle.bf16_from_f32(oracle.bf16_to_f32(kv.reshape(-1))).reshape(len(src), -1)
    assert_bits_equal(wire.cpu().numpy().view(np.uint16).reshape(len(src), -1), want, f"pack {geom}")
    dst = np.array([5, 6, 8, 9], np.int32)
    pool.unpack_blocks(torch.from_numpy(dst).cuda(), wire)
    gk, gv, _, _ = pool.snapshot()
    quiet = oracle.bf16_from_f32(oracle.bf16_to_f32(raw.reshape(-1))).reshape(raw.shape)
    assert_bits_equal(gk[dst].view(np.uint16), quiet[src, 0], f"unpack K {geom}")
    assert_bits_equal(gv[dst].view(np.uint16), quiet[src, 1], f"unpack V {geom}")
    assert_bits_equal(gk[[1, 2, 4, 10]].view(np.uint16), raw[[1, 2, 4, 10], 0], "untouched blocks")
    assert pool.error_count() == 0


def test_bf16_roundtrip_and_bad_ids():
    """bf16 pools: pack then unpack into other blocks reproduces the pages
    bit for bit; ids outside the pool are skipped and counted."""
    torch = torch_mod()
    pool = _filled_pool(airkv.BF16, nb=16, seed=3)
    src = torch.tensor([1, 2, 3], dtype=torch.int32, device="cuda")
    dst = torch.tensor([13, 14, 15], dtype=torch.int32, device="cuda")
    pool.unpack_blocks(dst, pool.pack_blocks(src))
    k, v, _, _ = pool.snapshot()
    assert np.array_equal(k[[13, 14, 15]], k[[1, 2, 3]]) and np.array_equal(v[[13, 14, 15]], v[[1, 2, 3]])
    pool.error_count(reset=True)
    out = pool.pack_blocks(torch.tensor([0, 99, -1], dtype=torch.int32, device="cuda"))
    pool.unpack_blocks(torch.tensor([77], dtype=torch.int32, device="cuda"), out[:1].contiguous())
    torch.cuda.synchronize()
    assert pool.error_count() == 3
    log("wire bad ids counted")


@pytest.mark.parametrize("dtype", [airkv.BF16, airkv.INT8])
def test_frames_of_device_pages_match_oracle(dtype):
    """Serialised KvBlocks of device-packed pages (the send side of
    src/pd_disagg.rs:534 and :267-276) equal the oracle's frames of the
    oracle's wire data, byte for byte, for both the plain and the int8
    payloads; the frames parse back to the same blocks."""
    from airkv import pd_wire
    pool = _filled_pool(dtype, seed=40 + int(dtype))
    ids = np.array([3, 17, 0, 9], np.int32)
    wire = _expected_wire(pool, ids)                       # bf16 bits [n][elems]
    got = pd_wire.frames_from_pool(pool, ids, layer_idx=5)
    want = b"".join(oracle.kvblock_serialise(int(i), 5, w.tobytes()) for i, w in zip(ids, wire))
    assert got == want
    step = 10 + wire.shape[1] * 2
    for j, i in enumerate(ids):
        blk = airkv.KvBlock.deserialise(got[j * step:(j + 1) * step])
        assert blk.block_id == i and blk.layer_idx == 5 and blk.data == wire[j].tobytes()
    got8 = pd_wire.int8_payloads_from_pool(pool, ids, layer_idx=5)
    want8 = b"".join(oracle.tcp_int8_payload(int(i), 5, w) for i, w in zip(ids, wire))
    assert got8 == want8
    log(f"frames dtype={dtype}: {len(got)} + {len(got8)} bytes byte-exact")
