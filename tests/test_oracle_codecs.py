"""Pins the oracle's scalar codecs (CPU only).

Each codec is checked three ways where possible: the reference's own unit
tests (known-answer bounds), hand-derived known answers for its quirks, and an
independent formulation of the same rounding rule in exact float64 value
arithmetic (not the bit manipulation the oracle uses), so that a wrong shift,
a dropped carry or a wrong tie rule fails.
"""
import math
import struct

import numpy as np
import pytest

import oracle

# ---------------------------------------------------------------------------
# FP8 E4M3 (src/fp8.rs:54-112)
# ---------------------------------------------------------------------------


def _fp8_decode_closed_form(b: int) -> float:
    """Decode from the format definition (src/fp8.rs:22-27): bias 7, 3-bit
    mantissa, S.1111.111 = NaN, exponent field 0 treated as zero."""
    if b == 0x7F:
        return math.nan
    s = -1.0 if b & 0x80 else 1.0
    e, m = (b >> 3) & 0xF, b & 7
    if e == 0:
        return 0.0
    return s * (2.0 ** (e - 7)) * (1.0 + m / 8.0)


def _fp8_encode_value_domain(x: float) -> int:
    """The reference encoder restated in the value domain with exact float64
    arithmetic: nearest 3-bit mantissa within the input's binade, ties away
    from zero, no carry into the next binade, |x| >= 256 saturates, below
    2^-6 flushes."""
    if math.isnan(x):
        return 0x7F
    s = 1 if x < 0.0 else 0
    a = abs(x)
    if a == 0.0 or a < 2.0 ** -6:
        return s << 7
    if a >= 256.0:
        return (s << 7) | 0x7E
    mant, exp = math.frexp(a)          # a = mant * 2^exp, mant in [0.5, 1)
    e = exp - 1                        # a = (2*mant) * 2^e, 2*mant in [1, 2)
    frac = a / 2.0 ** e - 1.0          # exact
    m = math.floor(frac * 8.0 + 0.5)   # half-up on the magnitude
    m = min(m, 7)
    return (s << 7) | ((e + 7) << 3) | m


def test_fp8_decode_all_256_codes_match_closed_form():
    table = oracle.fp8_decode_table()
    for b in range(256):
        want = _fp8_decode_closed_form(b)
        got = float(table[b])
        if math.isnan(want):
            assert math.isnan(got), b
        else:
            assert got == want and math.copysign(1, got) == math.copysign(1, want), (b, got, want)
    # quirks listed for the format: only 0x7F is NaN, 0xFF is -480, 0x80 is +0
    assert table[0xFF] == -480.0 and not math.isnan(table[0xFF])
    assert table[0x7E] == 448.0 and table[0xFE] == -448.0
    assert table[0x80] == 0.0 and math.copysign(1, table[0x80]) == 1.0


def test_fp8_decode_fixture_is_what_its_script_writes():
    """The committed fixture is the value-domain table of
    tests/golden/make_fp8_decode.py (Python floats, not the oracle's code)."""
    import os
    import sys
    here = os.path.join(os.path.dirname(__file__), "golden")
    sys.path.insert(0, here)
    try:
        import make_fp8_decode
    finally:
        sys.path.remove(here)
    assert make_fp8_decode.table_bytes() == open(os.path.join(here, "fp8_e4m3_decode.bin"), "rb").read()


def test_fp8_decode_table_matches_committed_fixture():
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "fp8_e4m3_decode.bin")
    fixture = np.fromfile(path, dtype="<f4")
    table = oracle.fp8_decode_table()
    assert fixture.shape == (256,)
    assert np.array_equal(fixture.view(np.uint32), table.view(np.uint32))


@pytest.mark.parametrize("x,code", [
    (300.0, 0x7E),        # [256, 448) saturates: exponent field 15 is overflow
    (256.0, 0x7E),
    (255.99998, 0x77),    # [240, 256) -> 240 (mantissa capped, no carry)
    (250.0, 0x77),
    (240.0, 0x77),
    (1.96875, 0x3F),      # half-up would carry to 2.0; capped at 1.875
    (1.9375, 0x3F),       # exact tie 1.875/2.0 stays in the binade
    (1.0625, 0x39),       # tie between 1.0 and 1.125 -> up (half-up)
    (1.0624999, 0x38),
    (-1.0625, 0xB9),
    (1e-3, 0x00),         # below 2^-6 flushes
    (-1e-3, 0x80),        # flush keeps the sign bit
    (-0.0, 0x00),         # sign is `x < 0.0`, false for -0.0
    (0.0, 0x00),
    (0.015625, 0x08),     # 2^-6, smallest normal
    (448.0, 0x7E),
    (-10000.0, 0xFE),
    (float("inf"), 0x7E),
    (float("-inf"), 0xFE),
    (float("nan"), 0x7F),
    (1.0, 0x38),
    (-3.5, 0xC6),
])
def test_fp8_encode_known_answers(x, code):
    assert oracle.fp8_from_f32_scalar(x) == code


def test_fp8_encode_matches_value_domain_restatement_on_binade_edges():
    xs = []
    for e in range(-8, 10):
        for m in range(0, 8):
            base = (2.0 ** e) * (1.0 + m / 8.0)
            mid = base + (2.0 ** e) / 16.0          # exact tie
            for v in (base, mid):
                f = np.float32(v)
                for ulp in (-2, -1, 0, 1, 2):
                    bits = int(f.view(np.uint32)) + ulp
                    xs.append(struct.unpack("<f", struct.pack("<I", bits & 0xFFFFFFFF))[0])
    xs = np.array(xs + [-x for x in xs], np.float32)
    got = oracle.fp8_from_f32(xs)
    want = np.array([_fp8_encode_value_domain(float(x)) for x in xs], np.uint8)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(xs[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]


def test_fp8_encode_matches_value_domain_restatement_random_bits():
    rng = np.random.default_rng(1234)
    bits = rng.integers(0, 2 ** 32, size=200_000, dtype=np.uint64).astype(np.uint32)
    xs = bits.view(np.float32)
    got = oracle.fp8_from_f32(xs)
    want = np.array([_fp8_encode_value_domain(float(x)) for x in xs], np.uint8)
    assert np.array_equal(got, want)


# reference unit tests, src/fp8.rs:338-387
def _rt_err(x):
    rt = oracle.fp8_to_f32_scalar(oracle.fp8_from_f32_scalar(x))
    return abs(rt) if abs(x) < 1e-6 else abs(rt - x) / abs(x)


def test_reference_e4m3_tests():
    assert oracle.fp8_to_f32_scalar(oracle.fp8_from_f32_scalar(0.0)) == 0.0
    for v in (1.0, 2.0, 4.0, 16.0, 100.0, 200.0, -1.0, -3.5, -100.0):
        assert _rt_err(v) < 0.15, v
    assert oracle.fp8_to_f32_scalar(oracle.fp8_from_f32_scalar(10_000.0)) <= 448.0 + 1.0
    assert math.isnan(oracle.fp8_to_f32_scalar(oracle.fp8_from_f32_scalar(float("nan"))))
    assert oracle.fp8_to_f32_scalar(oracle.fp8_from_f32_scalar(1e-10)) == 0.0
    for i in range(32):
        assert _rt_err((i - 16.0) * 5.0) < 0.15


def test_fp8_group_scale_rule():
    # src/fp8.rs:230-237: scale = absmax/448 (or 1 below 1e-8), code = enc(x / scale)
    q, s = oracle.fp8_quantize_group(np.zeros(32, np.float32))
    assert s == 1.0 and not q.any()
    q, s = oracle.fp8_quantize_group(np.full(32, 5e-9, np.float32))
    assert s == 1.0 and not q.any()          # 5e-9 < 2^-6 flushes
    x = np.linspace(-3.0, 7.0, 32).astype(np.float32)
    q, s = oracle.fp8_quantize_group(x)
    assert s == np.float32(7.0) / np.float32(448.0)
    assert q[-1] == 0x7E                      # the absmax element saturates to 448
    deq = oracle.fp8_to_f32(q) * s
    # Reference quirk: the encoder treats exponent field 15 as overflow, so
    # every element with |x|/scale >= 256 (above 256/448 of the group absmax)
    # saturates to +-448*scale; below that the 3-bit mantissa rounding holds.
    sat = np.abs(x / s) >= 256.0
    assert sat.any() and np.all(np.abs(deq[sat]) == np.float32(448.0) * s)
    ok = ~sat
    assert np.all(np.abs(deq[ok] - x[ok]) <= np.abs(x[ok]) * 0.0625 + s * 2 ** -6)


# ---------------------------------------------------------------------------
# bf16 RNE (half 2.7.1 bf16::from_f32)
# ---------------------------------------------------------------------------


def _bf16_nearest_even(x: np.ndarray) -> np.ndarray:
    """Value-domain round-to-nearest-even: pick the nearer of the two bf16
    neighbours in exact float64; ties go to the even mantissa."""
    u = x.view(np.uint32).astype(np.uint64)
    lo = (u >> 16).astype(np.uint64)
    hi = lo + 1
    xf = x.astype(np.float64)
    vlo = ((lo << 16).astype(np.uint32)).view(np.float32).astype(np.float64)
    vhi_bits = (hi << 16)
    vhi = np.where(vhi_bits < 2 ** 32, (vhi_bits % 2 ** 32).astype(np.uint32), 0).view(np.float32).astype(np.float64)
    dlo, dhi = np.abs(xf - vlo), np.abs(vhi - xf)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (lo % 2 == 1))
    return np.where(pick_hi, hi, lo).astype(np.uint16)


def test_bf16_rne_matches_nearest_even_random():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    finite = np.isfinite(x) & (np.abs(x) < np.float32(3.38e38))
    x = x[finite]
    got = oracle.bf16_from_f32(x)
    want = _bf16_nearest_even(x)
    assert np.array_equal(got, want)


def test_bf16_rne_ties_and_specials():
    def b(u):
        return np.array([u], np.uint32).view(np.float32)

    assert oracle.bf16_from_f32(b(0x3F808000))[0] == 0x3F80   # tie, even stays
    assert oracle.bf16_from_f32(b(0x3F818000))[0] == 0x3F82   # tie, odd rounds up
    assert oracle.bf16_from_f32(b(0x3F808001))[0] == 0x3F81   # above tie
    assert oracle.bf16_from_f32(b(0x7F7FFFFF))[0] == 0x7F80   # max finite -> inf
    assert oracle.bf16_from_f32(b(0x7F800000))[0] == 0x7F80   # inf stays
    assert oracle.bf16_from_f32(b(0xFF800000))[0] == 0xFF80
    assert oracle.bf16_from_f32(b(0x7F800001))[0] == 0x7FC0   # sNaN -> quiet, high half kept
    assert oracle.bf16_from_f32(b(0xFFC12345))[0] == 0xFFC1
    assert oracle.bf16_from_f32(b(0x80000000))[0] == 0x8000   # -0 keeps its sign


# ---------------------------------------------------------------------------
# Q8_0 (src/kv_cache.rs:26-98) and KvBlock::int8_quantize (src/pd_disagg.rs:65-83)
# ---------------------------------------------------------------------------


def test_reference_q8_roundtrip():
    # src/kv_cache.rs:563-584
    data = np.array([i * 0.5 - 16.0 for i in range(64)], np.float32)
    q, s = oracle.q8_quantize(data)
    assert len(s) == 2 and len(q) == 64
    rec = oracle.q8_dequantize(q, s)
    assert np.all(np.abs(rec - data) < 0.25)


def test_reference_q8_compression_ratio():
    # src/kv_cache.rs:587-596: 1024 ones -> 32 blocks of 36 bytes
    q, s = oracle.q8_quantize(np.ones(1024, np.float32))
    assert len(s) == 32 and len(s) * 36 == 1152 and 1024 * 4 / (len(s) * 36) > 3.5
    assert np.all(q == 127) and np.all(s == np.float32(1.0) / np.float32(127.0))


def test_reference_q8_save_load_roundtrip_shape():
    # src/kv_cache.rs:599-638: [1,4,2,32] of i*0.01-1.28, error < 0.05
    data = np.array([i * 0.01 - 1.28 for i in range(256)], np.float32)
    q, s = oracle.q8_quantize(data)
    assert np.all(np.abs(oracle.q8_dequantize(q, s) - data) < 0.05)


def test_q8_closed_forms():
    q, s = oracle.q8_quantize(np.zeros(32, np.float32))
    assert s[0] == 1.0 and not q.any()              # absmax 0 -> scale 1
    # absmax 127 -> scale exactly 1, so x*inv = x and rounding is visible:
    # f32::round is half away from zero (2.5 -> 3, -2.5 -> -3, 0.5 -> 1)
    x = np.zeros(32, np.float32)
    x[:6] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.4999999]
    q, s = oracle.q8_quantize(x)
    assert s[0] == 1.0
    assert list(q[:6]) == [127, 3, -3, 1, -1, 1]
    # NaN is ignored by the absmax fold and encodes to 0
    x = np.full(32, 2.0, np.float32)
    x[3] = np.nan
    q, s = oracle.q8_quantize(x)
    assert s[0] == np.float32(2.0) / np.float32(127.0) and q[3] == 0 and q[0] == 127
    # a short last block (numel not a multiple of 32)
    q, s = oracle.q8_quantize(np.arange(40, dtype=np.float32))
    assert len(s) == 2 and s[1] == np.float32(39.0) / np.float32(127.0)


@pytest.mark.parametrize("nan_bits", [0x7F800001, 0xFFBFFFFF, 0x7FC00000, 0xFFC00001])
def test_absmax_ignores_every_nan(nan_bits):
    """Rust's f32::max returns the other operand when one is NaN, signalling
    NaNs included (std docs), so a NaN anywhere in a group leaves the scale
    to the other values.  (glibc fmaxf would return NaN for a signalling NaN
    and reset the fold, giving 2/127 here.)"""
    x = np.array([5.0, 1.0, 2.0] + [0.5] * 29, np.float32)
    for pos in (0, 1, 31):
        xb = x.view(np.uint32).copy()
        xb[pos] = nan_bits
        xs = xb.view(np.float32)
        q, s = oracle.q8_quantize(xs)
        want = max(float(v) for i, v in enumerate(x) if i != pos)
        assert s[0] == np.float32(want) / np.float32(127.0) and q[pos] == 0
        q, s = oracle.fp8_quantize_group(xs)
        assert s == np.float32(want) / np.float32(448.0) and q[pos] == 0x7F


def test_q8_matches_float64_brute_force_on_small_groups():
    """Each code is the integer nearest to x/scale (ties away), clamped; this
    is evaluated in float64 from the f32 scale, and may differ from the f32
    product x*inv only when x*inv lands within one f32 ulp of a .5 boundary."""
    rng = np.random.default_rng(3)
    mism = 0
    for _ in range(2000):
        x = (rng.standard_normal(32) * rng.choice([1e-3, 1.0, 50.0])).astype(np.float32)
        q, s = oracle.q8_quantize(x)
        t = x.astype(np.float64) / float(s[0])
        want = np.clip(np.sign(t) * np.floor(np.abs(t) + 0.5), -127, 127)
        mism += int(np.sum(q != want))
    assert mism <= 4


def test_pd_int8_quantize_whole_buffer():
    # one scale for the whole page, no clamp, saturating cast
    x = np.array([1.0, -2.0, 0.5, 127.0] * 8, np.float32)
    bits = oracle.bf16_from_f32(x)
    q, s = oracle.pd_int8_quantize(bits)
    assert s == np.float32(127.0) / np.float32(127.0)
    assert list(q[:4]) == [1, -2, 1, 127]
    q, s = oracle.pd_int8_quantize(np.zeros(8, np.uint16))
    assert s == 1.0 and not q.any()


def test_pd_int8_quantize_saturates_like_rust_cast():
    """With a subnormal block maximum, 1/scale overflows to +inf and every
    nonzero product is +-inf: Rust's saturating `as i8` gives 127 / -128 (no
    clamp to +-127 as in Q8_0), zero gives NaN and so 0."""
    x = np.array([3e-40, -3e-40, 1e-40, -2e-40, 0.0], np.float32)
    bits = oracle.bf16_from_f32(x)
    q, s = oracle.pd_int8_quantize(bits)
    assert np.isinf(np.float32(1.0) / s)
    assert q.tolist() == [127, -128, 127, -128, 0]


# ---------------------------------------------------------------------------
# generators
# ---------------------------------------------------------------------------


def test_lcg_matches_reference_definition():
    # src/flash_decode.rs:220-223 evaluated with python integers + numpy f32
    s = 1
    want = []
    for _ in range(16):
        s = (s * 6364136223846793005 + 1442695040888963407) % 2 ** 64
        num = np.float32(s >> 33)
        want.append(num / np.float32(4294967296.0) * np.float32(2.0) - np.float32(1.0))
    got = oracle.lcg_fill(1, 16)
    assert np.array_equal(got, np.array(want, np.float32))
    assert np.all(got >= -1.0) and np.all(got < 1.0)


def test_box_muller_is_standard_normal():
    x = oracle.box_muller_fill(42, 200_000)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01


def _box_muller_uniforms(seed: int, pairs: int):
    """The two uniforms of each pair of src/kv_compress.rs:1001-1005, drawn
    with Python integers: the 64-bit LCG step, the top 53 bits converted to
    f32 (exact to f64, then one rounding), divided by 2^53 (exact), u1 floored
    at 1e-10."""
    s = seed + 1
    u1s, u2s = [], []
    for _ in range(pairs):
        s = (s * 6364136223846793005 + 1442695040888963407) % 2 ** 64
        u1 = np.float32(float(s >> 11)) / np.float32(2.0 ** 53)
        s = (s * 6364136223846793005 + 1442695040888963407) % 2 ** 64
        u2 = np.float32(float(s >> 11)) / np.float32(2.0 ** 53)
        u1s.append(max(u1, np.float32(1e-10)))
        u2s.append(u2)
    return np.array(u1s, np.float64), np.array(u2s, np.float64)


@pytest.mark.parametrize("fill", ["box_muller", "qjl_orig_dim_4"])
def test_box_muller_pairs_are_radius_and_angle(fill):
    """Each output pair (x0, x1) of the Box-Muller stream is the point at
    radius sqrt(-2 ln u1) and angle 2 pi u2 (src/kv_compress.rs:1007-1015):
    x0^2 + x1^2 = -2 ln u1 and atan2(x1, x0) = 2 pi u2 (mod 2 pi), to f32
    accuracy.  Swapping cos and sin, or u1 and u2, or dropping a sign moves
    one of the two far outside the tolerance."""
    pairs = 4096
    if fill == "box_muller":
        x = oracle.box_muller_fill(11, 2 * pairs).astype(np.float64)
    else:   # qjl_projection_matrix scales every value by 1 / sqrt(orig_dim) = 1/2
        x = oracle.qjl_projection_matrix(2 * pairs // 4, 4, 11).astype(np.float64) * 2.0
    u1, u2 = _box_muller_uniforms(11, pairs)
    x0, x1 = x[0::2], x[1::2]
    r2 = -2.0 * np.log(u1)
    assert np.allclose(x0 * x0 + x1 * x1, r2, rtol=2e-6, atol=1e-12)
    ang = np.mod(np.arctan2(x1, x0), 2 * np.pi)
    want = np.mod(2 * np.pi * u2, 2 * np.pi)
    d = np.abs(ang - want)
    d = np.minimum(d, 2 * np.pi - d)             # distance on the circle
    far = r2 > 1e-4                               # angles of tiny radii carry no information
    assert far.sum() > pairs * 0.99
    assert float(d[far].max()) < 2e-5
    # the mistakes this pins: each one moves the angle or the radius by far more
    assert np.abs(np.mod(np.arctan2(x0, x1), 2 * np.pi) - want)[far].max() > 1.0     # cos <-> sin
    assert not np.allclose(x0 * x0 + x1 * x1, -2.0 * np.log(np.maximum(u2, 1e-10)), rtol=1e-2)  # u1 <-> u2
