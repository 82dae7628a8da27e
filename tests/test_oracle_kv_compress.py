"""The kv_compress warm-tier codecs of the oracle (src/kv_compress.rs):
CompressedKey (1-bit sign + norm + mean), CompressedValue (affine u8) and
QJL (sign of a seeded Gaussian projection).  CPU only.

Pinned by the reference's own tests (src/kv_compress.rs:547-696 and
:1148-1213, restated below with their assertions) and by what the
mathematics fixes: exact codes on integer grids, half-away ties, the
quantization error bound, NaN handling, symmetric keys, the shared
Box-Muller generator, and the SimHash angle estimate at large m.
"""
import numpy as np
import pytest

import oracle


# ---- CompressedKey ---------------------------------------------------------

def test_reference_key_compress_decompress():
    key = (np.arange(128, dtype=np.float32) - 64.0) * np.float32(0.1)
    bits, mag, mean = oracle.key_compress(key)
    size_bytes = bits.size * 8 + 4 + 4
    assert size_bytes < key.size * 4
    assert oracle.key_decompress(bits, mag, mean, 128).size == 128


def test_reference_key_compression_ratio():
    bits, _, _ = oracle.key_compress(np.ones(128, np.float32))
    assert bits.size * 8 + 4 + 4 == 24 and 128 * 2 / 24 > 10.0


def test_reference_key_sign_encoding():
    bits, _, mean = oracle.key_compress(np.array([0.0, 1.0, 0.0, 1.0], np.float32))
    assert mean == np.float32(0.5)
    assert int(bits[0]) & 0b1010 == 0b1010 and int(bits[0]) & 0b0101 == 0


def test_reference_key_empty():
    bits, mag, mean = oracle.key_compress(np.zeros(0, np.float32))
    assert bits.size == 0 and mean == 0.0
    assert oracle.key_decompress(bits, mag, mean, 0).size == 0
    # the norm of nothing is the -0.0 start of Rust's float sum
    assert np.signbit(mag) and mag == 0.0


def test_key_symmetric_closed_form():
    """A key of +-pairs has mean exactly 0, so bit i = (k_i >= 0), and the
    reconstruction is +-|k|/sqrt(d) exactly as two roundings."""
    rng = np.random.default_rng(1)
    half = rng.standard_normal(64).astype(np.float32)
    key = np.empty(128, np.float32)
    key[0::2], key[1::2] = half, -half
    bits, mag, mean = oracle.key_compress(key)
    assert mean == 0.0
    want_bits = np.packbits((key >= 0).astype(np.uint8), bitorder="little").view(np.uint64)
    assert np.array_equal(bits, want_bits)
    assert abs(float(mag) - float(np.linalg.norm(key.astype(np.float64)))) <= 1e-6 * float(mag)
    rec = oracle.key_decompress(bits, mag, mean, 128)
    s = np.float32(mag) / np.float32(np.sqrt(np.float32(128)))
    assert np.array_equal(rec, np.where(key >= 0, s, -s).astype(np.float32))


def test_key_bits_across_words_and_nan():
    key = np.full(130, -1.0, np.float32)
    key[[0, 63, 64, 127, 128]] = 5.0
    key[5] = np.nan                                   # NaN >= mean is false
    bits, _, _ = oracle.key_compress(key)
    assert bits.size == 3
    got = [i for i in range(130) if (int(bits[i // 64]) >> (i % 64)) & 1]
    # the NaN poisons the mean, so every comparison is false
    assert got == []
    key[5] = -1.0
    bits, _, _ = oracle.key_compress(key)
    got = [i for i in range(130) if (int(bits[i // 64]) >> (i % 64)) & 1]
    assert got == [0, 63, 64, 127, 128]


# ---- CompressedValue -------------------------------------------------------

def test_reference_value_compress_decompress():
    v = np.arange(128, dtype=np.float32) * np.float32(0.01)
    q, scale, mn = oracle.value_compress(v)
    rec = oracle.value_decompress(q, scale, mn)
    assert np.all(np.abs(v - rec) < 0.01)


def test_reference_value_compression_ratio():
    q, _, _ = oracle.value_compress(np.full(128, 0.5, np.float32))
    assert q.size + 4 + 4 == 136 and 256 / 136 > 1.8


def test_reference_value_range():
    v = np.array([-10.0, 10.0, 0.0, 5.0, -5.0], np.float32)
    rec = oracle.value_decompress(*oracle.value_compress(v))
    assert abs(rec[0] + 10.0) < 0.1 and abs(rec[1] - 10.0) < 0.1


def test_reference_value_empty_and_constant():
    q, scale, mn = oracle.value_compress(np.zeros(0, np.float32))
    assert q.size == 0 and scale == 0.0 and mn == 0.0
    v = np.full(64, np.float32(np.pi), np.float32)
    q, scale, mn = oracle.value_compress(v)
    assert scale == 1.0 and np.all(q == 0)                # range 0: scale 1.0, all codes 0
    assert np.all(np.abs(oracle.value_decompress(q, scale, mn) - np.float32(np.pi)) < 0.01)


def test_value_integer_grid_and_half_away_ties():
    """With min 0 and max 255 the scale is exactly 1, so codes are the values
    rounded half away from zero: 0.5 -> 1, 2.5 -> 3, 254.5 -> 255 (ties to
    even would give 0, 2, 254)."""
    v = np.array([0.0, 255.0, 0.5, 2.5, 254.5, 17.0, 17.49, 17.51], np.float32)
    q, scale, mn = oracle.value_compress(v)
    assert scale == 1.0 and mn == 0.0
    assert q.tolist() == [0, 255, 1, 3, 255, 17, 17, 18]


def test_value_error_bound_and_endpoints():
    """Every reconstruction is within half a step (plus rounding of the
    step arithmetic) of its input; min maps to code 0 and back exactly, max
    maps to code 255."""
    rng = np.random.default_rng(3)
    for _ in range(50):
        v = (rng.standard_normal(128) * rng.uniform(0.01, 100)).astype(np.float32)
        q, scale, mn = oracle.value_compress(v)
        rec = oracle.value_decompress(q, scale, mn)
        assert mn == v.min()
        assert q[np.argmin(v)] == 0 and q[np.argmax(v)] == 255
        assert rec[np.argmin(v)] == v.min()
        tol = 0.5 * float(scale) * (1 + 1e-5) + 4 * np.finfo(np.float32).eps * float(np.abs(v).max())
        assert np.max(np.abs(rec.astype(np.float64) - v)) <= tol
        assert np.all(np.diff(q[np.argsort(v, kind="stable")].astype(int)) >= 0)   # monotone


def test_value_nan_elements():
    """min / max ignore NaN (Rust f32::min / max); a NaN element's code is 0
    (NaN survives round and clamp, and `as u8` maps it to 0)."""
    v = np.array([1.0, np.nan, 3.0, 2.0], np.float32)
    q, scale, mn = oracle.value_compress(v)
    assert mn == 1.0 and scale == np.float32(2.0) / np.float32(255.0)
    assert q[1] == 0 and q[0] == 0 and q[2] == 255


# ---- QJL -------------------------------------------------------------------

def test_reference_qjl_matrix_length_and_mean():
    assert oracle.qjl_projection_matrix(64, 128, 42).size == 64 * 128
    m = oracle.qjl_projection_matrix(64, 128, 7)
    assert abs(float(m.sum(dtype=np.float32)) / m.size) < 0.1


def test_qjl_matrix_is_the_box_muller_stream_scaled():
    """orig_dim = 1 makes the scale exactly 1: the matrix is the oracle's
    Box-Muller stream bit for bit; for orig_dim = 128 every value is that
    stream times 1/sqrt(128) (one rounding), and the values are N(0, 1/d)."""
    raw = oracle.box_muller_fill(9, 4096)
    assert np.array_equal(oracle.qjl_projection_matrix(4096, 1, 9).view(np.uint32), raw.view(np.uint32))
    m = oracle.qjl_projection_matrix(32, 128, 9)
    s = np.float32(1.0) / np.sqrt(np.float32(128))
    assert np.array_equal(m.view(np.uint32), (raw * s).astype(np.float32).view(np.uint32))
    big = oracle.qjl_projection_matrix(256, 128, 5).astype(np.float64) * np.sqrt(128)
    assert abs(big.mean()) < 0.02 and abs(big.std() - 1.0) < 0.02


def test_reference_qjl_compress_size_same_opposite_dot_magnitude():
    proj = oracle.qjl_projection_matrix(64, 128, 0)
    bits, _ = oracle.qjl_compress(np.ones(128, np.float32), proj, 64)
    assert bits.size == 1 and bits.size * 8 + 4 < 256 // 8
    proj = oracle.qjl_projection_matrix(64, 128, 1)
    a, _ = oracle.qjl_compress(np.full(128, 0.5, np.float32), proj, 64)
    b, _ = oracle.qjl_compress(np.full(128, 0.5, np.float32), proj, 64)
    assert abs(oracle.qjl_cos_sim(a, b, 64) - 1.0) < 1e-6
    proj = oracle.qjl_projection_matrix(64, 128, 2)
    p, _ = oracle.qjl_compress(np.ones(128, np.float32), proj, 64)
    n, _ = oracle.qjl_compress(-np.ones(128, np.float32), proj, 64)
    assert oracle.qjl_cos_sim(p, n, 64) < -0.5
    proj = oracle.qjl_projection_matrix(64, 128, 3)
    k1, m1 = oracle.qjl_compress(np.ones(128, np.float32), proj, 64)
    k2, m2 = oracle.qjl_compress(np.full(128, 2.0, np.float32), proj, 64)
    assert oracle.qjl_cos_sim(k1, k2, 64) * m1 * m2 > 0.0
    key = np.arange(128, dtype=np.float32) * np.float32(0.01)
    proj = oracle.qjl_projection_matrix(64, 128, 5)
    _, mag = oracle.qjl_compress(key, proj, 64)
    assert abs(float(mag) - float(np.sqrt(np.sum(key.astype(np.float64) ** 2)))) < 1e-4


def test_qjl_estimates_the_angle():
    """SimHash: each sign bit differs with probability angle/pi, so with many
    projections cos(pi * hamming / m) approaches the true cosine."""
    rng = np.random.default_rng(11)
    m = 8192
    proj = oracle.qjl_projection_matrix(m, 64, 4)
    for target in [0.9, 0.5, 0.0, -0.7]:
        x = rng.standard_normal(64)
        y = rng.standard_normal(64)
        y -= (y @ x) / (x @ x) * x
        x, y = x / np.linalg.norm(x), y / np.linalg.norm(y)
        k2 = target * x + np.sqrt(1 - target ** 2) * y
        a, _ = oracle.qjl_compress(x.astype(np.float32), proj, m)
        b, _ = oracle.qjl_compress(k2.astype(np.float32), proj, m)
        assert abs(float(oracle.qjl_cos_sim(a, b, m)) - target) < 0.05
