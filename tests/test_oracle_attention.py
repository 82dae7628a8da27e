"""Pins the oracle's flash-decode restatement (src/flash_decode.rs) on CPU.

The reference's own six tests are replayed with its LCG inputs and bounds,
then the oracle is checked against a float64 naive softmax (an independent
formulation) and against special cases whose answer the mathematics fixes.
"""
import numpy as np
import pytest

import oracle

HD = 64  # src/flash_decode.rs:230


def randn(n, seed):
    return oracle.lcg_fill(seed, n)


# --- reference tests, src/flash_decode.rs:232-305 --------------------------

def test_flash_decode_matches_reference_small():
    kv_len = 128
    q, k, v = randn(HD, 1), randn(kv_len * HD, 2), randn(kv_len * HD, 3)
    err = oracle.max_abs_error(oracle.flash_decode(q, k, v, kv_len, HD, 32),
                               oracle.reference_attention(q, k, v, kv_len, HD))
    assert err < 1e-4


def test_flash_decode_matches_reference_large():
    kv_len = 4096
    q, k, v = randn(HD, 10), randn(kv_len * HD, 11), randn(kv_len * HD, 12)
    err = oracle.max_abs_error(oracle.flash_decode(q, k, v, kv_len, HD, 64),
                               oracle.reference_attention(q, k, v, kv_len, HD))
    assert err < 1e-3


def test_flash_decode_single_chunk_equals_reference():
    kv_len = 32
    q, k, v = randn(HD, 20), randn(kv_len * HD, 21), randn(kv_len * HD, 22)
    err = oracle.max_abs_error(oracle.flash_decode(q, k, v, kv_len, HD, kv_len),
                               oracle.reference_attention(q, k, v, kv_len, HD))
    assert err < 1e-5


def test_flash_decode_output_length_correct():
    kv_len = 256
    out = oracle.flash_decode(randn(HD, 5), randn(kv_len * HD, 6), randn(kv_len * HD, 7),
                              kv_len, HD, 64)
    assert out.shape == (HD,)


def test_chunk_outputs_local_sum_positive():
    kv_len = 16
    _, m, l = oracle.chunk_attention(randn(HD, 99), randn(kv_len * HD, 100),
                                     randn(kv_len * HD, 101), HD)
    assert l > 0.0


def test_reduce_single_chunk_passthrough():
    out = oracle.reduce_chunks(np.array([[1.0, 2.0, 3.0]]), [0.0], [1.0], 3)
    assert np.all(np.abs(out - np.array([1.0, 2.0, 3.0])) < 1e-6)


# --- independent checks -----------------------------------------------------

@pytest.mark.parametrize("kv_len,chunk,d", [(1, 64, 64), (63, 64, 128), (65, 64, 128),
                                            (1000, 64, 128), (333, 17, 32)])
def test_flash_decode_vs_float64_softmax(kv_len, chunk, d):
    rng = np.random.default_rng(kv_len * 7 + d)
    q = rng.standard_normal(d).astype(np.float32)
    k = rng.standard_normal(kv_len * d).astype(np.float32)
    v = rng.standard_normal(kv_len * d).astype(np.float32)
    got = oracle.flash_decode(q, k, v, kv_len, d, chunk)
    want = oracle.reference_attention_f64(q, k, v, kv_len, d)
    # an independent numpy float64 evaluation too
    s = (k.reshape(kv_len, d).astype(np.float64) @ q.astype(np.float64)) / np.sqrt(d)
    p = np.exp(s - s.max())
    np_want = (p / p.sum()) @ v.reshape(kv_len, d).astype(np.float64)
    assert np.max(np.abs(want - np_want)) < 1e-12
    assert np.max(np.abs(got - want)) < 2e-6 * max(1.0, np.max(np.abs(want)))


def test_single_token_returns_v():
    d = 128
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal(d).astype(np.float32) for _ in range(3))
    assert np.array_equal(oracle.flash_decode(q, k, v, 1, d, 64), v)


def test_identical_keys_give_mean_of_values():
    d, n = 64, 200
    rng = np.random.default_rng(1)
    q = rng.standard_normal(d).astype(np.float32)
    k = np.tile(rng.standard_normal(d).astype(np.float32), n)
    v = rng.standard_normal(n * d).astype(np.float32)
    got = oracle.flash_decode(q, k, v, n, d, 64)
    want = v.reshape(n, d).astype(np.float64).mean(0)
    assert np.max(np.abs(got - want)) < 1e-5


def test_dominant_logit_selects_row():
    d, n = 64, 300
    rng = np.random.default_rng(2)
    k = rng.standard_normal((n, d)).astype(np.float32) * 0.01
    v = rng.standard_normal((n, d)).astype(np.float32)
    q = np.zeros(d, np.float32)
    q[5] = 1000.0
    k[137, 5] = 10.0
    got = oracle.flash_decode(q, k.ravel(), v.ravel(), n, d, 64)
    assert np.max(np.abs(got - v[137])) < 1e-5


def test_chunk_normalised_partials_and_merge_weights():
    """o_p is normalised by l_p (src/flash_decode.rs:104) and the merge weight
    is exp(m_p - m*) l_p / sum (:124-136): splitting one chunk into two must
    reproduce the single-chunk answer."""
    d, n = 32, 96
    rng = np.random.default_rng(5)
    q = rng.standard_normal(d).astype(np.float32)
    k = rng.standard_normal(n * d).astype(np.float32)
    v = rng.standard_normal(n * d).astype(np.float32)
    o1, m1, l1 = oracle.chunk_attention(q, k[:40 * d], v[:40 * d], d)
    o2, m2, l2 = oracle.chunk_attention(q, k[40 * d:], v[40 * d:], d)
    merged = oracle.reduce_chunks(np.stack([o1, o2]), [m1, m2], [l1, l2], d)
    whole, _, _ = oracle.chunk_attention(q, k, v, d)
    assert np.max(np.abs(merged - whole)) < 1e-6
    # the partial output is a convex combination of V rows (normalised)
    assert np.all(np.abs(o1) <= np.abs(v[:40 * d]).reshape(40, d).max(0) + 1e-6)


def test_reduce_rejects_zero_chunks():
    with pytest.raises(ValueError):
        oracle.reduce_chunks(np.zeros((0, 4)), [], [], 4)
