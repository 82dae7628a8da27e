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


# ---- blockwise causal attention (src/chunked_attn.rs:114-213) ---------------

def _make_qkv(seq_q, seq_kv, head_dim):
    """make_qkv of src/chunked_attn.rs tests: sin / cos ramps (f64 then f32)."""
    q = np.sin(np.arange(seq_q * head_dim, dtype=np.float64) * 0.314).astype(np.float32)
    k = q.copy()
    v = (np.cos(np.arange(seq_kv * head_dim, dtype=np.float64) * 0.271).astype(np.float32)
         * np.float32(0.5))
    return q, k, v


def test_reference_blockwise_shape_finite_and_causal_ones():
    q, k, v = _make_qkv(4, 4, 4)
    out = oracle.blockwise_attention_head(q, k, v, 4, 4, 4, 0.5, 2, True, 0)
    assert out.shape == (16,) and np.all(np.isfinite(out))
    ones = np.ones(16, np.float32)
    out = oracle.blockwise_attention_head(ones, ones, ones, 4, 4, 4, 1.0, 2, True, 0)
    assert np.all(np.abs(out - 1.0) < 1e-4)


def test_reference_blockwise_matches_full_for_small_seq():
    q, k, v = _make_qkv(3, 3, 4)
    full = oracle.blockwise_attention_head(q, k, v, 3, 3, 4, 1.0, 3, True, 0)
    chunked = oracle.blockwise_attention_head(q, k, v, 3, 3, 4, 1.0, 1, True, 0)
    assert np.max(np.abs(full - chunked)) < 1e-4


@pytest.mark.parametrize("seq_q,seq_kv,block", [(1, 70, 16), (9, 70, 7), (33, 33, 512), (5, 200, 64)])
def test_blockwise_rows_are_reference_attention_over_their_prefix(seq_q, seq_kv, block):
    """Causal with q_offset = seq_kv - seq_q: query row i is the plain softmax
    attention of that query over keys 0..=q_offset + i (orc_reference_attention,
    pinned by the flash_decode tests), and a float64 masked softmax agrees."""
    rng = np.random.default_rng(seq_q * 100 + seq_kv)
    d = 64
    q = rng.standard_normal(seq_q * d).astype(np.float32)
    k = rng.standard_normal(seq_kv * d).astype(np.float32)
    v = rng.standard_normal(seq_kv * d).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    off = seq_kv - seq_q
    out = oracle.blockwise_attention_head(q, k, v, seq_q, seq_kv, d, scale, block, True, off).reshape(seq_q, d)
    Q, K, V = (x.astype(np.float64).reshape(-1, d) for x in (q, k, v))
    for i in range(seq_q):
        n = off + i + 1
        want = oracle.reference_attention(q[i * d:(i + 1) * d], k[:n * d], v[:n * d], n, d, scale)
        assert np.max(np.abs(out[i] - want)) < 2e-6
        s = K[:n] @ Q[i] * float(scale)
        p = np.exp(s - s.max())
        assert np.max(np.abs(out[i] - (p / p.sum()) @ V[:n])) < 2e-6


def test_blockwise_block_size_and_noncausal():
    rng = np.random.default_rng(9)
    d, sq, skv = 32, 6, 50
    q, k, v = (rng.standard_normal(n * d).astype(np.float32) for n in (sq, skv, skv))
    outs = [oracle.blockwise_attention_head(q, k, v, sq, skv, d, 0.2, b, True, skv - sq) for b in (1, 3, 16, 512)]
    for o in outs[1:]:
        assert np.max(np.abs(o - outs[0])) < 1e-5
    nc = oracle.blockwise_attention_head(q, k, v, sq, skv, d, 0.2, 16, False, 0).reshape(sq, d)
    for i in range(sq):
        want = oracle.reference_attention(q[i * d:(i + 1) * d], k, v, skv, d, 0.2)
        assert np.max(np.abs(nc[i] - want)) < 2e-6


def test_paged_prefill_matches_dense_blockwise():
    """The paged wrapper on a shuffled f32 pool equals the dense function on
    the gathered K/V, per query head on kv head h // group."""
    rng = np.random.default_rng(4)
    bs, nkv, d, group = 16, 2, 32, 2
    lens = np.array([40, 17, 33], np.int32)
    qlens = np.array([5, 17, 1], np.int32)
    nb = 16
    pool = oracle.HostPool(nb, bs, nkv, d, oracle.F32)
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.full((3, 3), -1, np.int32)
    used = 0
    dense_k, dense_v = [], []
    for b, L in enumerate(lens):
        nblk = -(-L // bs)
        tables[b, :nblk] = perm[used:used + nblk]
        used += nblk
        kk = rng.standard_normal((L, nkv, d)).astype(np.float32)
        vv = rng.standard_normal((L, nkv, d)).astype(np.float32)
        slots = np.array([tables[b, t // bs] * bs + t % bs for t in range(L)], np.int64)
        assert pool.append(kk, vv, slots) == 0
        dense_k.append(kk)
        dense_v.append(vv)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    q = rng.standard_normal((cu[-1], nkv * group, d)).astype(np.float32)
    got = pool.paged_prefill(q, cu, tables, lens, scale=0.25, kv_block=8)
    for b in range(3):
        for h in range(nkv * group):
            kh = h // group
            qh = q[cu[b]:cu[b + 1], h].reshape(-1)
            want = oracle.blockwise_attention_head(qh, dense_k[b][:, kh].reshape(-1), dense_v[b][:, kh].reshape(-1),
                                                   qlens[b], lens[b], d, 0.25, 8, True, lens[b] - qlens[b])
            assert np.array_equal(got[cu[b]:cu[b + 1], h].reshape(-1), want)
