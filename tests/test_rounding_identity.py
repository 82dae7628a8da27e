"""The rounding the warm-tier codecs use for Rust's f32::round (half away
from zero): for 0 <= q <= 256, trunc(q + (0.5 - 2^-25)) with the sum rounded
to f32 (nearest even) equals floor(q + 0.5) computed exactly.  The value
codec's codes (src/kv_compress.rs:204-209) and the fused int8 wire pack's
codes (src/pd_disagg.rs:78-80, magnitudes below 127.5) take it in place of a
compare, a floor and a select.  Checked here on every float within 2^12 ulps
of each integer and half-integer of [0, 256], on the subnormals and the
smallest normals, and on a million random floats of the range (an exhaustive
pass over all 1.13e9 floats of [0, 256] found no mismatch either); the
negative mirror follows from copysign.  A plausible slip -- adding 0.5
itself, or rounding to nearest even -- fails the half-integers or 0.5."""
import numpy as np

C = np.float32(0.49999997)


def _check(q):
    q = q[(q >= 0) & (q <= 256)]
    got = np.trunc(q + C).astype(np.float64)
    want = np.floor(q.astype(np.float64) + 0.5)
    bad = q[got != want]
    assert bad.size == 0, bad[:8]
    return q.size


def test_constant_is_half_minus_2_pow_minus_25():
    assert C == np.float32(0.5) - np.float32(2.0 ** -25)
    assert np.float32(0.5) + C == np.float32(1.0)          # the tie at 0.5 lands on 1
    assert np.trunc(np.float32(0.49999997) + C) == 0.0      # the float below 0.5 stays under 1


def test_near_integers_and_half_integers():
    centres = np.arange(0, 513, dtype=np.float64) / 2              # 0, 0.5, 1, ..., 256
    bits = centres.astype(np.float32).view(np.int32)
    offs = np.arange(-4096, 4097, dtype=np.int32)
    q = (bits[:, None] + offs[None, :]).reshape(-1)
    q = q[(q >= 0)].astype(np.int32).view(np.float32)
    assert _check(q) > 4_000_000


def test_tiny_and_random():
    tiny = np.arange(0, 1 << 24, 7, dtype=np.uint32).view(np.float32)   # subnormals, small normals
    rng = np.random.default_rng(0)
    rand = rng.uniform(0, 256, 1_000_000).astype(np.float32)
    assert _check(tiny) + _check(rand) > 3_000_000


def test_plausible_slips_fail():
    """Adding 0.5 itself rounds the float just below 0.5 up to 1; rounding
    to nearest even sends 0.5 and 2.5 down.  The check above rejects both."""
    below = np.array([np.float32(0.49999997)], np.float32)
    assert np.trunc(below + np.float32(0.5))[0] == 1.0 and np.floor(below.astype(np.float64) + 0.5)[0] == 0.0
    ties = np.array([0.5, 2.5], np.float32)
    assert not np.array_equal(np.rint(ties), np.floor(ties.astype(np.float64) + 0.5))
