"""KvBlock framing on the host (src/pd_disagg.rs:39-104, :267-276): the
product's C ABI against the oracle's
restatement, byte for byte, and the reference's own wire tests restated.
CPU only (the GPU side -- frames of device-packed pages -- is in
test_gpu_wire.py)."""
import struct

import numpy as np
import pytest

import airkv
import oracle
from airkv import pd_wire


# --- the reference's tests (src/pd_disagg.rs:799-821), product and oracle ---

def make_block(block_id, layer, size):
    return airkv.KvBlock(block_id, layer, b"\xab" * size)


def test_kv_block_serialise_roundtrip():
    block = make_block(42, 7, 64)
    raw = block.serialise()
    decoded = airkv.KvBlock.deserialise(raw)
    assert decoded is not None
    assert decoded.block_id == 42 and decoded.layer_idx == 7 and decoded.data == block.data
    assert oracle.kvblock_deserialise(raw) == (42, 7, block.data)


def test_kv_block_deserialise_too_short():
    assert airkv.KvBlock.deserialise(bytes(5)) is None
    assert oracle.kvblock_deserialise(bytes(5)) is None


def test_kv_block_deserialise_truncated_data():
    raw = make_block(1, 0, 32).serialise()[:-10]
    assert airkv.KvBlock.deserialise(raw) is None
    assert oracle.kvblock_deserialise(raw) is None


# --- byte layout -------------------------------------------------------------

def test_frame_layout_is_little_endian_fields_then_data():
    """A hand-built frame: id 0x01020304, layer 0x0506, 3 data bytes."""
    raw = airkv.KvBlock(0x01020304, 0x0506, b"xyz").serialise()
    assert raw == bytes([4, 3, 2, 1, 6, 5, 3, 0, 0, 0]) + b"xyz"
    assert raw == struct.pack("<IHI", 0x01020304, 0x0506, 3) + b"xyz"


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_frames_match_oracle_random(seed):
    rng = np.random.default_rng(seed)
    for _ in range(50):
        n = int(rng.integers(0, 4096))
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        bid, layer = int(rng.integers(0, 1 << 32)), int(rng.integers(0, 1 << 16))
        raw = airkv.KvBlock(bid, layer, data).serialise()
        assert raw == oracle.kvblock_serialise(bid, layer, data)
        # any prefix shorter than the frame is rejected by both, the frame itself accepted
        cut = int(rng.integers(0, len(raw) + 1))
        p, o = airkv.KvBlock.deserialise(raw[:cut]), oracle.kvblock_deserialise(raw[:cut])
        assert (p is None) == (o is None) == (cut < len(raw))
        if p is not None:
            assert (p.block_id, p.layer_idx, p.data) == o


def test_serialise_n_equals_single_frames():
    rng = np.random.default_rng(5)
    ids = rng.integers(0, 1 << 20, 7).astype(np.uint32)
    bb = 96
    data = rng.integers(0, 256, (7, bb), dtype=np.uint8)
    out = np.empty(7 * (10 + bb), np.uint8)
    airkv.load().air_kv_block_serialise_n(ids.ctypes.data, 3, data.ctypes.data, bb, 7, out.ctypes.data)
    want = b"".join(oracle.kvblock_serialise(int(i), 3, d.tobytes()) for i, d in zip(ids, data))
    assert out.tobytes() == want


def test_serialise_rejects_short_output():
    L = airkv.load()
    import ctypes
    buf = ctypes.create_string_buffer(12)
    rc = L.air_kv_block_serialise(1, 2, b"abcd", 4, buf, 12, None)
    assert rc == airkv.AIR_KV_E_INVALID_ARG


# --- the int8 TCP payload ----------------------------------------------------

@pytest.mark.parametrize("seed", [0, 1])
def test_int8_payload_matches_oracle(seed):
    """The payload from the oracle's int8_quantize codes and scale, framed
    by the product, equals the oracle's payload byte for byte; parsing it
    returns the fields."""
    rng = np.random.default_rng(seed)
    for _ in range(20):
        n = int(rng.integers(1, 2048))
        x = (rng.standard_normal(n) * rng.uniform(0.01, 50)).astype(np.float32)
        bits = oracle.bf16_from_f32(x)
        q, s = oracle.pd_int8_quantize(bits)
        bid, layer = int(rng.integers(0, 1 << 32)), int(rng.integers(0, 1 << 16))
        raw = pd_wire.int8_payload(bid, layer, float(s), q)
        assert raw == oracle.tcp_int8_payload(bid, layer, bits)
        got = pd_wire.parse_int8_payload(raw)
        assert got[:2] == (bid, layer) and np.float32(got[2]) == s and np.array_equal(got[3], q)
        assert pd_wire.parse_int8_payload(raw[:-1]) is None


def test_reference_receiver_misreads_int8_payloads():
    """The reference's TCP receiver hands every payload to
    KvBlock::deserialise (src/pd_disagg.rs:238), which reads the scale's
    bits as data_len: a payload whose scale is an ordinary float announces
    ~10^9 data bytes and is dropped.  Kept here as a documented quirk: the
    product parses the layout the sender writes."""
    bits = oracle.bf16_from_f32(np.linspace(-3, 3, 256).astype(np.float32))
    raw = oracle.tcp_int8_payload(9, 1, bits)
    assert oracle.kvblock_deserialise(raw) is None
    assert pd_wire.parse_int8_payload(raw)[0] == 9
