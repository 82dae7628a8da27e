"""KvBlock and the disaggregation wire framing (src/pd_disagg.rs:39-104,
:267-276) over the C ABI.

``KvBlock`` keeps the reference's fields and methods (serialise /
deserialise / int8_quantize); ``frames_from_pool`` and
``int8_payloads_from_pool`` turn device pages into the framed bytes the
reference's connectors send: the device packs the wire data
(air_kv_pack_blocks / air_kv_pack_blocks_int8), the host frames it.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib


@dataclass
class KvBlock:
    block_id: int
    layer_idx: int
    data: bytes          # bf16 wire data [block_size][n_kv_heads][head_dim][K|V]

    def serialise(self) -> bytes:
        """[block_id:4][layer_idx:2][data_len:4][data] (src/pd_disagg.rs:52-62)."""
        L = _lib.load()
        n = len(self.data)
        out = ctypes.create_string_buffer(int(L.air_kv_block_frame_bytes(n)))
        src = ctypes.create_string_buffer(bytes(self.data), n) if n else None
        written = ctypes.c_size_t()
        _lib.check(L.air_kv_block_serialise(self.block_id, self.layer_idx, src, n, out, len(out),
                                            ctypes.byref(written)), "KvBlock.serialise")
        return out.raw[:written.value]

    @staticmethod
    def deserialise(buf: bytes):
        """None where the reference returns None (src/pd_disagg.rs:85-104)."""
        L = _lib.load()
        b = ctypes.create_string_buffer(bytes(buf), len(buf)) if len(buf) else None
        bid, layer = ctypes.c_uint32(), ctypes.c_uint16()
        data, n = ctypes.c_void_p(), ctypes.c_size_t()
        rc = L.air_kv_block_deserialise(b, len(buf), ctypes.byref(bid), ctypes.byref(layer), ctypes.byref(data),
                                        ctypes.byref(n))
        if rc != _lib.AIR_KV_OK:
            return None
        return KvBlock(bid.value, layer.value, bytes(buf[10:10 + n.value]))

    @staticmethod
    def int8_quantize(bf16_data: bytes):
        """(codes int8, scale) of KvBlock::int8_quantize (src/pd_disagg.rs:65-83),
        computed on the device (air_kv_wire_int8_quantize)."""
        from .pool import _torch, wire_int8_quantize
        torch = _torch()
        wire = torch.from_numpy(np.frombuffer(bytes(bf16_data), np.uint8).copy()).cuda().view(1, -1)
        codes, scales = wire_int8_quantize(wire)
        torch.cuda.synchronize()
        return codes.cpu().numpy().reshape(-1), float(scales.cpu().numpy()[0])


def int8_payload(block_id: int, layer_idx: int, scale: float, codes) -> bytes:
    """[block_id:4][layer_idx:2][scale:4][len:4][codes] (src/pd_disagg.rs:267-276)."""
    L = _lib.load()
    c = np.ascontiguousarray(codes, np.int8)
    out = ctypes.create_string_buffer(int(L.air_kv_int8_payload_bytes(len(c))))
    written = ctypes.c_size_t()
    _lib.check(L.air_kv_int8_payload_serialise(block_id, layer_idx, ctypes.c_float(scale),
                                               c.ctypes.data if len(c) else None, len(c), out, len(out),
                                               ctypes.byref(written)), "int8_payload")
    return out.raw[:written.value]


def parse_int8_payload(buf: bytes):
    """(block_id, layer_idx, scale, codes) of an int8 payload, or None."""
    L = _lib.load()
    b = ctypes.create_string_buffer(bytes(buf), len(buf)) if len(buf) else None
    bid, layer, scale = ctypes.c_uint32(), ctypes.c_uint16(), ctypes.c_float()
    codes, n = ctypes.c_void_p(), ctypes.c_size_t()
    rc = L.air_kv_int8_payload_deserialise(b, len(buf), ctypes.byref(bid), ctypes.byref(layer), ctypes.byref(scale),
                                           ctypes.byref(codes), ctypes.byref(n))
    if rc != _lib.AIR_KV_OK:
        return None
    return bid.value, layer.value, scale.value, np.frombuffer(bytes(buf[14:14 + n.value]), np.int8)


def frames_from_pool(pool, ids, layer_idx: int) -> bytes:
    """The serialised KvBlocks of pool blocks `ids` (device pack, host framing),
    back to back."""
    from .pool import _torch
    torch = _torch()
    ids = np.ascontiguousarray(ids, np.int32)
    wire = pool.pack_blocks(torch.from_numpy(ids).cuda())
    host = np.ascontiguousarray(wire.cpu().numpy().view(np.uint8)).reshape(len(ids), -1)
    out = np.empty(len(ids) * (10 + host.shape[1]), np.uint8)
    bids = ids.astype(np.uint32)
    _lib.check(_lib.load().air_kv_block_serialise_n(bids.ctypes.data, layer_idx, host.ctypes.data, host.shape[1],
                                                    len(ids), out.ctypes.data), "frames_from_pool")
    return out.tobytes()


def int8_payloads_from_pool(pool, ids, layer_idx: int) -> bytes:
    """The int8 payloads of pool blocks `ids` (device pack + quantize, host
    framing), back to back."""
    from .pool import _torch
    torch = _torch()
    ids = np.ascontiguousarray(ids, np.int32)
    codes, scales = pool.pack_blocks_int8(torch.from_numpy(ids).cuda())
    c = np.ascontiguousarray(codes.cpu().numpy().view(np.int8)).reshape(len(ids), -1)
    s = np.ascontiguousarray(scales.cpu().numpy(), np.float32)
    out = np.empty(len(ids) * (14 + c.shape[1]), np.uint8)
    bids = ids.astype(np.uint32)
    _lib.check(_lib.load().air_kv_int8_payload_serialise_n(bids.ctypes.data, layer_idx, s.ctypes.data, c.ctypes.data,
                                                           c.shape[1], len(ids), out.ctypes.data),
               "int8_payloads_from_pool")
    return out.tobytes()
