"""Warm-tier KV codecs of src/kv_compress.rs on the GPU (batched).

The reference compresses one vector per call (CompressedKey::compress,
CompressedValue::compress, QjlKey::compress); these take [n_rows][dim]
device tensors and return every row's result at once, bit-exact with the
reference.  Bits are returned as int64 tensors holding the reference's u64
words (torch has no general uint64 arithmetic); reinterpret with
`.cpu().numpy().view(np.uint64)`.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import BF16, F32
from .pool import _dev, _stream_ptr, _torch


def _rows(rows):
    torch = _torch()
    if rows.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("rows must be float32 or bfloat16")
    if rows.dim() != 2:
        raise ValueError("rows must be [n_rows][dim]")
    _dev(rows, rows.dtype, "rows")
    return (F32 if rows.dtype == torch.float32 else BF16), rows.shape[0], rows.shape[1]


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def key_compress(rows, stream=None):
    """CompressedKey::compress of every row -> (bits int64[n][ceil(d/64)],
    magnitude f32[n], mean f32[n])."""
    torch = _torch()
    dt, n, d = _rows(rows)
    bits = torch.empty((n, (d + 63) // 64), dtype=torch.int64, device=rows.device)
    mag = torch.empty(n, dtype=torch.float32, device=rows.device)
    mean = torch.empty(n, dtype=torch.float32, device=rows.device)
    _lib.check(_lib.load().air_kv_key_compress(_stream_ptr(stream), _ptr(rows), dt, n, d, _ptr(bits),
                                               _ptr(mag), _ptr(mean)), "air_kv_key_compress")
    return bits, mag, mean


def key_decompress(bits, magnitude, mean, dim, stream=None):
    torch = _torch()
    n = magnitude.shape[0]
    _dev(bits, torch.int64, "bits", (n, (dim + 63) // 64))
    _dev(magnitude, torch.float32, "magnitude", (n,))
    _dev(mean, torch.float32, "mean", (n,))
    out = torch.empty((n, dim), dtype=torch.float32, device=bits.device)
    _lib.check(_lib.load().air_kv_key_decompress(_stream_ptr(stream), _ptr(bits), _ptr(magnitude),
                                                 _ptr(mean), n, dim, _ptr(out)), "air_kv_key_decompress")
    return out


def value_compress(rows, stream=None):
    """CompressedValue::compress of every row -> (codes uint8[n][d],
    scale f32[n], min f32[n])."""
    torch = _torch()
    dt, n, d = _rows(rows)
    codes = torch.empty((n, d), dtype=torch.uint8, device=rows.device)
    scale = torch.empty(n, dtype=torch.float32, device=rows.device)
    mn = torch.empty(n, dtype=torch.float32, device=rows.device)
    _lib.check(_lib.load().air_kv_value_compress(_stream_ptr(stream), _ptr(rows), dt, n, d, _ptr(codes),
                                                 _ptr(scale), _ptr(mn)), "air_kv_value_compress")
    return codes, scale, mn


def value_decompress(codes, scale, min_val, stream=None):
    torch = _torch()
    n, d = codes.shape
    _dev(codes, torch.uint8, "codes")
    _dev(scale, torch.float32, "scale", (n,))
    _dev(min_val, torch.float32, "min_val", (n,))
    out = torch.empty((n, d), dtype=torch.float32, device=codes.device)
    _lib.check(_lib.load().air_kv_value_decompress(_stream_ptr(stream), _ptr(codes), _ptr(scale),
                                                   _ptr(min_val), n, d, _ptr(out)),
               "air_kv_value_decompress")
    return out


def qjl_compress(rows, proj, proj_dim, stream=None):
    """QjlKey::compress of every row with the [proj_dim][d] matrix `proj` ->
    (bits int64[n][ceil(m/64)], magnitude f32[n])."""
    torch = _torch()
    dt, n, d = _rows(rows)
    _dev(proj, torch.float32, "proj")
    if proj.numel() != proj_dim * d:
        raise ValueError("proj must hold proj_dim x dim values")
    bits = torch.empty((n, (proj_dim + 63) // 64), dtype=torch.int64, device=rows.device)
    mag = torch.empty(n, dtype=torch.float32, device=rows.device)
    _lib.check(_lib.load().air_kv_qjl_compress(_stream_ptr(stream), _ptr(rows), dt, n, d, _ptr(proj),
                                               proj_dim, _ptr(bits), _ptr(mag)), "air_kv_qjl_compress")
    return bits, mag


def qjl_scores(key_bits, key_magnitude, query_bits, query_magnitude, proj_dim, stream=None):
    """approx_cos_sim and approx_dot of one query against every key."""
    torch = _torch()
    n = key_bits.shape[0]
    w = (proj_dim + 63) // 64
    _dev(key_bits, torch.int64, "key_bits", (n, w))
    _dev(key_magnitude, torch.float32, "key_magnitude", (n,))
    _dev(query_bits, torch.int64, "query_bits", (w,))
    cos = torch.empty(n, dtype=torch.float32, device=key_bits.device)
    dot = torch.empty(n, dtype=torch.float32, device=key_bits.device)
    _lib.check(_lib.load().air_kv_qjl_scores(_stream_ptr(stream), _ptr(key_bits), _ptr(key_magnitude), n,
                                             proj_dim, _ptr(query_bits), float(query_magnitude), _ptr(cos),
                                             _ptr(dot)), "air_kv_qjl_scores")
    return cos, dot


def compress_blocks(pool, ids, stream=None):
    """Warm-tier compression of pool blocks (CompressedKvEntry::compress per
    (head, token) row, rows ordered [block][head][token]) -> dict of tensors."""
    torch = _torch()
    _dev(ids, torch.int32, "ids")
    n = ids.shape[0]
    rows = n * pool.n_kv_heads * pool.block_size
    d = pool.head_dim
    dev = ids.device
    out = {
        "key_bits": torch.empty((rows, (d + 63) // 64), dtype=torch.int64, device=dev),
        "key_magnitude": torch.empty(rows, dtype=torch.float32, device=dev),
        "key_mean": torch.empty(rows, dtype=torch.float32, device=dev),
        "value_codes": torch.empty((rows, d), dtype=torch.uint8, device=dev),
        "value_scale": torch.empty(rows, dtype=torch.float32, device=dev),
        "value_min": torch.empty(rows, dtype=torch.float32, device=dev),
    }
    _lib.check(_lib.load().air_kv_compress_blocks(
        pool.handle, _stream_ptr(stream), _ptr(ids), n, _ptr(out["key_bits"]), _ptr(out["key_magnitude"]),
        _ptr(out["key_mean"]), _ptr(out["value_codes"]), _ptr(out["value_scale"]), _ptr(out["value_min"])),
        "air_kv_compress_blocks")
    return out


def qjl_compress_blocks(pool, ids, proj, proj_dim, stream=None):
    torch = _torch()
    _dev(ids, torch.int32, "ids")
    _dev(proj, torch.float32, "proj")
    n = ids.shape[0]
    rows = n * pool.n_kv_heads * pool.block_size
    bits = torch.empty((rows, (proj_dim + 63) // 64), dtype=torch.int64, device=ids.device)
    mag = torch.empty(rows, dtype=torch.float32, device=ids.device)
    _lib.check(_lib.load().air_kv_qjl_compress_blocks(pool.handle, _stream_ptr(stream), _ptr(ids), n,
                                                      _ptr(proj), proj_dim, _ptr(bits), _ptr(mag)),
               "air_kv_qjl_compress_blocks")
    return bits, mag


def as_u64(bits) -> np.ndarray:
    """Device int64 bit words -> host uint64 (the reference's u64 words)."""
    return bits.cpu().numpy().view(np.uint64)
