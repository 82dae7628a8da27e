"""CPU oracle for the paged KV-cache path -- TEST INFRASTRUCTURE ONLY.

This package is the checker.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it; the product library never
does.  The arithmetic lives in ``airkv_oracle.c`` (plain C restating the
reference's Rust functions, each cited file:line there); this module wraps it
with numpy and adds the allocator restatement (``paged_attention_ref``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# AIRKV_ORACLE_LIB selects another build of the same sources (the
# AddressSanitizer + UBSan build, `make -C oracle asan`, for the sanitizer test)
LIB_PATH = os.environ.get("AIRKV_ORACLE_LIB") or os.path.join(HERE, "libairkv_oracle.so")

F32, BF16, INT8, FP8 = 0, 1, 2, 3
ELEM_BYTES = {F32: 4, BF16: 2, INT8: 1, FP8: 1}
PAGE_NP_DTYPE = {F32: np.float32, BF16: np.uint16, INT8: np.int8, FP8: np.uint8}

_lock = threading.Lock()
_lib = None

_P = ctypes.c_void_p
_i32, _i64, _u64, _f32, _f64 = ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_double
_SZ = ctypes.c_size_t


def build(force: bool = False) -> str:
    """Compile the oracle with gcc (oracle/Makefile)."""
    args = ["make", "-s", "-C", HERE]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)
    return LIB_PATH


def lib():
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                build()
            L = ctypes.CDLL(LIB_PATH)
            sig = {
                "orc_lcg_next": (_f32, [_P]),
                "orc_lcg_fill": (None, [_u64, _P, _SZ]),
                "orc_box_muller_fill": (None, [_u64, _P, _SZ]),
                "orc_bf16_from_f32": (ctypes.c_uint16, [_f32]),
                "orc_bf16_to_f32": (_f32, [ctypes.c_uint16]),
                "orc_fp8_from_f32": (ctypes.c_uint8, [_f32]),
                "orc_fp8_to_f32": (_f32, [ctypes.c_uint8]),
                "orc_bf16_from_f32_n": (None, [_P, _SZ, _P]),
                "orc_fp8_from_f32_n": (None, [_P, _SZ, _P]),
                "orc_fp8_to_f32_n": (None, [_P, _SZ, _P]),
                "orc_q8_quantize_group": (_f32, [_P, _i32, _P]),
                "orc_q8_quantize": (None, [_P, _SZ, _P, _P]),
                "orc_q8_dequantize": (None, [_P, _P, _SZ, _P]),
                "orc_fp8_quantize_group": (_f32, [_P, _i32, _P]),
                "orc_pd_int8_quantize": (_f32, [_P, _SZ, _P]),
                "orc_kvblock_serialise": (_SZ, [ctypes.c_uint32, ctypes.c_uint16, _P, ctypes.c_uint32, _P]),
                "orc_kvblock_deserialise": (_i32, [_P, _SZ, _P, _P, _P]),
                "orc_tcp_int8_payload": (_SZ, [ctypes.c_uint32, ctypes.c_uint16, _P, _SZ, _P]),
                "orc_kv_append": (_i32, [_i32, _i32, _i32, _i32, _i32, _i64, _P, _P, _P, _i32,
                                         _P, _P, _P, _P]),
                "orc_kv_gather": (_i32, [_i32, _i32, _i32, _i32, _i32, _i64, _P, _P, _P, _P,
                                         _P, _P, _P, _i32, _i32, _P, _P, _i32, _i32]),
                "orc_chunk_attention": (None, [_P, _P, _P, _i32, _i32, _f32, _P, _P, _P]),
                "orc_reduce_chunks": (_i32, [_P, _P, _P, _i32, _i32, _P]),
                "orc_flash_decode": (_i32, [_P, _P, _P, _i32, _i32, _i32, _f32, _P]),
                "orc_reference_attention": (None, [_P, _P, _P, _i32, _i32, _f32, _P]),
                "orc_reference_attention_f64": (None, [_P, _P, _P, _i32, _i32, _f64, _P]),
                "orc_paged_decode": (_i32, [_i32, _i32, _i32, _i32, _i32, _i64, _P, _P, _P, _P,
                                            _P, _i32, _P, _P, _i32, _i32, _f32, _i32, _P]),
                "orc_blockwise_attention_head": (None, [_P, _P, _P, _i32, _i32, _i32, _f32, _i32,
                                                        _i32, _i32, _P]),
                "orc_paged_prefill": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, _i64, _P, _P, _P, _P,
                                             _P, _i32, _P, _P, _P, _i32, _i32, _f32, _i32, _P]),
                "orc_key_compress": (None, [_P, _SZ, _P, _P, _P]),
                "orc_key_decompress": (None, [_P, _f32, _f32, _SZ, _P]),
                "orc_value_compress": (None, [_P, _SZ, _P, _P, _P]),
                "orc_value_decompress": (None, [_P, _f32, _f32, _SZ, _P]),
                "orc_qjl_projection_matrix": (None, [_SZ, _SZ, _u64, _P]),
                "orc_qjl_compress": (None, [_P, _SZ, _P, _SZ, _P, _P]),
                "orc_qjl_cos_sim": (_f32, [_P, _P, _SZ]),
            }
            for name, (res, args) in sig.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# generators
# --------------------------------------------------------------------------

def lcg_fill(seed: int, n: int) -> np.ndarray:
    """Uniform [-1, 1) stream of the reference's flash_decode tests."""
    out = np.empty(n, np.float32)
    lib().orc_lcg_fill(seed, _ptr(out), n)
    return out


def box_muller_fill(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_box_muller_fill(seed, _ptr(out), n)
    return out


# --------------------------------------------------------------------------
# scalar codecs (vectorised by looping in C where it matters)
# --------------------------------------------------------------------------

def bf16_from_f32(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_from_f32_n(_ptr(x), x.size, _ptr(out))
    return out


def fp8_from_f32(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().orc_fp8_from_f32_n(_ptr(x), x.size, _ptr(out))
    return out


def fp8_to_f32(b) -> np.ndarray:
    b = _c(b, np.uint8)
    out = np.empty(b.shape, np.float32)
    lib().orc_fp8_to_f32_n(_ptr(b), b.size, _ptr(out))
    return out


def bf16_to_f32(b) -> np.ndarray:
    b = _c(b, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def fp8_from_f32_scalar(x: float) -> int:
    return lib().orc_fp8_from_f32(ctypes.c_float(x))


def fp8_to_f32_scalar(b: int) -> float:
    return lib().orc_fp8_to_f32(b)


def fp8_decode_table() -> np.ndarray:
    L = lib()
    return np.array([L.orc_fp8_to_f32(b) for b in range(256)], np.float32)


def q8_quantize(x):
    """Q8Tensor::quantize over a flat buffer -> (codes int8, scales f32)."""
    x = _c(x, np.float32).ravel()
    q = np.empty(len(x), np.int8)
    s = np.empty((len(x) + 31) // 32, np.float32)
    lib().orc_q8_quantize(_ptr(x), len(x), _ptr(q), _ptr(s))
    return q, s


def q8_dequantize(q, s):
    q = _c(q, np.int8).ravel()
    s = _c(s, np.float32).ravel()
    out = np.empty(len(q), np.float32)
    lib().orc_q8_dequantize(_ptr(q), _ptr(s), len(q), _ptr(out))
    return out


def fp8_quantize_group(x):
    x = _c(x, np.float32).ravel()
    q = np.empty(len(x), np.uint8)
    s = lib().orc_fp8_quantize_group(_ptr(x), len(x), _ptr(q))
    return q, np.float32(s)


def pd_int8_quantize(bf16_bits):
    b = _c(bf16_bits, np.uint16).ravel()
    q = np.empty(len(b), np.int8)
    s = lib().orc_pd_int8_quantize(_ptr(b), len(b), _ptr(q))
    return q, np.float32(s)


def kvblock_serialise(block_id, layer_idx, data: bytes) -> bytes:
    """KvBlock::serialise (src/pd_disagg.rs:52-62)."""
    d = np.frombuffer(bytes(data), np.uint8)
    out = np.empty(10 + len(d), np.uint8)
    n = lib().orc_kvblock_serialise(block_id, layer_idx, _ptr(d) if len(d) else None, len(d), _ptr(out))
    return out[:n].tobytes()


def kvblock_deserialise(buf: bytes):
    """KvBlock::deserialise (src/pd_disagg.rs:85-104): None or
    (block_id, layer_idx, data)."""
    b = np.frombuffer(bytes(buf), np.uint8)
    bid, layer, n = ctypes.c_uint32(), ctypes.c_uint16(), ctypes.c_uint32()
    ok = lib().orc_kvblock_deserialise(_ptr(b) if len(b) else None, len(b), ctypes.byref(bid),
                                       ctypes.byref(layer), ctypes.byref(n))
    if not ok:
        return None
    return bid.value, layer.value, b[10:10 + n.value].tobytes()


def tcp_int8_payload(block_id, layer_idx, bf16_bits) -> bytes:
    """The int8 payload TcpKvConnector::send_blocks writes (src/pd_disagg.rs:267-276)."""
    b = _c(bf16_bits, np.uint16).ravel()
    out = np.empty(14 + len(b), np.uint8)
    n = lib().orc_tcp_int8_payload(block_id, layer_idx, _ptr(b), len(b), _ptr(out))
    return out[:n].tobytes()


# --------------------------------------------------------------------------
# paged pool (host mirror of the device layout)
# --------------------------------------------------------------------------

class HostPool:
    """Host copy of one layer's paged pool in the device layout."""

    def __init__(self, num_blocks, block_size, n_kv_heads, head_dim, dtype=F32, group=32,
                 fill=0):
        self.num_blocks, self.block_size = int(num_blocks), int(block_size)
        self.n_kv_heads, self.head_dim, self.dtype = int(n_kv_heads), int(head_dim), int(dtype)
        self.group = int(group)
        shape = (self.num_blocks, self.n_kv_heads, self.block_size, self.head_dim)
        npd = PAGE_NP_DTYPE[self.dtype]
        self.k = np.full(shape, fill, npd)
        self.v = np.full(shape, fill, npd)
        if self.dtype in (INT8, FP8):
            sshape = shape[:3] + (self.head_dim // self.group,)
            self.k_scales = np.zeros(sshape, np.float32)
            self.v_scales = np.zeros(sshape, np.float32)
        else:
            self.k_scales = self.v_scales = None

    def append(self, k_src, v_src, slot_mapping) -> int:
        k_src = _c(k_src, np.float32)
        v_src = _c(v_src, np.float32)
        slots = _c(slot_mapping, np.int64)
        n = len(slots)
        assert k_src.size == n * self.n_kv_heads * self.head_dim
        return lib().orc_kv_append(self.dtype, self.block_size, self.n_kv_heads, self.head_dim,
                                   self.group, self.num_blocks, _ptr(k_src), _ptr(v_src),
                                   _ptr(slots), n, _ptr(self.k), _ptr(self.v),
                                   _ptr(self.k_scales), _ptr(self.v_scales))

    def gather(self, block_tables, seq_lens, out_dtype=F32, out_layout=0):
        tables = _c(block_tables, np.int32)
        lens = _c(seq_lens, np.int32)
        batch, max_blocks = tables.shape
        per = lens.astype(np.int64) * self.n_kv_heads * self.head_dim
        offs = np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)
        total = int(per.sum())
        odt = np.float32 if out_dtype == F32 else np.uint16
        ok = np.zeros(total, odt)
        ov = np.zeros(total, odt)
        bad = lib().orc_kv_gather(self.dtype, self.block_size, self.n_kv_heads, self.head_dim,
                                  self.group, self.num_blocks, _ptr(self.k), _ptr(self.v),
                                  _ptr(self.k_scales), _ptr(self.v_scales), _ptr(tables),
                                  _ptr(lens), _ptr(offs), batch, max_blocks, _ptr(ok), _ptr(ov),
                                  out_dtype, out_layout)
        return ok, ov, offs, bad

    def paged_prefill(self, q, cu_q, block_tables, seq_lens, scale=None, kv_block=512):
        """Causal attention of each sequence's newest cu_q[b+1] - cu_q[b]
        tokens over its pages (blockwise_attention_head with q_offset =
        seq_len - q_len).  q: [total_q][n_q][d] f32."""
        q = _c(q, np.float32)
        total, n_q, d = q.shape
        tables = _c(block_tables, np.int32)
        lens = _c(seq_lens, np.int32)
        cu = _c(cu_q, np.int32)
        if scale is None:
            scale = np.float32(1.0) / np.sqrt(np.float32(d))
        out = np.empty_like(q)
        rc = lib().orc_paged_prefill(self.dtype, self.block_size, self.n_kv_heads, self.head_dim,
                                     self.group, n_q // self.n_kv_heads, self.num_blocks, _ptr(self.k),
                                     _ptr(self.v), _ptr(self.k_scales), _ptr(self.v_scales), _ptr(q), n_q,
                                     _ptr(cu), _ptr(tables), _ptr(lens), len(lens), tables.shape[1],
                                     float(scale), kv_block, _ptr(out))
        if rc:
            raise ValueError("oracle paged_prefill rejected its inputs")
        return out

    def paged_decode(self, q, block_tables, seq_lens, scale=None, chunk=64):
        q = _c(q, np.float32)
        batch, n_q, d = q.shape
        tables = _c(block_tables, np.int32)
        lens = _c(seq_lens, np.int32)
        if scale is None:
            scale = np.float32(1.0) / np.sqrt(np.float32(d))
        out = np.empty_like(q)
        rc = lib().orc_paged_decode(self.dtype, self.block_size, self.n_kv_heads, self.head_dim,
                                    self.group, self.num_blocks, _ptr(self.k), _ptr(self.v),
                                    _ptr(self.k_scales), _ptr(self.v_scales), _ptr(q), n_q,
                                    _ptr(tables), _ptr(lens), batch, tables.shape[1],
                                    float(scale), chunk, _ptr(out))
        if rc:
            raise ValueError("oracle paged_decode rejected its inputs")
        return out


# --------------------------------------------------------------------------
# flash decode
# --------------------------------------------------------------------------

def flash_decode(q, k, v, kv_len, head_dim, chunk, scale=None):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    if scale is None:
        scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
    out = np.empty(head_dim, np.float32)
    rc = lib().orc_flash_decode(_ptr(q), _ptr(k), _ptr(v), kv_len, head_dim, chunk,
                                float(scale), _ptr(out))
    if rc:
        raise ValueError("flash_decode: reference assertion (no chunks or zero sum)")
    return out


def chunk_attention(q, k, v, head_dim, scale=None):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    if scale is None:
        scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
    out = np.empty(head_dim, np.float32)
    m, l = ctypes.c_float(), ctypes.c_float()
    lib().orc_chunk_attention(_ptr(q), _ptr(k), _ptr(v), k.size // head_dim, head_dim,
                              float(scale), _ptr(out), ctypes.byref(m), ctypes.byref(l))
    return out, m.value, l.value


def reduce_chunks(outs, maxes, sums, head_dim):
    outs = _c(outs, np.float32)
    maxes, sums = _c(maxes, np.float32), _c(sums, np.float32)
    out = np.empty(head_dim, np.float32)
    rc = lib().orc_reduce_chunks(_ptr(outs), _ptr(maxes), _ptr(sums), len(maxes), head_dim,
                                 _ptr(out))
    if rc:
        raise ValueError("reduce_chunks: reference assertion")
    return out


def reference_attention(q, k, v, kv_len, head_dim, scale=None):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    if scale is None:
        scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
    out = np.empty(head_dim, np.float32)
    lib().orc_reference_attention(_ptr(q), _ptr(k), _ptr(v), kv_len, head_dim, float(scale),
                                  _ptr(out))
    return out


def reference_attention_f64(q, k, v, kv_len, head_dim, scale=None):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    if scale is None:
        scale = 1.0 / np.sqrt(float(head_dim))
    out = np.empty(head_dim, np.float64)
    lib().orc_reference_attention_f64(_ptr(q), _ptr(k), _ptr(v), kv_len, head_dim,
                                      float(scale), _ptr(out))
    return out


def max_abs_error(a, b) -> float:
    """src/flash_decode.rs:210-212."""
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


# --------------------------------------------------------------------------
# kv_compress warm-tier codecs (src/kv_compress.rs)
# --------------------------------------------------------------------------

def key_compress(key):
    """CompressedKey::compress -> (sign bits uint64[ceil(d/64)], magnitude, mean)."""
    key = _c(key, np.float32).ravel()
    bits = np.zeros(max((len(key) + 63) // 64, 1), np.uint64)
    mag, mean = ctypes.c_float(), ctypes.c_float()
    lib().orc_key_compress(_ptr(key), len(key), _ptr(bits), ctypes.byref(mag), ctypes.byref(mean))
    return bits[:(len(key) + 63) // 64], np.float32(mag.value), np.float32(mean.value)


def key_decompress(bits, magnitude, mean, dim):
    bits = _c(bits, np.uint64)
    out = np.empty(dim, np.float32)
    lib().orc_key_decompress(_ptr(bits) if bits.size else None, float(magnitude), float(mean), dim,
                             _ptr(out))
    return out


def value_compress(v):
    """CompressedValue::compress -> (codes uint8[d], scale, min)."""
    v = _c(v, np.float32).ravel()
    q = np.empty(len(v), np.uint8)
    scale, mn = ctypes.c_float(), ctypes.c_float()
    lib().orc_value_compress(_ptr(v), len(v), _ptr(q), ctypes.byref(scale), ctypes.byref(mn))
    return q, np.float32(scale.value), np.float32(mn.value)


def value_decompress(q, scale, min_val):
    q = _c(q, np.uint8).ravel()
    out = np.empty(len(q), np.float32)
    lib().orc_value_decompress(_ptr(q), float(scale), float(min_val), len(q), _ptr(out))
    return out


def qjl_projection_matrix(proj_dim, orig_dim, seed):
    out = np.empty(proj_dim * orig_dim, np.float32)
    lib().orc_qjl_projection_matrix(proj_dim, orig_dim, seed, _ptr(out))
    return out


def qjl_compress(key, proj, proj_dim):
    """QjlKey::compress -> (bits uint64[ceil(m/64)], magnitude)."""
    key = _c(key, np.float32).ravel()
    proj = _c(proj, np.float32).ravel()
    assert proj.size == proj_dim * key.size
    bits = np.zeros((proj_dim + 63) // 64, np.uint64)
    mag = ctypes.c_float()
    lib().orc_qjl_compress(_ptr(key), len(key), _ptr(proj), proj_dim, _ptr(bits), ctypes.byref(mag))
    return bits, np.float32(mag.value)


def qjl_cos_sim(a, b, proj_dim):
    return np.float32(lib().orc_qjl_cos_sim(_ptr(_c(a, np.uint64)), _ptr(_c(b, np.uint64)), proj_dim))


# --------------------------------------------------------------------------
# blockwise causal attention (src/chunked_attn.rs)
# --------------------------------------------------------------------------

def blockwise_attention_head(q, k, v, seq_q, seq_kv, head_dim, scale, block_size, causal, q_offset):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    out = np.empty(seq_q * head_dim, np.float32)
    lib().orc_blockwise_attention_head(_ptr(q), _ptr(k), _ptr(v), seq_q, seq_kv, head_dim, float(scale),
                                       block_size, 1 if causal else 0, q_offset, _ptr(out))
    return out
