"""Device pool bound to torch tensors (the C ABI with shape checks in front).

torch supplies device memory and streams; every byte of K/V work is done by
the HIP kernels in libairkv.so.  Shapes, dtypes and devices are validated on
the host before each launch so a kernel never sees operands that disagree
with its grid.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import BF16, F32, FP8, INT8, LAYOUT_HEAD_MAJOR, PoolDesc

ELEM_BYTES = {F32: 4, BF16: 2, INT8: 1, FP8: 1}
PAGE_NP_DTYPE = {F32: np.float32, BF16: np.uint16, INT8: np.int8, FP8: np.uint8}


def _torch():
    import torch
    return torch


def _stream_ptr(stream):
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _dev(t, dtype, what, shape=None):
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{what} must be a CUDA/HIP torch tensor")
    if t.dtype != dtype:
        raise TypeError(f"{what} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{what} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    return ctypes.c_void_p(t.data_ptr())


def _launcher(fn, args, name, keep):
    """A zero-argument launcher of fn(*args).  args holds raw device
    addresses, so the launcher also holds `keep`, every tensor (and stream)
    those addresses point into: they live as long as the launcher does.
    Without that, a tensor the caller dropped would return to torch's caching
    allocator while the launcher still wrote through its address."""
    def launch():
        rc = fn(*args)
        if rc:
            _lib.check(rc, name)
    launch.keep = tuple(keep)
    return launch


_TORCH_OF = {F32: "float32", BF16: "bfloat16"}


class KvPool:
    """One layer's paged K/V pool on the current HIP device."""

    def __init__(self, num_blocks, block_size=16, n_kv_heads=8, head_dim=128, dtype=BF16,
                 scale_group=32):
        L = _lib.load()
        d = PoolDesc(num_blocks, block_size, n_kv_heads, head_dim, dtype, scale_group)
        h = ctypes.c_void_p()
        _lib.check(L.air_kv_pool_create(ctypes.byref(d), ctypes.byref(h)), "air_kv_pool_create")
        self.handle = h
        info = PoolDesc()
        bb = ctypes.c_size_t()
        ptrs = [ctypes.c_void_p() for _ in range(4)]
        _lib.check(L.air_kv_pool_info(h, ctypes.byref(info), *[ctypes.byref(p) for p in ptrs],
                                      ctypes.byref(bb)))
        self.num_blocks, self.block_size = info.num_blocks, info.block_size
        self.n_kv_heads, self.head_dim = info.n_kv_heads, info.head_dim
        self.dtype, self.scale_group = info.dtype, info.scale_group
        self.block_bytes = bb.value
        # device base pointers of the pool's arrays (k_pages, v_pages, k_scales, v_scales)
        self.device_ptrs = tuple(p.value or 0 for p in ptrs)
        self.quantized = dtype in (INT8, FP8)
        rows = self.n_kv_heads * self.block_size
        self.slab_bytes = rows * self.head_dim * ELEM_BYTES[dtype]
        self.scale_slab_bytes = rows * (self.head_dim // self.scale_group) * 4 if self.quantized else 0

    def close(self):
        if getattr(self, "handle", None):
            _lib.load().air_kv_pool_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- kernels --------------------------------------------------------------

    def append(self, k, v, slot_mapping, stream=None):
        torch = _torch()
        n = slot_mapping.shape[0] if slot_mapping.dim() == 1 else -1
        shape = (n, self.n_kv_heads, self.head_dim)
        kp = _dev(k, torch.float32, "k", shape)
        vp = _dev(v, torch.float32, "v", shape)
        sp = _dev(slot_mapping, torch.int64, "slot_mapping", (n,))
        _lib.check(_lib.load().air_kv_append(self.handle, _stream_ptr(stream), kp, vp, sp, n),
                   "air_kv_append")

    def gather(self, block_tables, seq_lens, out_offsets, out_k, out_v, out_dtype=None,
               layout=LAYOUT_HEAD_MAJOR, stream=None, validate=True):
        torch = _torch()
        if out_dtype is None:
            out_dtype = F32 if self.dtype == F32 else BF16
        batch, max_blocks = block_tables.shape
        _dev(block_tables, torch.int32, "block_tables")
        _dev(seq_lens, torch.int32, "seq_lens", (batch,))
        _dev(out_offsets, torch.int64, "out_offsets", (batch,))
        tdt = torch.float32 if out_dtype == F32 else torch.bfloat16
        _dev(out_k, tdt, "out_k")
        _dev(out_v, tdt, "out_v")
        if out_k.numel() != out_v.numel():
            raise ValueError("out_k and out_v differ in size")
        if validate and batch:
            lens = seq_lens.cpu().numpy().astype(np.int64)
            offs = out_offsets.cpu().numpy()
            lens = np.clip(lens, 0, max_blocks * self.block_size)
            end = offs + lens * self.n_kv_heads * self.head_dim
            if (offs < 0).any() or int(end.max()) > out_k.numel():
                raise ValueError("gather output buffers are too small for seq_lens/out_offsets")
        _lib.check(_lib.load().air_kv_gather(
            self.handle, _stream_ptr(stream), ctypes.c_void_p(block_tables.data_ptr()),
            ctypes.c_void_p(seq_lens.data_ptr()), ctypes.c_void_p(out_offsets.data_ptr()), batch,
            max_blocks, ctypes.c_void_p(out_k.data_ptr()), ctypes.c_void_p(out_v.data_ptr()),
            out_dtype, layout), "air_kv_gather")

    def decode_workspace_size(self, n_q_heads, batch, max_blocks, max_splits=64):
        out = ctypes.c_size_t()
        _lib.check(_lib.load().air_paged_decode_workspace_size(self.handle, n_q_heads, batch,
                                                               max_blocks, max_splits,
                                                               ctypes.byref(out)))
        return out.value

    def new_workspace(self, n_q_heads, batch, max_blocks, max_splits=64):
        torch = _torch()
        n = self.decode_workspace_size(n_q_heads, batch, max_blocks, max_splits)
        return torch.empty(max(n, 16), dtype=torch.uint8, device="cuda")

    def _decode_args(self, q, block_tables, seq_lens, out, scale, max_splits, workspace, stream):
        torch = _torch()
        batch, n_q, d = q.shape
        if d != self.head_dim:
            raise ValueError("q head_dim differs from the pool")
        if q.dtype not in (torch.float32, torch.bfloat16) or out.dtype not in (torch.float32,
                                                                               torch.bfloat16):
            raise TypeError("q and out must be float32 or bfloat16")
        _dev(q, q.dtype, "q")
        _dev(out, out.dtype, "out", (batch, n_q, d))
        _dev(block_tables, torch.int32, "block_tables")
        if block_tables.shape[0] != batch:
            raise ValueError("block_tables rows differ from batch")
        _dev(seq_lens, torch.int32, "seq_lens", (batch,))
        max_blocks = block_tables.shape[1]
        if workspace is None:
            workspace = self.new_workspace(n_q, batch, max_blocks, max_splits)
        _dev(workspace, workspace.dtype, "workspace")
        ws_bytes = workspace.numel() * workspace.element_size()
        if scale is None:
            scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
        qdt = F32 if q.dtype == torch.float32 else BF16
        odt = F32 if out.dtype == torch.float32 else BF16
        head = (self.handle, _stream_ptr(stream), ctypes.c_void_p(q.data_ptr()), qdt, n_q)
        tail = (ctypes.c_void_p(block_tables.data_ptr()), ctypes.c_void_p(seq_lens.data_ptr()), batch,
                max_blocks, scale, max_splits, ctypes.c_void_p(workspace.data_ptr()), ws_bytes,
                ctypes.c_void_p(out.data_ptr()), odt)
        return head, tail

    def _new_rows(self, q, k_new, v_new):
        torch = _torch()
        shape = (q.shape[0], self.n_kv_heads, self.head_dim)
        _dev(k_new, torch.float32, "k_new", shape)
        _dev(v_new, torch.float32, "v_new", shape)
        return (ctypes.c_void_p(k_new.data_ptr()), ctypes.c_void_p(v_new.data_ptr()))

    def paged_decode(self, q, block_tables, seq_lens, out, scale=None, max_splits=64,
                     workspace=None, stream=None):
        head, tail = self._decode_args(q, block_tables, seq_lens, out, scale, max_splits, workspace, stream)
        _lib.check(_lib.load().air_paged_decode(*head, *tail), "air_paged_decode")
        return out

    def paged_decode_append(self, q, k_new, v_new, block_tables, seq_lens, out, scale=None,
                            max_splits=64, workspace=None, stream=None):
        """One decode step: append k_new / v_new (float32 [batch, n_kv_heads,
        head_dim]) as each sequence's token seq_lens[b] - 1, then attend as
        paged_decode.  One launch on pools of the matrix-core decode (head_dim
        128, BF16, or INT8 / FP8 quantized as append quantizes); every other
        pool appends, then decodes, with the same result."""
        head, tail = self._decode_args(q, block_tables, seq_lens, out, scale, max_splits, workspace, stream)
        rows = self._new_rows(q, k_new, v_new)
        _lib.check(_lib.load().air_paged_decode_append(*head, *rows, *tail), "air_paged_decode_append")
        return out

    def bind_decode(self, q, block_tables, seq_lens, out, workspace, scale=None, max_splits=64,
                    stream=None):
        """Validate once, return a zero-argument launcher (for timing loops:
        no per-call Python checks between launches)."""
        if workspace is None:
            workspace = self.new_workspace(q.shape[1], q.shape[0], block_tables.shape[1], max_splits)
        self.paged_decode(q, block_tables, seq_lens, out, scale, max_splits, workspace, stream)
        head, tail = self._decode_args(q, block_tables, seq_lens, out, scale, max_splits, workspace, stream)
        return _launcher(_lib.load().air_paged_decode, head + tail, "air_paged_decode",
                         (q, block_tables, seq_lens, out, workspace, stream))

    def bind_decode_append(self, q, k_new, v_new, block_tables, seq_lens, out, workspace, scale=None,
                           max_splits=64, stream=None):
        """bind_decode for paged_decode_append.  The launcher appends on every
        call: a timing loop rewrites the same rows with the same values."""
        if workspace is None:
            workspace = self.new_workspace(q.shape[1], q.shape[0], block_tables.shape[1], max_splits)
        self.paged_decode_append(q, k_new, v_new, block_tables, seq_lens, out, scale, max_splits,
                                 workspace, stream)
        head, tail = self._decode_args(q, block_tables, seq_lens, out, scale, max_splits, workspace, stream)
        return _launcher(_lib.load().air_paged_decode_append, head + self._new_rows(q, k_new, v_new) + tail,
                         "air_paged_decode_append",
                         (q, k_new, v_new, block_tables, seq_lens, out, workspace, stream))

    def prefill_workspace_size(self, n_q_heads, batch, max_q_len):
        """Bytes of the key-split workspace air_paged_prefill takes for this shape."""
        n = ctypes.c_size_t(0)
        _lib.check(_lib.load().air_paged_prefill_workspace_size(self.handle, n_q_heads, batch, max_q_len,
                                                                ctypes.byref(n)),
                   "air_paged_prefill_workspace_size")
        return n.value

    def _prefill_args(self, q, cu_q, block_tables, seq_lens, out, max_q_len, scale, stream, workspace,
                      split):
        torch = _torch()
        total_q, n_q, d = q.shape
        if d != self.head_dim:
            raise ValueError("q head_dim differs from the pool")
        if n_q % self.n_kv_heads:
            raise ValueError("n_q_heads must be a multiple of n_kv_heads")
        if q.dtype not in (torch.float32, torch.bfloat16) or out.dtype not in (torch.float32,
                                                                               torch.bfloat16):
            raise TypeError("q and out must be float32 or bfloat16")
        _dev(q, q.dtype, "q")
        _dev(out, out.dtype, "out", (total_q, n_q, d))
        _dev(block_tables, torch.int32, "block_tables")
        batch = block_tables.shape[0]
        _dev(seq_lens, torch.int32, "seq_lens", (batch,))
        _dev(cu_q, torch.int32, "cu_q", (batch + 1,))
        if max_q_len is None:
            max_q_len = int((cu_q[1:] - cu_q[:-1]).max().item()) if batch else 0
        if scale is None:
            scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
        qdt = F32 if q.dtype == torch.float32 else BF16
        odt = F32 if out.dtype == torch.float32 else BF16
        if split and workspace is None and batch:
            n = self.prefill_workspace_size(n_q, batch, max_q_len)
            if n:
                workspace = torch.empty(n, dtype=torch.uint8, device="cuda")
        if not split:
            workspace = None
        ws_ptr = ctypes.c_void_p(workspace.data_ptr()) if workspace is not None else None
        ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
        # the workspace tensor rides along in the tuple so a bound launcher keeps it alive
        return (self.handle, _stream_ptr(stream), ctypes.c_void_p(q.data_ptr()), qdt, n_q,
                ctypes.c_void_p(cu_q.data_ptr()), total_q, max_q_len,
                ctypes.c_void_p(block_tables.data_ptr()), ctypes.c_void_p(seq_lens.data_ptr()), batch,
                block_tables.shape[1], scale, ws_ptr, ws_bytes, ctypes.c_void_p(out.data_ptr()), odt), workspace

    def paged_prefill(self, q, cu_q, block_tables, seq_lens, out, max_q_len=None, scale=None,
                      stream=None, workspace=None, split=True):
        """Causal attention of each sequence's newest cu_q[b+1] - cu_q[b]
        tokens over its pages (air_paged_prefill).  q / out: [total_q][n_q][d];
        cu_q int32 [batch + 1]; max_q_len defaults to the largest q_len (read
        back from cu_q, which synchronises).  With split (the default) long
        work groups' keys are cut over several workgroups through a workspace
        (allocated here when none is given); split=False passes none."""
        args, _ws = self._prefill_args(q, cu_q, block_tables, seq_lens, out, max_q_len, scale, stream,
                                       workspace, split)
        _lib.check(_lib.load().air_paged_prefill(*args), "air_paged_prefill")
        return out

    def bind_prefill(self, q, cu_q, block_tables, seq_lens, out, max_q_len=None, scale=None,
                     stream=None, workspace=None, split=True):
        """Validate once, return a zero-argument prefill launcher."""
        args, ws = self._prefill_args(q, cu_q, block_tables, seq_lens, out, max_q_len, scale, stream,
                                      workspace, split)
        fn = _lib.load().air_paged_prefill
        _lib.check(fn(*args), "air_paged_prefill")
        launch = _launcher(fn, args, "air_paged_prefill", (q, cu_q, block_tables, seq_lens, out, ws, stream))
        launch.workspace = ws
        return launch

    def bind_append(self, k, v, slot_mapping, stream=None):
        """Validate once, return a zero-argument append launcher."""
        self.append(k, v, slot_mapping, stream)
        fn = _lib.load().air_kv_append
        args = (self.handle, _stream_ptr(stream), ctypes.c_void_p(k.data_ptr()),
                ctypes.c_void_p(v.data_ptr()), ctypes.c_void_p(slot_mapping.data_ptr()),
                slot_mapping.shape[0])
        return _launcher(fn, args, "air_kv_append", (k, v, slot_mapping, stream))

    def bind_gather(self, block_tables, seq_lens, out_offsets, out_k, out_v, out_dtype=None,
                    layout=LAYOUT_HEAD_MAJOR, stream=None):
        """Validate once, return a zero-argument gather launcher."""
        if out_dtype is None:
            out_dtype = F32 if self.dtype == F32 else BF16
        self.gather(block_tables, seq_lens, out_offsets, out_k, out_v, out_dtype, layout, stream)
        fn = _lib.load().air_kv_gather
        args = (self.handle, _stream_ptr(stream), ctypes.c_void_p(block_tables.data_ptr()),
                ctypes.c_void_p(seq_lens.data_ptr()), ctypes.c_void_p(out_offsets.data_ptr()),
                block_tables.shape[0], block_tables.shape[1], ctypes.c_void_p(out_k.data_ptr()),
                ctypes.c_void_p(out_v.data_ptr()), out_dtype, layout)
        return _launcher(fn, args, "air_kv_gather", (block_tables, seq_lens, out_offsets, out_k, out_v, stream))

    def copy_blocks(self, src, dst, stream=None):
        torch = _torch()
        n = src.shape[0]
        sp = _dev(src, torch.int32, "src", (n,))
        dp = _dev(dst, torch.int32, "dst", (n,))
        _lib.check(_lib.load().air_kv_copy_blocks(self.handle, _stream_ptr(stream), sp, dp, n),
                   "air_kv_copy_blocks")

    # -- host copies ------------------------------------------------------------

    def read_blocks(self, ids, stream=None):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((len(ids), self.block_bytes), np.uint8)
        _lib.check(_lib.load().air_kv_read_blocks(
            self.handle, _stream_ptr(stream) if stream is not None else None,
            ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(ids),
            out.ctypes.data_as(ctypes.c_void_p)), "air_kv_read_blocks")
        return out

    def write_blocks(self, ids, data, stream=None):
        ids = np.ascontiguousarray(ids, np.int32)
        data = np.ascontiguousarray(data, np.uint8).reshape(len(ids), self.block_bytes)
        _lib.check(_lib.load().air_kv_write_blocks(
            self.handle, _stream_ptr(stream) if stream is not None else None,
            ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(ids),
            data.ctypes.data_as(ctypes.c_void_p)), "air_kv_write_blocks")

    # ---- KvBlock wire format (src/pd_disagg.rs:39-83) ----------------------

    @property
    def wire_bytes(self):
        out = ctypes.c_size_t()
        _lib.check(_lib.load().air_kv_block_wire_bytes(self.handle, ctypes.byref(out)))
        return out.value

    def pack_blocks(self, ids, out=None, stream=None):
        """Wire data of blocks `ids` (int32 device tensor) as a uint8 device
        tensor [n, wire_bytes]: bf16 [block_size][n_kv_heads][head_dim][K|V]."""
        torch = _torch()
        _dev(ids, torch.int32, "ids")
        n = ids.numel()
        if out is None:
            out = torch.empty(n, self.wire_bytes, dtype=torch.uint8, device="cuda")
        _dev(out, torch.uint8, "out", (n, self.wire_bytes))
        _lib.check(_lib.load().air_kv_pack_blocks(self.handle, _stream_ptr(stream),
                                                  ctypes.c_void_p(ids.data_ptr()), n,
                                                  ctypes.c_void_p(out.data_ptr())), "air_kv_pack_blocks")
        return out

    def unpack_blocks(self, ids, wire, stream=None):
        torch = _torch()
        _dev(ids, torch.int32, "ids")
        n = ids.numel()
        _dev(wire, torch.uint8, "wire", (n, self.wire_bytes))
        _lib.check(_lib.load().air_kv_unpack_blocks(self.handle, _stream_ptr(stream),
                                                    ctypes.c_void_p(ids.data_ptr()), n,
                                                    ctypes.c_void_p(wire.data_ptr())), "air_kv_unpack_blocks")

    def pack_blocks_int8(self, ids, stream=None):
        """(codes int8 [n, wire_bytes / 2], scales f32 [n]) device tensors."""
        torch = _torch()
        _dev(ids, torch.int32, "ids")
        n = ids.numel()
        codes = torch.empty(n, self.wire_bytes // 2, dtype=torch.int8, device="cuda")
        scales = torch.empty(n, dtype=torch.float32, device="cuda")
        _lib.check(_lib.load().air_kv_pack_blocks_int8(self.handle, _stream_ptr(stream),
                                                       ctypes.c_void_p(ids.data_ptr()), n,
                                                       ctypes.c_void_p(codes.data_ptr()),
                                                       ctypes.c_void_p(scales.data_ptr())),
                   "air_kv_pack_blocks_int8")
        return codes, scales

    def split_blocks(self, raw):
        """Split read_blocks output into (k, v, k_scales, v_scales) arrays in
        the device layout [n][n_kv_heads][block_size][...]."""
        n = raw.shape[0]
        o0, o1 = self.slab_bytes, 2 * self.slab_bytes
        shp = (n, self.n_kv_heads, self.block_size, self.head_dim)
        npd = PAGE_NP_DTYPE[self.dtype]
        k = raw[:, :o0].copy().view(npd).reshape(shp)
        v = raw[:, o0:o1].copy().view(npd).reshape(shp)
        if not self.quantized:
            return k, v, None, None
        o2 = o1 + self.scale_slab_bytes
        sshp = shp[:3] + (self.head_dim // self.scale_group,)
        ks = raw[:, o1:o2].copy().view(np.float32).reshape(sshp)
        vs = raw[:, o2:].copy().view(np.float32).reshape(sshp)
        return k, v, ks, vs

    def snapshot(self):
        """Whole pool copied to host, in the device layout."""
        return self.split_blocks(self.read_blocks(np.arange(self.num_blocks, dtype=np.int32)))

    def error_count(self, reset=False, stream=None):
        out = ctypes.c_int64()
        _lib.check(_lib.load().air_kv_pool_error_count(
            self.handle, _stream_ptr(stream) if stream is not None else None, ctypes.byref(out),
            1 if reset else 0))
        return out.value


def wire_int8_quantize(wire, stream=None):
    """KvBlock::int8_quantize of every row of `wire` (uint8 device tensor
    [n_blocks, bytes] of bf16 data) -> (codes int8 [n_blocks, bytes / 2],
    scales f32 [n_blocks])."""
    torch = _torch()
    _dev(wire, torch.uint8, "wire")
    n, nbytes = wire.shape
    codes = torch.empty(n, nbytes // 2, dtype=torch.int8, device="cuda")
    scales = torch.empty(n, dtype=torch.float32, device="cuda")
    _lib.check(_lib.load().air_kv_wire_int8_quantize(_stream_ptr(stream), ctypes.c_void_p(wire.data_ptr()), n,
                                                     nbytes // 2, ctypes.c_void_p(codes.data_ptr()),
                                                     ctypes.c_void_p(scales.data_ptr())),
               "air_kv_wire_int8_quantize")
    return codes, scales
