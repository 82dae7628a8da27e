"""Seeded synthetic workloads of the benchmark configurations.

Each builder drives the product's SequenceManager exactly as a serving loop
would (create sequences, append tokens, export block tables) and produces
K/V rows, so the same construction serves the parity tests and bench.py.
Random block tables come from a seeded permutation of the free list
(Fisher-Yates over the reference's test LCG, src/flash_decode.rs:220-223), so
consecutive allocations land on scattered physical blocks.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from ._lib import BF16, F32, FP8, INT8
from .paged_attention import SequenceManager

_LCG_A = 6364136223846793005
_LCG_C = 1442695040888963407
_M64 = (1 << 64) - 1


def lcg_permutation(n: int, seed: int) -> np.ndarray:
    """Fisher-Yates shuffle of 0..n-1 driven by the reference LCG."""
    perm = list(range(n))
    s = seed & _M64
    for i in range(n - 1, 0, -1):
        s = (s * _LCG_A + _LCG_C) & _M64
        j = (s >> 33) % (i + 1)
        perm[i], perm[j] = perm[j], perm[i]
    return np.array(perm, np.uint32)


@dataclass
class Config:
    name: str
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    block_size: int
    dtype: int
    batch: int
    max_splits: int = 64
    scale_group: int = 32


CONFIGS = {
    # BASELINE.json configs[0..4]
    "c1": Config("kv_append_gather_f32", 8, 8, 64, 16, F32, 4),
    "c2": Config("paged_decode_bf16_llama3_8b", 32, 8, 128, 16, BF16, 64),
    "c3": Config("int8_kv_decode_llama3_70b", 64, 8, 128, 16, INT8, 32),
    "c4": Config("fp8_kv_long_context_decode", 64, 8, 128, 32, FP8, 8, max_splits=64),
    "c5": Config("mixed_continuous_batching_bf16", 32, 8, 128, 32, BF16, 256),
}


@dataclass
class Workload:
    cfg: Config
    num_blocks: int
    mgr: SequenceManager
    seqs: list
    free_order: np.ndarray
    # append batches: list of int64 slot arrays, and the row index range of
    # the K/V source each batch consumes
    batches: list = field(default_factory=list)
    n_rows: int = 0

    def tables(self, max_blocks=None):
        lens = [self.mgr.table(s).num_tokens for s in self.seqs]
        if max_blocks is None:
            max_blocks = max(1, max(math.ceil(x / self.cfg.block_size) for x in lens))
        return self.mgr.export_tables(self.seqs, max_blocks)


def _pool_blocks(total_tokens: int, n_seqs: int, bs: int, headroom: float) -> int:
    return int(math.ceil(headroom * (total_tokens + n_seqs * bs) / bs))


def build_prefill_decode(cfg: Config, ctx_lens, seed: int, headroom: float = 1.25,
                         decode_steps: int = 1, num_blocks: int | None = None) -> Workload:
    """Prefill every sequence to ctx_lens[i] tokens (one append batch per
    sequence), then `decode_steps` batches of one token per sequence."""
    ctx_lens = [int(x) for x in ctx_lens]
    total = sum(ctx_lens) + decode_steps * len(ctx_lens)
    nb = num_blocks or _pool_blocks(total, len(ctx_lens), cfg.block_size, headroom)
    order = lcg_permutation(nb, seed)
    mgr = SequenceManager(nb, cfg.block_size, free_order=order)
    seqs = [mgr.create_sequence() for _ in ctx_lens]
    w = Workload(cfg, nb, mgr, seqs, order)
    for s, L in zip(seqs, ctx_lens):
        if L:
            w.batches.append(mgr.append_slots(s, L))
    for _ in range(decode_steps):
        w.batches.append(np.concatenate([mgr.append_slots(s, 1) for s in seqs]))
    w.n_rows = sum(len(b) for b in w.batches)
    return w


def c1_workload(seed: int = 1) -> Workload:
    """prefill 37/128/200/511, then 16 steps of one token each,
    over a 256-block pool whose free list is a seeded permutation."""
    cfg = CONFIGS["c1"]
    return build_prefill_decode(cfg, [37, 128, 200, 511], seed, decode_steps=16, num_blocks=256)


def c2_lengths(batch: int = 64, lo: int = 512, hi: int = 4096, seed: int = 2):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=batch).tolist()


def c4_lengths(batch: int = 8, lo: int = 32768, hi: int = 131072, seed: int = 4):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=batch).tolist()


def c5_lengths(n: int = 256, median: int = 1024, sigma: float = 1.0, lo: int = 16, hi: int = 32768,
               seed: int = 5):
    rng = np.random.default_rng(seed)
    x = np.exp(rng.normal(math.log(median), sigma, size=n))
    return np.clip(np.round(x), lo, hi).astype(np.int64).tolist()


def outlier_channels(n_kv_heads: int, head_dim: int, frac: float = 0.01, seed: int = 3):
    """round(1% of n_kv*d) (kv_head, dim) channels scaled x20,
    the same channels for K and V."""
    n = int(round(frac * n_kv_heads * head_dim))
    rng = np.random.default_rng(seed)
    flat = rng.choice(n_kv_heads * head_dim, size=n, replace=False)
    return [(int(f // head_dim), int(f % head_dim)) for f in flat]


def kv_rows(n_rows: int, n_kv_heads: int, head_dim: int, seed: int, outliers=None,
            device=None, chunk_rows: int = 1 << 15):
    """Generator of (k, v) f32 chunks ~ N(0,1), [rows][n_kv][d], seeded; on
    `device` (a torch device) when given, else numpy."""
    if device is None:
        rng = np.random.default_rng(seed)
        done = 0
        while done < n_rows:
            n = min(chunk_rows, n_rows - done)
            k = rng.standard_normal((n, n_kv_heads, head_dim), dtype=np.float32)
            v = rng.standard_normal((n, n_kv_heads, head_dim), dtype=np.float32)
            if outliers:
                for h, d in outliers:
                    k[:, h, d] *= 20.0
                    v[:, h, d] *= 20.0
            yield k, v
            done += n
        return
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    done = 0
    while done < n_rows:
        n = min(chunk_rows, n_rows - done)
        k = torch.randn((n, n_kv_heads, head_dim), generator=g, device=device, dtype=torch.float32)
        v = torch.randn((n, n_kv_heads, head_dim), generator=g, device=device, dtype=torch.float32)
        if outliers:
            for h, d in outliers:
                k[:, h, d] *= 20.0
                v[:, h, d] *= 20.0
        yield k, v
        done += n
