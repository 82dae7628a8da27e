"""GPU parity at the full sizes of configs[2..4] (c3, c4, c5): the paged decode
against a plain torch float32 attention over the gathered cache, and the
configs[4] continuous-batching workflow at its full size with every step's
gather checked bit for bit against a torch page-index gather of the appended
rows.

The gather itself is pinned bit-exact to the oracle (test_gpu_append_gather,
the c1 digests); quantized caches are gathered dequantized (code * scale,
exactly the reference's dequantization), so the comparison measures the
attention kernel's error on the same cache (decision D3), not quantization
error.  Tolerances, relative to max |reference| per sequence: 2e-2 for int8 /
fp8 caches, 1e-3 for bf16 (the reference's flash_decode tolerance structure,
src/flash_decode.rs:232-275).  The reference attention is
softmax(q . K^T / sqrt(d)) . V per query head over kv head h / group
(src/ops.rs:514-568, src/chunked_attn.rs:240-243).
"""
import numpy as np
import pytest

import airkv
from airkv import workloads
from gpu_helpers import decode_pieces, log, torch_mod

pytestmark = pytest.mark.gpu


def _fill(pool, w, seed, outliers=None):
    """Append every batch of the workload with rows from a seeded device
    generator; returns nothing (rows are not kept: the gather reads them back)."""
    torch = torch_mod()
    cfg = w.cfg
    gen = workloads.kv_rows(10 ** 12, cfg.n_kv_heads, cfg.head_dim, seed=seed, device="cuda",
                            chunk_rows=1 << 15, outliers=outliers)
    for slots in w.batches:
        st = torch.from_numpy(slots).cuda()
        done = 0
        while done < len(slots):
            k, v = next(gen)
            n = min(len(slots) - done, k.shape[0])
            pool.append(k[:n].contiguous(), v[:n].contiguous(), st[done:done + n].contiguous())
            done += n


def _gathered(pool, tt, lt, lens, out_dtype):
    torch = torch_mod()
    per = lens.astype(np.int64) * pool.n_kv_heads * pool.head_dim
    offs = np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)
    tdt = torch.float32 if out_dtype == airkv.F32 else torch.bfloat16
    gk = torch.empty(int(per.sum()), dtype=tdt, device="cuda")
    gv = torch.empty_like(gk)
    pool.gather(tt, lt, torch.from_numpy(offs).cuda(), gk, gv, out_dtype=out_dtype)
    return gk, gv, offs


def _worst_rel_err(out, q, gk, gv, offs, lens, nkv, d):
    """max over sequences of max|out - ref| / max|ref|, ref in float32."""
    torch = torch_mod()
    torch.backends.cuda.matmul.allow_tf32 = False
    batch, nq, _ = q.shape
    g = nq // nkv
    worst = 0.0
    for b in range(batch):
        L = int(lens[b])
        if L == 0:
            continue
        K = gk[offs[b]:offs[b] + L * nkv * d].view(nkv, L, d).float()
        V = gv[offs[b]:offs[b] + L * nkv * d].view(nkv, L, d).float()
        qb = q[b].float().view(nkv, g, d)
        s = torch.matmul(qb, K.transpose(1, 2).contiguous()) / np.sqrt(float(d))
        p = torch.softmax(s, dim=-1)
        ref = torch.matmul(p, V).reshape(nq, d)
        worst = max(worst, (out[b].float() - ref).abs().max().item() / ref.abs().max().item())
    return worst


def _full_decode(name, lens, tol, seed, outliers=None):
    torch = torch_mod()
    cfg = workloads.CONFIGS[name]
    w = workloads.build_prefill_decode(cfg, lens, seed=seed, decode_steps=1)
    pool = airkv.KvPool(w.num_blocks, cfg.block_size, cfg.n_kv_heads, cfg.head_dim, cfg.dtype, cfg.scale_group)
    _fill(pool, w, seed + 1, outliers)
    tables, seq_lens = w.tables()
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(seq_lens).cuda()
    q = torch.randn(cfg.batch, cfg.n_q_heads, cfg.head_dim, device="cuda").to(torch.bfloat16)
    out = torch.empty(cfg.batch, cfg.n_q_heads, cfg.head_dim, device="cuda")
    ws = pool.new_workspace(cfg.n_q_heads, cfg.batch, tables.shape[1], cfg.max_splits)
    pool.paged_decode(q, tt, lt, out, max_splits=cfg.max_splits, workspace=ws)
    pieces = decode_pieces(ws, seq_lens)
    log(f"full {name}: pieces per sequence {pieces.min()}..{pieces.max()} (max_splits {cfg.max_splits})")
    assert pieces.max() <= cfg.max_splits
    gdt = airkv.F32 if cfg.dtype in (airkv.INT8, airkv.FP8) else airkv.BF16
    gk, gv, offs = _gathered(pool, tt, lt, seq_lens, gdt)
    worst = _worst_rel_err(out, q, gk, gv, offs, seq_lens, cfg.n_kv_heads, cfg.head_dim)
    log(f"full {name}: batch {cfg.batch}, {int(seq_lens.sum())} cached tokens, worst rel err {worst:.2e}")
    assert worst <= tol
    assert pool.error_count() == 0


def test_full_c3_int8_outliers_against_torch_fp32():
    """64 q / 8 kv heads, int8 Q8_0 pages (bs 16), batch 32 x
    context 8192 (+1 appended), 1% of channels x20 outliers."""
    log("full c3")
    outl = workloads.outlier_channels(8, 128, seed=3)
    _full_decode("c3", [8192] * 32, 2e-2, seed=31, outliers=outl)


def test_full_c4_fp8_long_context_against_torch_fp32():
    """fp8 E4M3 (reference encoding) pages, bs 32, batch 8 x
    contexts U[32768, 131072], split-K over up to 64 partitions."""
    log("full c4")
    _full_decode("c4", workloads.c4_lengths(8), 2e-2, seed=41)


def test_full_c5_bf16_against_torch_fp32():
    """configs[4]'s decode: 256 sequences, lognormal contexts (median 1024,
    clipped to [16, 32768]), bf16 pages, bs 32."""
    log("full c5")
    _full_decode("c5", workloads.c5_lengths(256), 1e-3, seed=51)


def test_full_c5_continuous_batching_workflow():
    """configs[4] as a workflow at full size: 256 sequences with lognormal
    target contexts (median 1024, clipped to [16, 32768]); each step appends,
    in one launch, 512-token prefill chunks for 8 sequences still prefilling
    and one token for the 248 others, then frees 13 sequences (5%) and starts
    13 new ones from the fragmented FIFO free list.  After every step every
    live sequence is gathered (bit-exact against a torch page-index gather of
    a bf16 mirror of every appended row) and decoded (within 1e-3 of torch
    float32)."""
    torch = torch_mod()
    NQ, NKV, D, BS, CHUNK, N_SEQ, STEPS = 32, 8, 128, 32, 512, 256, 4
    rng = np.random.default_rng(170)
    targets0 = workloads.c5_lengths(N_SEQ, seed=171)
    # the pool holds every sequence's target plus the new sequences' and the decode tokens
    cap = int(1.3 * (sum(targets0) + 13 * STEPS * 4096 + N_SEQ * STEPS) / BS) + N_SEQ
    mgr = airkv.SequenceManager(cap, BS, free_order=workloads.lcg_permutation(cap, 172))
    pool = airkv.KvPool(cap, BS, NKV, D, airkv.BF16)
    mirror_k = torch.zeros(cap * BS, NKV, D, dtype=torch.bfloat16, device="cuda")
    mirror_v = torch.zeros_like(mirror_k)
    g = torch.Generator(device="cuda")
    g.manual_seed(173)

    def append(slots_np):
        n = len(slots_np)
        k = torch.randn(n, NKV, D, generator=g, device="cuda")
        v = torch.randn(n, NKV, D, generator=g, device="cuda")
        st = torch.from_numpy(slots_np).cuda()
        pool.append(k, v, st)
        mirror_k[st] = k.to(torch.bfloat16)        # round to nearest even, as the pages
        mirror_v[st] = v.to(torch.bfloat16)

    seqs = [mgr.create_sequence() for _ in range(N_SEQ)]
    target = dict(zip(seqs, targets0))
    have = {s: 0 for s in seqs}
    # contexts exist before the measured steps: every sequence but eight is
    # prefilled; those eight take the first step's prefill chunks
    for s in seqs[: N_SEQ - 8]:
        slots = mgr.append_slots(s, target[s])
        have[s] = target[s]
        append(slots)
    new_targets = iter(workloads.c5_lengths(13 * STEPS, seed=174))
    for step in range(STEPS):
        slots, n_pref = [], 0
        for s in seqs:
            if have[s] < target[s]:
                if n_pref == 8:
                    continue                        # waits for a prefill slot
                n = min(CHUNK, target[s] - have[s])
                n_pref += 1
            else:
                n = 1
            slots.append(mgr.append_slots(s, n))
            have[s] += n
        slots = np.concatenate(slots)
        append(slots)
        live = [s for s in seqs if have[s] > 0]
        mb = max(-(-have[s] // BS) for s in live)
        tables, lens = mgr.export_tables(live, mb)
        tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
        gk, gv, offs = _gathered(pool, tt, lt, lens, airkv.BF16)
        # torch page-index gather of the mirror: slot of token t = table[t / bs] * bs + t % bs
        for b, s in enumerate(live):
            L = int(lens[b])
            pos = torch.arange(L, device="cuda")
            sl = tt[b, pos // BS].long() * BS + pos % BS
            want_k = mirror_k[sl].permute(1, 0, 2).reshape(-1)     # [head][t][d]
            want_v = mirror_v[sl].permute(1, 0, 2).reshape(-1)
            got_k = gk[offs[b]:offs[b] + L * NKV * D]
            got_v = gv[offs[b]:offs[b] + L * NKV * D]
            assert torch.equal(got_k.view(torch.int16), want_k.view(torch.int16)), (step, b)
            assert torch.equal(got_v.view(torch.int16), want_v.view(torch.int16)), (step, b)
        q = torch.randn(len(live), NQ, D, device="cuda").to(torch.bfloat16)
        out = torch.empty(len(live), NQ, D, device="cuda")
        pool.paged_decode(q, tt, lt, out)
        worst = _worst_rel_err(out, q, gk, gv, offs, lens, NKV, D)
        log(f"c5 step {step}: {len(slots)} tokens appended ({n_pref} prefill chunks), {len(live)} live, "
            f"{int(lens.sum())} cached, {mgr.allocator.num_free_blocks()} blocks free, decode err {worst:.2e}")
        n_decode = sum(1 for s in seqs if have[s] >= target[s] and s in live)
        assert n_pref <= 8 and len(slots) >= n_decode and worst <= 1e-3
        assert pool.error_count() == 0
        # 5% churn: free 13 sequences, start 13 new ones (their prefill follows)
        for s in rng.choice(seqs, size=13, replace=False).tolist():
            mgr.free_sequence(s)
            seqs.remove(s)
            del have[s], target[s]
            t = mgr.create_sequence()
            seqs.append(t)
            have[t] = 0
            target[t] = int(next(new_targets))
