#!/usr/bin/env python3
"""Benchmark of the paged KV-cache hot path on one MI355X.

Workload: Llama-3-8B decode shape, bf16 KV pages,
32 q / 8 kv heads, head_dim 128, block_size 16, batch 64, contexts
U[512, 4096], block tables over a shuffled pool of 1.25x the tokens.  One
step = append one new token per sequence (reshape-and-cache of f32 K/V) then
split-K paged decode attention over every cached token.  All inputs are
resident in HBM before timing starts.

Prints one JSON line: whole-step HBM throughput (`value`, GB/s of
algorithmic bytes), the decode call's roofline fraction (HIP events on the
launch stream; HBM traffic from the committed rocprofv3 counter runs),
gather / large-append bandwidths, decode at the c3 / c4 / c5 configs, paged
prefill at the c5 chunk geometry (TFLOP/s), warm-tier block compression
(GB/s), and the CPU oracle timed on the same workload on this host (all cores
and one core).
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "air.rs_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_HBM_GBPS = 8000.0   # MI355X HBM3E spec
PEAK_F32_TFLOPS = 157.3  # MI355X published fp32 peak
# rocprofv3 FETCH_SIZE + WRITE_SIZE of the decode call on this workload, scaled
# by the counters' reading for a 1 GiB copy (the summary lists the commands)
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "paged_decode_c2.md")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--max-splits", type=int, default=64)
    ap.add_argument("--kernel-iters", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-decode", action="store_true",
                    help="skip the gather / append bandwidth legs (for profiling runs)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the c3 / c4 / c5 decode legs")
    ap.add_argument("--legs", default="all",
                    help="comma list of the legs after the c2 step and decode to run (for profiling runs): "
                         "gather_append, ceilings, configs, quant_append, c5_step, prefill, compress, blocks; "
                         "default all")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def profiled_traffic():
    """HBM bytes per decode call measured by the committed rocprofv3 counter
    runs of this same command (None when the summary is absent)."""
    import re
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", text)
    return int(m.group(1)) if m else None


def timed_loop(torch, fn, iters, lead_sleep=True):
    """Average GPU time per launch of fn() over `iters` back-to-back launches,
    measured with events on the current stream; a sleep kernel first lets the
    host queue every launch before the first one starts."""
    torch.cuda.synchronize()
    if lead_sleep:
        torch.cuda._sleep(20_000_000)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters   # ms


def per_call_us(torch, fn, iters=100, warmup=10):
    """(p10, p50, p90) in us of single launches of fn(): events recorded
    between back-to-back launches (a sleep kernel first lets the host queue
    them all), after `warmup` untimed launches."""
    import numpy as np
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(iters + 1)]
    torch.cuda._sleep(20_000_000)
    ev[0].record()
    for i in range(iters):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    d = np.array([ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(iters)])
    return tuple(round(float(x), 2) for x in np.percentile(d, [10, 50, 90]))


def twin_pool(torch, pool):
    """A second pool of the same geometry holding the same bytes (device to
    device copy of pages and scales), so timed calls can alternate between
    two copies: no call then re-reads pages the previous call left in the
    256 MB MALL."""
    import ctypes

    import airkv
    twin = airkv.KvPool(pool.num_blocks, pool.block_size, pool.n_kv_heads, pool.head_dim, pool.dtype,
                        pool.scale_group)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    slab = pool.num_blocks * pool.slab_bytes
    sc = pool.num_blocks * pool.scale_slab_bytes
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, n in enumerate((slab, slab, sc, sc)):
        if n:
            rc = hip.hipMemcpyAsync(ctypes.c_void_p(twin.device_ptrs[i]), ctypes.c_void_p(pool.device_ptrs[i]),
                                    n, 3, stream)     # hipMemcpyDeviceToDevice
            assert rc == 0, f"hipMemcpyAsync failed ({rc})"
    torch.cuda.synchronize()
    return twin


def alternating(fns):
    """One call per invocation, cycling through fns (one per pool copy)."""
    state = [0]

    def call():
        fns[state[0]]()
        state[0] = (state[0] + 1) % len(fns)
    return call


def ceilings_leg(torch, iters=20):
    """HBM ceilings of this GPU, measured in this run with the bench-only
    kernels of air.rs_amd/csrc/bench/ceilings.hip on 1 GiB buffers (2 GiB for
    the page pools): contiguous read, contiguous write, copy (1 byte written
    per byte read), mix21 (2 bytes read per byte written), and page_read
    (4 KB K and V pages in a shuffled order, one wave per page), and
    page_copy (half of those pages copied to consecutive 4 KB slots: the
    gather's pattern) and page_mix21 (a quarter of them written from 8 KB
    of contiguous rows each: the append's pattern), page_read2k (2 KB pages
    in a shuffled order: the int8 decode's per-head run at block size 16)
    and block_read2k (the same pages, eight consecutive waves reading the
    eight pieces of one shuffled 16 KB block), page_read2k_halflines
    (page_read2k with each load instruction reading half of every line it
    touches, as the 1-byte decode's MFMA operand layout would if loaded
    directly; the variant field says which cache policy was faster).  Copy, mix21 and write
    also run with 32 to 256 bytes per thread, as persistent grid-stride
    loops (copy, mix21) and as the runtime's device copy; `*_best` is the
    fastest form.  Each pattern runs with plain and non-temporal loads /
    stores; the faster is kept, with its variant."""
    import ctypes

    import numpy as np
    lib = ctypes.CDLL(os.path.join(ROOT, "air.rs_amd", "airkv", "libairkv_ceilings.so"))
    lib.air_ceiling_launch.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                       ctypes.c_void_p]
    nbytes = 1 << 30
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    a.view(torch.int32).random_()
    b.view(torch.int32).random_()
    sink = torch.zeros(64, dtype=torch.int32, device="cuda")
    pages = torch.from_numpy(np.random.default_rng(13).permutation(nbytes // 4096).astype(np.int32)).cuda()
    # page_copy: half of each pool's pages (shuffled) into a 1 GiB output
    half = pages[: nbytes // 8192].contiguous()
    # page_mix21: a quarter of each pool's pages written from 1 GiB of rows
    quarter = pages[: nbytes // 16384].contiguous()
    # 2 KB pages (the int8 decode's per-head run at block size 16), and 16 KB
    # blocks whose eight 2 KB pieces consecutive waves read
    pages2k = torch.from_numpy(np.random.default_rng(14).permutation(nbytes // 2048).astype(np.int32)).cuda()
    blocks16k = torch.from_numpy(np.random.default_rng(15).permutation(nbytes // 16384).astype(np.int32)).cuda()
    pc_out = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    kinds = {  # name: (kind, bytes moved per launch, (load nt options), (store nt options), n_pages)
        "read": (0, nbytes, (0, 1), (0,), 0),
        "write": (1, nbytes, (0,), (0, 1), 0),
        "copy": (2, 2 * nbytes, (0, 1), (0, 1), 0),
        "mix21": (3, nbytes + nbytes // 2, (0, 1), (0, 1), 0),
        "page_read": (4, 2 * nbytes, (0, 1), (0,), nbytes // 4096),
        "page_copy": (5, 2 * nbytes, (0, 1), (0, 1), nbytes // 8192),
        "page_mix21": (6, nbytes // 2 * 3, (0, 1), (0, 1), nbytes // 16384),
        "copy_persist128": (7, 2 * nbytes, (0, 1), (0, 1), 0),
        "copy_persist256": (8, 2 * nbytes, (0, 1), (0, 1), 0),
        "mix21_persist128": (9, nbytes + nbytes // 2, (0, 1), (0, 1), 0),
        "mix21_persist256": (10, nbytes + nbytes // 2, (0, 1), (0, 1), 0),
        "copy_w32": (11, 2 * nbytes, (0, 1), (0, 1), 0),
        "copy_w128": (12, 2 * nbytes, (0, 1), (0, 1), 0),
        "copy_w256": (13, 2 * nbytes, (0, 1), (0, 1), 0),
        "mix21_w128": (14, nbytes + nbytes // 2, (0, 1), (0, 1), 0),
        "write_w32": (15, nbytes, (0,), (0, 1), 0),
        "write_w128": (16, nbytes, (0,), (0, 1), 0),
        "page_read2k": (17, 2 * nbytes, (0, 1), (0,), nbytes // 2048),
        "block_read2k": (18, 2 * nbytes, (0, 1), (0,), nbytes // 16384),
        "page_read2k_halflines": (19, 2 * nbytes, (0, 1), (0,), nbytes // 2048),
    }
    out = {}
    for name, (kind, moved, lds, sts, npg) in kinds.items():
        best = None
        for ntl in lds:
            for nts in sts:
                def fn(kind=kind, ntl=ntl, nts=nts, npg=npg):
                    if kind == 5:      # K / V pools a, b -> pc_out
                        args = (P(a), P(b), P(half), P(pc_out))
                    elif kind == 6:    # rows in pc_out -> K / V pools a, b
                        args = (P(pc_out), P(a), P(quarter), P(b))
                    elif kind in (17, 18, 19):
                        args = (P(a), P(b), P(blocks16k if kind == 18 else pages2k), P(sink))
                    else:
                        args = (P(a), P(b), P(pages) if npg else None, P(sink))
                    rc = lib.air_ceiling_launch(kind, ntl, nts, args[0], args[1], nbytes, args[2], npg, args[3],
                                                stream)
                    assert rc == 0, f"ceiling launch {kind} failed ({rc})"
                fn()
                ms = timed_loop(torch, fn, iters)
                gbps = moved / (ms * 1e-3) / 1e9
                parts = []
                if len(lds) > 1:
                    parts.append(("nt" if ntl else "plain") + " loads")
                if len(sts) > 1:
                    parts.append(("nt" if nts else "plain") + " stores")
                variant = ", ".join(parts)
                if best is None or gbps > best["gbps"]:
                    best = {"gbps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4), "variant": variant}
        out[name] = best
    # the runtime's own device-to-device copy of 1 GiB
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]

    def memcpy():
        rc = hip.hipMemcpyAsync(P(b), P(a), nbytes, 3, stream)     # hipMemcpyDeviceToDevice
        assert rc == 0, f"hipMemcpyAsync failed ({rc})"
    memcpy()
    ms = timed_loop(torch, memcpy, iters)
    gbps = 2 * nbytes / (ms * 1e-3) / 1e9
    out["memcpy_d2d"] = {"gbps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4), "variant": "hipMemcpyAsync"}
    # best of each pattern over its one-shot, persistent and runtime forms
    out["copy_best"] = max((out[k] | {"form": k} for k in ("copy", "copy_w32", "copy_w128", "copy_w256",
                                                           "copy_persist128", "copy_persist256", "memcpy_d2d")),
                           key=lambda r: r["gbps"])
    out["mix21_best"] = max((out[k] | {"form": k} for k in ("mix21", "mix21_w128", "mix21_persist128",
                                                            "mix21_persist256")), key=lambda r: r["gbps"])
    out["write_best"] = max((out[k] | {"form": k} for k in ("write", "write_w32", "write_w128")),
                            key=lambda r: r["gbps"])
    del a, b, pc_out
    return out


def cpu_info():
    """(threads to use, description): the process's CPU share on this host.
    os.cpu_count() counts every CPU of the machine; the affinity mask and
    OMP_NUM_THREADS say what this process may use (16 on the GPU boxes)."""
    ncpu = os.cpu_count() or 1
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = ncpu
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = max(1, min(aff, omp) if omp > 0 else aff)
    # the first processor's fields: a bare "AMD EPYC" model name still names
    # its generation by family / model / stepping (family 25: Zen 3 / Zen 4,
    # family 26: Zen 5), and the flags say whether AVX-512 is there
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break
            key, _, val = line.partition(":")
            fields.setdefault(key.strip(), val.strip())
    except OSError:
        pass
    flags = fields.get("flags", "").split()
    return threads, {"cpu_model": fields.get("model name", "unknown"), "cpu_family": fields.get("cpu family"),
                     "cpu_model_id": fields.get("model"), "cpu_stepping": fields.get("stepping"),
                     "cpu_mhz": fields.get("cpu MHz"), "avx512": "avx512f" in flags,
                     "host_cpus": ncpu, "affinity_cpus": aff, "omp_num_threads": omp or None}


def cpu_baseline(pool, w, tables, lens, q_f32, budget_s, decode_bytes_of):
    """The oracle's paged decode (gather + flash_decode with chunk 64 per query
    head, src/flash_decode.rs:153-173) on whole sequences of the same workload,
    on this host's cores: first on one thread (every sequence, or about
    budget_s of work), then on every CPU this process may use (its affinity
    mask, capped by OMP_NUM_THREADS: the GPU box's share of the host) over
    every sequence (ctypes releases the GIL, so the C oracle calls run in
    parallel).  GB/s counts the same algorithmic bytes as the GPU figure."""
    import concurrent.futures

    import numpy as np

    import oracle
    cfg = w.cfg
    k, v, _, _ = pool.snapshot()
    host = oracle.HostPool(pool.num_blocks, cfg.block_size, cfg.n_kv_heads, cfg.head_dim, oracle.BF16)
    host.k[:], host.v[:] = k, v
    del k, v

    def one(b):
        host.paged_decode(q_f32[b:b + 1], tables[b:b + 1], lens[b:b + 1], chunk=64)

    batch = len(lens)
    done, t0 = 0, time.perf_counter()
    for b in range(batch):
        one(b)
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    t1 = time.perf_counter() - t0
    v1 = decode_bytes_of(lens[:done], done) / t1 / 1e9
    threads, hostinfo = cpu_info()
    with concurrent.futures.ThreadPoolExecutor(threads) as ex:
        t0 = time.perf_counter()
        list(ex.map(one, range(batch)))
        tn = time.perf_counter() - t0
    vn = decode_bytes_of(lens, batch) / tn / 1e9
    return {"value": vn, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"all {batch} sequences of the final state ({int(np.sum(lens))} cached tokens, "
                      f"32 q heads each), oracle gather + flash_decode chunk 64 per query head, "
                      f"{threads} threads over sequences: {tn:.2f} s; one thread: {done} sequences "
                      f"in {t1:.2f} s",
            "value_1core": v1, "seq_per_s": batch / tn, **hostinfo}


def config_decode(torch, name, iters=20):
    """Decode bandwidth at another BASELINE config's full size (c3 int8, c4
    fp8, c5 bf16): pool filled by the append kernel, then `iters` timed
    decode calls.  Reported beside the c2 line, not as `value`."""
    import numpy as np

    import airkv
    from airkv import workloads
    cfg = workloads.CONFIGS[name]
    lens0 = {"c3": lambda: [8192] * cfg.batch, "c4": lambda: workloads.c4_lengths(cfg.batch),
             "c5": lambda: workloads.c5_lengths(cfg.batch)}[name]()
    w = workloads.build_prefill_decode(cfg, lens0, seed=3, decode_steps=1)
    pool = airkv.KvPool(w.num_blocks, cfg.block_size, cfg.n_kv_heads, cfg.head_dim, cfg.dtype)
    outl = workloads.outlier_channels(cfg.n_kv_heads, cfg.head_dim, seed=3) if name == "c3" else None
    gen = workloads.kv_rows(10 ** 12, cfg.n_kv_heads, cfg.head_dim, seed=5, device="cuda",
                            chunk_rows=32768, outliers=outl)
    for slots in w.batches:
        st = torch.from_numpy(slots).cuda()
        done = 0
        while done < len(slots):
            k, v = next(gen)
            n = min(len(slots) - done, k.shape[0])
            pool.append(k[:n].contiguous(), v[:n].contiguous(), st[done:done + n].contiguous())
            done += n
    tables, lens = w.tables()
    tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
    q = torch.randn(cfg.batch, cfg.n_q_heads, cfg.head_dim, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(q)
    ws = pool.new_workspace(cfg.n_q_heads, cfg.batch, tables.shape[1], cfg.max_splits)
    twin = twin_pool(torch, pool)
    fn = alternating([p.bind_decode(q, tt, lt, out, ws, max_splits=cfg.max_splits) for p in (pool, twin)])
    fn()
    ms = timed_loop(torch, fn, iters)
    eb = {airkv.BF16: 2, airkv.INT8: 1, airkv.FP8: 1}[cfg.dtype]
    per_tok = cfg.n_kv_heads * cfg.head_dim * 2 * eb
    if cfg.dtype in (airkv.INT8, airkv.FP8):
        per_tok += cfg.n_kv_heads * (cfg.head_dim // cfg.scale_group) * 4 * 2
    tok = int(lens.astype(np.int64).sum())
    pages = int(((lens + cfg.block_size - 1) // cfg.block_size).sum())
    nbytes = tok * per_tok + 4 * pages + cfg.batch * cfg.n_q_heads * cfg.head_dim * 4
    res = {"decode_gbps": round(nbytes / (ms * 1e-3) / 1e9, 1), "decode_us": round(ms * 1e3, 1),
           "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4), "cached_tokens": tok,
           "batch": cfg.batch, "kv_dtype": {airkv.BF16: "bf16", airkv.INT8: "int8", airkv.FP8: "fp8"}[cfg.dtype],
           "block_size": cfg.block_size, "n_q_heads": cfg.n_q_heads}
    # the decode step as one launch (air_paged_decode_append: each
    # sequence's new K / V row -- quantized on 1-byte pages -- written by the
    # wave that attends over it) and as two calls (append, then decode); the
    # step rewrites each sequence's last token, so every call moves the same
    # bytes
    kn = torch.randn(cfg.batch, cfg.n_kv_heads, cfg.head_dim, device="cuda")
    vn = torch.randn_like(kn)
    last = (lens.astype(np.int64) - 1)
    step_slots = torch.from_numpy(tables[np.arange(cfg.batch), last // cfg.block_size].astype(np.int64)
                                  * cfg.block_size + last % cfg.block_size).cuda()
    fused = alternating([p.bind_decode_append(q, kn, vn, tt, lt, out, ws, max_splits=cfg.max_splits)
                         for p in (pool, twin)])
    fused()
    ms_f = timed_loop(torch, fused, iters)
    apps = [p.bind_append(kn, vn, step_slots) for p in (pool, twin)]
    decs = [p.bind_decode(q, tt, lt, out, ws, max_splits=cfg.max_splits) for p in (pool, twin)]
    two = alternating([(lambda a=a, d=d: (a(), d())) for a, d in zip(apps, decs)])
    two()
    ms_2 = timed_loop(torch, two, iters)
    app_bytes = cfg.batch * (cfg.n_kv_heads * cfg.head_dim * 2 * 4 + per_tok)   # f32 rows in, page row out
    step_bytes = nbytes + app_bytes
    res["step_fused"] = {"us": round(ms_f * 1e3, 1), "gbps": round(step_bytes / (ms_f * 1e-3) / 1e9, 1),
                         "frac": round(step_bytes / (ms_f * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
    res["step_two_call"] = {"us": round(ms_2 * 1e3, 1),
                            "gbps": round((step_bytes + 8 * cfg.batch) / (ms_2 * 1e-3) / 1e9, 1)}
    if cfg.dtype in (airkv.INT8, airkv.FP8):
        # the dequantizing gather of every sequence to contiguous f32
        # [head][len][dim] (code * scale, src/kv_cache.rs:78-92,
        # src/fp8.rs:263-264): codes and scales read, f32 written
        per = lens.astype(np.int64) * cfg.n_kv_heads * cfg.head_dim
        offs = torch.from_numpy(np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)).cuda()
        gk = torch.empty(int(per.sum()), dtype=torch.float32, device="cuda")
        gv = torch.empty_like(gk)
        gather = alternating([p.bind_gather(tt, lt, offs, gk, gv, out_dtype=airkv.F32) for p in (pool, twin)])
        gather()
        ms_g = timed_loop(torch, gather, 10)
        g_bytes = tok * (per_tok + cfg.n_kv_heads * cfg.head_dim * 2 * 4) + 4 * pages
        res["gather_f32"] = {"gbps": round(g_bytes / (ms_g * 1e-3) / 1e9, 1), "us": round(ms_g * 1e3, 1),
                             "frac": round(g_bytes / (ms_g * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                             "algorithmic_bytes": int(g_bytes)}
        del gk, gv
    assert pool.error_count() == 0 and twin.error_count() == 0
    twin.close()
    pool.close()
    return res


def prefill_leg(torch, iters=20, prefix=None, int8_70b=False):
    """Paged prefill at the configs[4] geometry: 512-token chunks (32 q / 8 kv
    heads, d 128, bs 32, bf16 pages and queries) over given prefixes (default:
    eight drawn from the lognormal context mix); with int8_70b, at the
    configs[2] geometry instead (64 q / 8 kv heads, bs 16, int8 Q8_0 pages
    with 1% outlier channels x20).  Algorithmic flops count QK^T and PV over
    the causal keys only: 4 * d per (query row, head, key).  The launch gets
    the key-split workspace the library asks for (none for the c5 chunk mix;
    one for a single long sequence)."""
    import numpy as np

    import airkv
    from airkv import workloads
    chunk = 512
    if prefix is None:
        prefix = workloads.c5_lengths(8, seed=5)
    if int8_70b:
        cfg = workloads.Config("c3-prefill", 64, 8, 128, 16, airkv.INT8, len(prefix))
    else:
        cfg = workloads.Config("c5-prefill", 32, 8, 128, 32, airkv.BF16, len(prefix))
    w = workloads.build_prefill_decode(cfg, [p + chunk for p in prefix], seed=5, decode_steps=0)
    pool = airkv.KvPool(w.num_blocks, cfg.block_size, cfg.n_kv_heads, cfg.head_dim, cfg.dtype)
    gen = workloads.kv_rows(10 ** 12, cfg.n_kv_heads, cfg.head_dim, seed=6, device="cuda", chunk_rows=32768,
                            outliers=workloads.outlier_channels(cfg.n_kv_heads, cfg.head_dim, seed=3) if int8_70b
                            else None)
    for slots in w.batches:
        st = torch.from_numpy(slots).cuda()
        done = 0
        while done < len(slots):
            k, v = next(gen)
            n = min(len(slots) - done, k.shape[0])
            pool.append(k[:n].contiguous(), v[:n].contiguous(), st[done:done + n].contiguous())
            done += n
    tables, lens = w.tables()
    cu = torch.arange(cfg.batch + 1, dtype=torch.int32, device="cuda") * chunk
    q = torch.randn(cfg.batch * chunk, cfg.n_q_heads, cfg.head_dim, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(q)
    fn = pool.bind_prefill(q, cu, torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda(), out,
                           max_q_len=chunk)
    ws = fn.workspace
    ms = timed_loop(torch, fn, iters)
    keys = sum(sum(int(L) - chunk + r + 1 for r in range(chunk)) for L in lens)
    flops = keys * cfg.n_q_heads * 4 * cfg.head_dim
    tf = flops / (ms * 1e-3) / 1e12
    assert pool.error_count() == 0
    pool.close()
    return {"tflops": round(tf, 1), "us": round(ms * 1e3, 1), "frac_of_bf16_mfma": round(tf / 2500.0, 4),
            "kv_dtype": "int8" if int8_70b else "bf16", "n_q_heads": cfg.n_q_heads, "block_size": cfg.block_size,
            "prefix_tokens": [int(x) for x in prefix], "chunk": chunk, "q_rows": cfg.batch * chunk,
            "flops": int(flops), "key_split_workspace_bytes": 0 if ws is None else int(ws.numel())}


def compress_leg(torch, iters=10):
    """Warm-tier compression of 8192 bf16 blocks (bs 16, 8 kv heads, d 128:
    1M K rows and 1M V rows) with air_kv_compress_blocks.  Algorithmic bytes:
    the pages read (512 B per K and V row) plus the outputs written (16 B bits
    + 8 B per key row, 128 B codes + 8 B per value row) and 4 B per id."""
    import numpy as np

    import airkv
    from airkv import kv_compress as kc
    nb = 8192
    pool = airkv.KvPool(nb + 64, 16, 8, 128, airkv.BF16)
    k = torch.randn(nb * 16, 8, 128, device="cuda")
    slots = torch.arange(nb * 16, dtype=torch.int64, device="cuda")
    pool.append(k, torch.randn_like(k), slots)
    del k
    ids = torch.from_numpy(np.random.default_rng(7).permutation(nb).astype(np.int32)).cuda()
    kc.compress_blocks(pool, ids)
    outs = kc.compress_blocks(pool, ids)
    L = airkv.load()
    import ctypes
    args = (pool.handle, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), ctypes.c_void_p(ids.data_ptr()),
            nb, *[ctypes.c_void_p(outs[n].data_ptr()) for n in
                  ("key_bits", "key_magnitude", "key_mean", "value_codes", "value_scale", "value_min")])
    ms = timed_loop(torch, lambda: L.air_kv_compress_blocks(*args), iters)
    rows = nb * 16 * 8
    nbytes = rows * (2 * 256 + 16 + 8 + 128 + 8) + 4 * nb
    res = {"gbps": round(nbytes / (ms * 1e-3) / 1e9, 1), "us": round(ms * 1e3, 1), "rows": rows,
           "blocks": nb, "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
    # QJL (src/kv_compress.rs:908-975) at the reference's QJL_PROJ_DIM = 64: the
    # sign projection of the same 1M key rows (m dot products of d products
    # and sums each, contraction off as the reference folds them), then one
    # query's Hamming scores against every compressed key
    m = 64
    proj = torch.randn(m * 128, device="cuda") / 128 ** 0.5
    qbits, qmag = kc.qjl_compress_blocks(pool, ids, proj, m)
    ms_q = timed_loop(torch, lambda: kc.qjl_compress_blocks(pool, ids, proj, m), iters)
    flops = rows * m * 128 * 2
    res["qjl_compress"] = {"us": round(ms_q * 1e3, 1), "rows": rows, "proj_dim": m,
                           "tflops_f32": round(flops / (ms_q * 1e-3) / 1e12, 1),
                           "frac_of_f32_peak": round(flops / (ms_q * 1e-3) / 1e12 / PEAK_F32_TFLOPS, 4),
                           "gbps": round(rows * (256 + 8 + 4) / (ms_q * 1e-3) / 1e9, 1)}
    qb = qbits[0].clone()
    ms_s = timed_loop(torch, lambda: kc.qjl_scores(qbits, qmag, qb, 1.0, m), iters)
    sbytes = rows * (8 + 4 + 4 + 4)
    res["qjl_scores"] = {"us": round(ms_s * 1e3, 1), "keys": rows,
                         "gbps": round(sbytes / (ms_s * 1e-3) / 1e9, 1),
                         "frac": round(sbytes / (ms_s * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
    assert pool.error_count() == 0
    pool.close()
    return res


def blocks_leg(torch, iters=20):
    """Page-granular block work (the f1 CoW / swap hooks and the f2 KvBlock
    wire format) on a bf16 pool (bs 16, 8 kv heads, d 128: 64 KB of K+V per
    block), 4096 shuffled blocks per call, device-resident:
      copy_blocks      read + write of every block (CoW copy);
      pack_blocks      pages read, [bs][heads][d][K|V] bf16 wire written;
      unpack_blocks    wire read, pages written;
      pack_blocks_int8 pages read, int8 wire codes + one f32 scale written.
    Two disjoint block sets (and wire buffers) alternate between calls, so no
    call finds its 512 MB in the 256 MB MALL.  The host swap copies
    (read_blocks / write_blocks: synchronous, pageable host memory) are timed
    on 1024 blocks with the wall clock; their rate is PCIe-inclusive and is
    reported beside, never as a device figure."""
    import numpy as np

    import airkv
    n = 4096
    nb = 4 * n + 64
    pool = airkv.KvPool(nb, 16, 8, 128, airkv.BF16)
    for c0 in range(0, nb * 16, 1 << 17):
        c1 = min(nb * 16, c0 + (1 << 17))
        k = torch.randn(c1 - c0, 8, 128, device="cuda")
        pool.append(k, torch.randn_like(k), torch.arange(c0, c1, dtype=torch.int64, device="cuda"))
    del k
    perm = np.random.default_rng(11).permutation(nb).astype(np.int32)
    sets = [(torch.from_numpy(perm[j * 2 * n:j * 2 * n + n]).cuda(),
             torch.from_numpy(perm[j * 2 * n + n:(j + 1) * 2 * n]).cuda()) for j in range(2)]
    blk = pool.block_bytes
    wires = [pool.pack_blocks(src) for src, _ in sets]
    res = {"blocks": n, "block_bytes": blk}
    flip = [0]

    def rate(name, fn, nbytes):
        def call():
            fn(flip[0])
            flip[0] ^= 1
        call()
        ms = timed_loop(torch, call, iters)
        res[name] = {"gbps": round(nbytes / (ms * 1e-3) / 1e9, 1), "us": round(ms * 1e3, 1),
                     "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}

    rate("copy_blocks", lambda j: pool.copy_blocks(*sets[j]), 2 * n * blk + 8 * n)
    rate("pack_blocks", lambda j: pool.pack_blocks(sets[j][0], out=wires[j]), 2 * n * blk + 4 * n)
    rate("unpack_blocks", lambda j: pool.unpack_blocks(sets[j][1], wires[j]), 2 * n * blk + 4 * n)
    rate("pack_blocks_int8", lambda j: pool.pack_blocks_int8(sets[j][0]), n * blk + n * blk // 2 + 8 * n)
    ids = perm[:1024]
    host = pool.read_blocks(ids)
    for name, fn in (("host_read_blocks", lambda: pool.read_blocks(ids)),
                     ("host_write_blocks", lambda: pool.write_blocks(ids, host))):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / 3
        res[name] = {"gbps_pcie_inclusive": round(len(ids) * blk / dt / 1e9, 2), "ms": round(dt * 1e3, 2),
                     "blocks": len(ids), "host_memory": "pageable"}
    assert pool.error_count() == 0
    pool.close()
    return res


QUANT_APPEND_ROWS = 32768


def quant_append_workload(name):
    """The slots of two 32768-row append launches at a 1-byte config's
    geometry (c3: int8 Q8_0, bs 16; c4: fp8, bs 32): eight sequences of
    8192 tokens over a pool of 1.25x the tokens with a shuffled free list, so
    each launch writes four whole sequences' pages scattered over the pool."""
    import numpy as np

    from airkv import workloads
    cfg = workloads.CONFIGS[name]
    w = workloads.build_prefill_decode(cfg, [8192] * 8, seed=61 if name == "c3" else 71, decode_steps=0)
    allslots = np.concatenate(w.batches)
    n = QUANT_APPEND_ROWS
    return cfg, w, [allslots[j * n:(j + 1) * n] for j in range(2)]


def quant_append_bytes(cfg, n_rows):
    """f32 K and V rows read, 1-byte codes and f32 group scales written, int64 slots read."""
    row = cfg.n_kv_heads * cfg.head_dim
    return n_rows * (row * 2 * (4 + 1) + cfg.n_kv_heads * (cfg.head_dim // cfg.scale_group) * 4 * 2 + 8)


def quant_append_leg(torch, name, iters=20):
    """Quantize-on-append at full size for c3 (int8 Q8_0, 1% outlier channels
    x20) and c4 (fp8, reference E4M3 with the absmax/448 scale): 32768 f32
    K/V rows per launch (the c2 leg's size), two source / slot sets used
    alternately (2 x 268 MB of rows exceed the 256 MB MALL)."""
    import airkv
    from airkv import workloads
    cfg, w, sets = quant_append_workload(name)
    pool = airkv.KvPool(w.num_blocks, cfg.block_size, cfg.n_kv_heads, cfg.head_dim, cfg.dtype, cfg.scale_group)
    outl = workloads.outlier_channels(cfg.n_kv_heads, cfg.head_dim, seed=3) if name == "c3" else None
    gen = workloads.kv_rows(10 ** 12, cfg.n_kv_heads, cfg.head_dim, seed=62, device="cuda",
                            chunk_rows=QUANT_APPEND_ROWS, outliers=outl)
    fns = []
    for s in sets:
        k, v = next(gen)
        fns.append(pool.bind_append(k, v, torch.from_numpy(s).cuda()))
    call = alternating(fns)
    call()
    ms = timed_loop(torch, call, iters)
    nbytes = quant_append_bytes(cfg, QUANT_APPEND_ROWS)
    assert pool.error_count() == 0
    pool.close()
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"gbps": round(gbps, 1), "us": round(ms * 1e3, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4),
            "rows": QUANT_APPEND_ROWS, "kv_dtype": {airkv.INT8: "int8", airkv.FP8: "fp8"}[cfg.dtype],
            "block_size": cfg.block_size, "algorithmic_bytes": int(nbytes)}


def c5_step_leg(torch, warmup=2, steps=6):
    """configs[4] as timed steps at full size: 256 sequences (32 q / 8 kv
    heads, head_dim 128, bf16 pages, block 32, lognormal target contexts
    median 1024 clipped to [16, 32768]); per step one append launch of the
    512-token prefill chunks of up to 8 sequences still prefilling plus one
    token for every other sequence, then the gather of every live sequence to
    contiguous bf16 [head][len][dim], then the split-K paged decode of every
    live sequence; after the step 13 sequences (5%) are freed and 13 new ones
    created, whose blocks later come from the FIFO free list the frees have
    fragmented (src/paged_attention.rs:115-135).  The same workflow is
    checked bit for bit in tests/test_gpu_full_configs.py.

    The host work of each step (slot allocation through the SequenceManager,
    table export, the frees and creations) is planned first and timed on
    the CPU; every step's slots, tables, rows and queries are then resident
    in HBM, and the device part is timed with HIP events: the whole step
    (three launches), then each launch kind alone over the same steps."""
    import numpy as np

    import airkv
    from airkv import workloads
    NQ, NKV, D, BS, CHUNK, N_SEQ, CHURN = 32, 8, 128, 32, 512, 256, 13
    n_steps = warmup + steps
    rng = np.random.default_rng(180)
    targets0 = workloads.c5_lengths(N_SEQ, seed=181)
    cap = int(1.3 * (sum(targets0) + CHURN * n_steps * 4096 + N_SEQ * n_steps) / BS) + N_SEQ
    mgr = airkv.SequenceManager(cap, BS, free_order=workloads.lcg_permutation(cap, 182))
    pool = airkv.KvPool(cap, BS, NKV, D, airkv.BF16)
    g = torch.Generator(device="cuda")
    g.manual_seed(183)
    seqs = [mgr.create_sequence() for _ in range(N_SEQ)]
    target = dict(zip(seqs, targets0))
    have = {s: 0 for s in seqs}
    # contexts before the measured steps (untimed): all but eight sequences
    # prefilled; those eight take the first step's prefill chunks
    for s in seqs[: N_SEQ - 8]:
        slots = torch.from_numpy(mgr.append_slots(s, target[s])).cuda()
        have[s] = target[s]
        for c0 in range(0, len(slots), 32768):
            sl = slots[c0:c0 + 32768]
            k = torch.randn(len(sl), NKV, D, generator=g, device="cuda")
            pool.append(k, torch.randn_like(k), sl)
    new_targets = iter(workloads.c5_lengths(CHURN * n_steps, seed=184))
    plans, host_us = [], []
    for step in range(n_steps):
        t0 = time.perf_counter()
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
        live = [s for s in seqs if have[s] > 0]
        mb = max(-(-have[s] // BS) for s in live)
        tables, lens = mgr.export_tables(live, mb)
        t1 = time.perf_counter()
        for s in rng.choice(seqs, size=CHURN, replace=False).tolist():
            mgr.free_sequence(s)
            seqs.remove(s)
            del have[s], target[s]
            t = mgr.create_sequence()
            seqs.append(t)
            have[t] = 0
            target[t] = int(next(new_targets))
        t2 = time.perf_counter()
        host_us.append(((t1 - t0) * 1e6, (t2 - t1) * 1e6))
        plans.append((slots, tables, lens, n_pref))
    # device inputs of every step, resident before timing
    dev = []
    max_tok = max(int(p[2].astype(np.int64).sum()) for p in plans)
    gk = torch.empty(max_tok * NKV * D, dtype=torch.bfloat16, device="cuda")
    gv = torch.empty_like(gk)
    ws = pool.new_workspace(NQ, max(len(p[2]) for p in plans), max(p[1].shape[1] for p in plans))
    for slots, tables, lens, _ in plans:
        st = torch.from_numpy(slots).cuda()
        k = torch.randn(len(slots), NKV, D, generator=g, device="cuda")
        v = torch.randn_like(k)
        tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
        per = lens.astype(np.int64) * NKV * D
        offs = torch.from_numpy(np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)).cuda()
        q = torch.randn(len(lens), NQ, D, generator=g, device="cuda").to(torch.bfloat16)
        out = torch.empty_like(q)
        dev.append((pool.bind_append(k, v, st), pool.bind_gather(tt, lt, offs, gk, gv),
                    pool.bind_decode(q, tt, lt, out, ws)))
    torch.cuda.synchronize()

    def run(parts):
        for i in range(warmup):
            for j in parts:
                dev[i][j]()
        torch.cuda.synchronize()
        torch.cuda._sleep(20_000_000)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(warmup, n_steps):
            for j in parts:
                dev[i][j]()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps * 1e3    # us per step

    us_step = run((0, 1, 2))
    us_parts = [run((j,)) for j in range(3)]
    assert pool.error_count() == 0
    timed = plans[warmup:]
    tok_app = sum(len(p[0]) for p in timed) / steps
    ctx = [p[2].astype(np.int64) for p in timed]
    tok = sum(int(c.sum()) for c in ctx) / steps
    pages = sum(int(((c + BS - 1) // BS).sum()) for c in ctx) / steps
    live = sum(len(c) for c in ctx) / steps
    row = NKV * D * 2                                  # K+V elements per token
    b_app = tok_app * (row * (4 + 2) + 8)
    b_gat = tok * row * (2 + 2) + 4 * pages
    b_dec = tok * row * 2 + 4 * pages + live * NQ * D * (2 + 2)

    def part(us, nbytes):
        gbps = nbytes / (us * 1e-6) / 1e9
        return {"us": round(us, 1), "gbps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4),
                "algorithmic_bytes": int(nbytes)}
    res = {"step": part(us_step, b_app + b_gat + b_dec), "append": part(us_parts[0], b_app),
           "gather": part(us_parts[1], b_gat), "decode": part(us_parts[2], b_dec),
           "steps_timed": steps, "appended_tokens_per_step": tok_app,
           "prefill_chunks_per_step": sum(p[3] for p in timed) / steps,
           "live_sequences_per_step": live, "cached_tokens_per_step": tok,
           "tokens_per_step_list": [int(len(p[0])) for p in timed],
           "host_alloc_us_per_step": round(sum(h[0] for h in host_us[warmup:]) / steps, 1),
           "host_free_realloc_us_per_step": round(sum(h[1] for h in host_us[warmup:]) / steps, 1),
           "host_note": "SequenceManager work through the C ABI from Python (ctypes), timed on the CPU; "
                        "not inside the device figures"}
    pool.close()
    return res


def cpu_rate(fn, items, bytes_of, budget_s, threads):
    """One thread: items in order until budget_s (at least one); then every
    item over `threads` threads (ctypes releases the GIL around the C oracle).
    Returns (GB/s on 1 thread, GB/s on all, items done on 1 thread, s)."""
    import concurrent.futures
    done, t0 = 0, time.perf_counter()
    for it in items:
        fn(it)
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    t1 = time.perf_counter() - t0
    with concurrent.futures.ThreadPoolExecutor(threads) as ex:
        t0 = time.perf_counter()
        list(ex.map(fn, items))
        tn = time.perf_counter() - t0
    return bytes_of(items[:done]) / t1 / 1e9, bytes_of(items) / tn / 1e9, done, tn


def cpu_append_gather(budget_s, threads):
    """The oracle's append (f32 rows -> bf16 / Q8_0 int8 / reference fp8
    pages, src/kv_cache.rs:54-75, src/fp8.rs:54-91 + :228-238), its gather
    of the pages back to contiguous [head][len][dim] (bf16 -> bf16, int8 /
    fp8 -> f32 dequantized, src/kv_cache.rs:78-92, src/fp8.rs:263-264), and
    Q8Tensor::quantize over the flattened rows as save_layer calls it
    (src/kv_cache.rs:307-315), on the same geometries, slot sets and byte
    counts as the GPU legs: 32768 rows per config in 512-row items, gathers
    of those rows' four sequences in 1024-token pieces."""
    import numpy as np

    import oracle
    from airkv import workloads
    res = {}
    rows = QUANT_APPEND_ROWS
    for name, dt in (("c2", oracle.BF16), ("c3", oracle.INT8), ("c4", oracle.FP8)):
        if name == "c2":
            cfg = workloads.CONFIGS["c2"]
            w = workloads.build_prefill_decode(cfg, [8192] * 4, seed=51, decode_steps=0)
            slots = np.concatenate(w.batches)[:rows]
        else:
            cfg, w, sets = quant_append_workload(name)
            slots = sets[0]
        host = oracle.HostPool(w.num_blocks, cfg.block_size, cfg.n_kv_heads, cfg.head_dim, dt, cfg.scale_group)
        outl = workloads.outlier_channels(cfg.n_kv_heads, cfg.head_dim, seed=3) if name == "c3" else None
        k, v = next(workloads.kv_rows(rows, cfg.n_kv_heads, cfg.head_dim, seed=63, outliers=outl,
                                      chunk_rows=rows))
        items = [(i, min(i + 512, rows)) for i in range(0, rows, 512)]
        eb = oracle.ELEM_BYTES[dt]
        rb = cfg.n_kv_heads * cfg.head_dim * 2 * (4 + eb) + 8
        if dt != oracle.BF16:
            rb += cfg.n_kv_heads * (cfg.head_dim // cfg.scale_group) * 4 * 2

        def app(it):
            host.append(k[it[0]:it[1]], v[it[0]:it[1]], slots[it[0]:it[1]])
        a1, an, d1, tn = cpu_rate(app, items, lambda its: rb * sum(b - a for a, b in its), budget_s, threads)
        kd = {oracle.BF16: "bf16", oracle.INT8: "int8", oracle.FP8: "fp8"}[dt]
        res[f"append_{kd}"] = {"gbps_1thread": round(a1, 3), "gbps_all": round(an, 3),
                               "sample": f"{name} geometry, {rows} f32 K/V rows in 512-row appends over a shuffled "
                                         f"pool; one thread {d1} appends, {threads} threads all in {tn:.2f} s"}
        # gather of the appended rows' four sequences, 1024-token pieces
        tables, lens = w.tables()
        per_blk = 1024 // cfg.block_size
        pieces = [(b, j) for b in range(4) for j in range(int(lens[b]) // 1024)]
        odt = oracle.BF16 if dt == oracle.BF16 else oracle.F32
        ob = 2 if odt == oracle.BF16 else 4
        gb = 1024 * (cfg.n_kv_heads * cfg.head_dim * 2 * (eb + ob)) + 4 * per_blk
        if dt != oracle.BF16:
            gb += 1024 * cfg.n_kv_heads * (cfg.head_dim // cfg.scale_group) * 4 * 2

        def gat(p):
            b, j = p
            t = np.ascontiguousarray(tables[b:b + 1, j * per_blk:(j + 1) * per_blk])
            _, _, _, bad = host.gather(t, np.array([1024], np.int32), odt)
            assert bad == 0
        g1, gn, d1, tn = cpu_rate(gat, pieces, lambda ps: gb * len(ps), budget_s, threads)
        res[f"gather_{kd}_to_{'bf16' if ob == 2 else 'f32'}"] = {
            "gbps_1thread": round(g1, 3), "gbps_all": round(gn, 3),
            "sample": f"{name} geometry, four 8192-token sequences in {len(pieces)} pieces of 1024 tokens; one "
                      f"thread {d1} pieces, {threads} threads all in {tn:.2f} s"}
        if dt == oracle.INT8:
            flat = k.reshape(-1)

            def q8(it):
                a, b = it[0] * cfg.n_kv_heads * cfg.head_dim, it[1] * cfg.n_kv_heads * cfg.head_dim
                oracle.q8_quantize(flat[a:b])
            qb = cfg.n_kv_heads * cfg.head_dim * (4 + 1) + cfg.n_kv_heads * (cfg.head_dim // 32) * 4
            q1, qn, d1, tn = cpu_rate(q8, items, lambda its: qb * sum(b - a for a, b in its), budget_s, threads)
            res["quantize_q8"] = {"gbps_1thread": round(q1, 3), "gbps_all": round(qn, 3),
                                  "sample": f"Q8Tensor::quantize of {rows} K rows (x {cfg.n_kv_heads * cfg.head_dim} "
                                            f"f32) in 512-row pieces; one thread {d1} pieces, {threads} threads "
                                            f"all in {tn:.2f} s"}
        del host
    return res


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the paged KV path runs on one "
                                   "MI355X and no multi-GPU figure is produced (--gpus 1)"}))
        sys.exit(2)

    import numpy as np
    import torch

    import airkv
    from airkv import workloads

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    dev = "cuda"
    cfg = workloads.CONFIGS["c2"]
    n_steps = args.warmup + args.steps
    lens0 = workloads.c2_lengths(cfg.batch, 512, 4096, seed=2)
    t_setup = time.perf_counter()
    w = workloads.build_prefill_decode(cfg, lens0, seed=2, decode_steps=n_steps)
    pool = airkv.KvPool(w.num_blocks, cfg.block_size, cfg.n_kv_heads, cfg.head_dim, cfg.dtype)
    log(f"pool {w.num_blocks} blocks, {sum(lens0)} prefill tokens, {n_steps} steps")

    # prefill (untimed): stream f32 K/V through the append kernel
    n_prefill = len(lens0)
    gen = workloads.kv_rows(10 ** 12, cfg.n_kv_heads, cfg.head_dim, seed=5, device=dev,
                            chunk_rows=8192)
    for slots in w.batches[:n_prefill]:
        done = 0
        while done < len(slots):
            k, v = next(gen)
            n = min(len(slots) - done, k.shape[0])
            pool.append(k[:n].contiguous(), v[:n].contiguous(),
                        torch.from_numpy(slots[done:done + n]).to(dev))
            done += n
    # per-step inputs, resident before timing
    step_slots = [torch.from_numpy(s).to(dev) for s in w.batches[n_prefill:]]
    step_k = [torch.randn(cfg.batch, cfg.n_kv_heads, cfg.head_dim, device=dev) for _ in range(n_steps)]
    step_v = [torch.randn(cfg.batch, cfg.n_kv_heads, cfg.head_dim, device=dev) for _ in range(n_steps)]
    step_q = [torch.randn(cfg.batch, cfg.n_q_heads, cfg.head_dim, device=dev).to(torch.bfloat16)
              for _ in range(n_steps)]
    tables_np, lens_final = w.tables()
    max_blocks = tables_np.shape[1]
    tables = torch.from_numpy(tables_np).to(dev)
    step_lens = [torch.from_numpy((np.array(lens0) + i + 1).astype(np.int32)).to(dev)
                 for i in range(n_steps)]
    out = torch.empty(cfg.batch, cfg.n_q_heads, cfg.head_dim, device=dev, dtype=torch.bfloat16)
    ws = pool.new_workspace(cfg.n_q_heads, cfg.batch, max_blocks, args.max_splits)
    # Steps alternate between the pool and a copy of it (same bytes, same
    # tables), so no step finds pages the previous one left in the 256 MB
    # MALL: in a model, the other layers' pages pass through it between two
    # steps of one layer.  Each copy takes the appends of its own steps; the
    # bytes every step moves are the same.
    twin = twin_pool(torch, pool)
    pools = (pool, twin)
    appends = [pools[i % 2].bind_append(step_k[i], step_v[i], step_slots[i]) for i in range(n_steps)]
    decodes = [pools[i % 2].bind_decode(step_q[i], tables, step_lens[i], out, ws, max_splits=args.max_splits)
               for i in range(n_steps)]
    # the step as one launch: step i's K/V rows land at token step_lens[i] - 1,
    # the slot step_slots[i] names, written by the decode that reads them
    fused = [pools[i % 2].bind_decode_append(step_q[i], step_k[i], step_v[i], tables, step_lens[i], out, ws,
                                             max_splits=args.max_splits) for i in range(n_steps)]
    torch.cuda.synchronize()
    log(f"setup {time.perf_counter() - t_setup:.1f} s")

    def timed_steps(step_fns):
        for i in range(args.warmup):
            for f in step_fns[i]:
                f()
        torch.cuda.synchronize()
        torch.cuda._sleep(20_000_000)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(args.warmup, n_steps):
            for f in step_fns[i]:
                f()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    # ---- timed steps: append + decode in one launch, then as two calls ----
    ms_step = timed_steps([(f,) for f in fused])
    ms_two = timed_steps(list(zip(appends, decodes)))
    assert pool.error_count() == 0 and twin.error_count() == 0

    kv_b = cfg.n_kv_heads * cfg.head_dim * 2 * 2           # K+V bytes per cached token (bf16)
    bs = cfg.block_size
    lens_t = np.array(lens0) + args.warmup + 1 + np.arange(args.steps)[:, None]   # [steps][batch]

    def decode_bytes(lens):
        tok = int(np.sum(lens))
        pages = int(np.sum((lens + bs - 1) // bs))
        qo = cfg.batch * cfg.n_q_heads * cfg.head_dim * (2 + 2)
        return tok * kv_b + 4 * pages + qo

    # new rows: f32 K and V read, bf16 written; the two-call step also reads
    # the int64 slot mapping
    append_bytes_step = cfg.batch * cfg.n_kv_heads * cfg.head_dim * 2 * (4 + 2)
    step_bytes = sum(decode_bytes(l) for l in lens_t) / args.steps + append_bytes_step
    value = step_bytes / (ms_step * 1e-3) / 1e9
    two_gbps = (step_bytes + 8 * cfg.batch) / (ms_two * 1e-3) / 1e9
    extra_step = {"step_two_call_us": round(ms_two * 1e3, 2), "step_two_call_gbps": round(two_gbps, 1)}
    log(f"step {ms_step * 1e3:.1f} us, {value:.0f} GB/s (two calls: {ms_two * 1e3:.1f} us, {two_gbps:.0f} GB/s)")

    # ---- decode kernel alone, final state ---------------------------------
    # calls alternate between the pool and a copy of it (same bytes, same
    # tables), so no call finds pages the previous one left in the MALL
    last = alternating([p.bind_decode(step_q[-1], tables, step_lens[-1], out, ws, max_splits=args.max_splits)
                        for p in (pool, twin)])
    ms_dec = timed_loop(torch, last, args.kernel_iters)
    dec_bytes = decode_bytes(np.array(lens0) + n_steps)
    dec_gbps = dec_bytes / (ms_dec * 1e-3) / 1e9
    log(f"decode {ms_dec * 1e3:.1f} us, {dec_gbps:.0f} GB/s ({dec_gbps / PEAK_HBM_GBPS:.1%} of peak)")
    dec_pct = per_call_us(torch, last)
    log(f"decode per call p10 / p50 / p90: {dec_pct} us")

    extra = dict(extra_step)
    extra["decode_us_p10_p50_p90"] = list(dec_pct)
    legs = set(args.legs.split(",")) if args.legs != "all" else {
        "gather_append", "ceilings", "configs", "quant_append", "c5_step", "prefill", "compress", "blocks"}
    if args.only_decode:
        legs = set()
    if args.no_configs:
        legs -= {"configs", "quant_append", "c5_step", "prefill", "compress", "blocks"}
    if "gather_append" in legs:
        # gather of every sequence to contiguous bf16 [head][len][dim]
        lens_f = np.array(lens0) + n_steps
        per = lens_f.astype(np.int64) * cfg.n_kv_heads * cfg.head_dim
        offs = torch.from_numpy(np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)).to(dev)
        gk = torch.empty(int(per.sum()), dtype=torch.bfloat16, device=dev)
        gv = torch.empty_like(gk)
        gather = alternating([p.bind_gather(tables, step_lens[-1], offs, gk, gv) for p in (pool, twin)])
        ms_g = timed_loop(torch, gather, 20)
        g_bytes = int(per.sum()) * 2 * 2 * 2 + 4 * int(np.sum((lens_f + bs - 1) // bs))
        extra["gather_gbps"] = round(g_bytes / (ms_g * 1e-3) / 1e9, 1)
        extra["gather_us"] = round(ms_g * 1e3, 1)
        del gk, gv
        # large append: 32768 prefill-like tokens (rewrites existing slots)
        # (two source / slot sets used alternately: 2 x 268 MB of f32 rows
        # exceed the 256 MB MALL, so no launch reads a cached source)
        allslots = np.concatenate(w.batches[:n_prefill])
        sets = []
        for j in range(2):
            big = allslots[j * 32768:(j + 1) * 32768]
            bk = torch.randn(len(big), cfg.n_kv_heads, cfg.head_dim, device=dev)
            bv = torch.randn_like(bk)
            sets.append(pool.bind_append(bk, bv, torch.from_numpy(big).to(dev)))
        flip = [0]

        def big_app():
            sets[flip[0]]()
            flip[0] ^= 1
        ms_a = timed_loop(torch, big_app, 20)
        a_bytes = len(big) * cfg.n_kv_heads * cfg.head_dim * 2 * (4 + 2) + 8 * len(big)
        extra["append_gbps"] = round(a_bytes / (ms_a * 1e-3) / 1e9, 1)
        extra["append_us"] = round(ms_a * 1e3, 1)
        extra["append_tokens"] = int(len(big))
        # the per-step 64-token append alone
        ms_sa = timed_loop(torch, appends[-1], 50)
        extra["step_append_us"] = round(ms_sa * 1e3, 2)
        log(f"gather {extra['gather_gbps']} GB/s, append {extra['append_gbps']} GB/s")

    # ---- plain device copy: a measured reference point, and the known-size
    # kernel that calibrates the FETCH_SIZE / WRITE_SIZE counters of the
    # profiling runs (1 GiB read + 1 GiB written per launch)
    nbytes = 1 << 30
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).uniform_()
    dst = torch.empty_like(src)
    ms_c = timed_loop(torch, lambda: dst.copy_(src), 20)
    extra["copy_gbps"] = round(2 * nbytes / (ms_c * 1e-3) / 1e9, 1)
    del src, dst
    log(f"torch copy {extra['copy_gbps']} GB/s")

    if "ceilings" in legs:
        extra["ceilings"] = ceilings_leg(torch)
        log(f"ceilings {extra['ceilings']}")
        c = extra["ceilings"]
    if "ceilings" in legs and "gather_append" in legs:
        extra["frac_of_ceiling"] = {
            "decode_vs_page_read": round(dec_gbps / c["page_read"]["gbps"], 4),
            "gather_vs_copy": round(extra["gather_gbps"] / c["copy"]["gbps"], 4),
            "gather_vs_copy_best": round(extra["gather_gbps"] / c["copy_best"]["gbps"], 4),
            "gather_vs_page_copy": round(extra["gather_gbps"] / c["page_copy"]["gbps"], 4),
            "append_vs_mix21": round(extra["append_gbps"] / c["mix21"]["gbps"], 4),
            "append_vs_mix21_best": round(extra["append_gbps"] / c["mix21_best"]["gbps"], 4),
            "append_vs_page_mix21": round(extra["append_gbps"] / c["page_mix21"]["gbps"], 4),
        }

    if "configs" in legs:
        extra["other_configs"] = {}
        for name in ("c3", "c4", "c5"):
            extra["other_configs"][name] = config_decode(torch, name)
            if "ceilings" in extra:
                extra["other_configs"][name]["frac_of_page_read_ceiling"] = round(
                    extra["other_configs"][name]["decode_gbps"] / extra["ceilings"]["page_read"]["gbps"], 4)
            log(f"{name} decode {extra['other_configs'][name]}")
    if "quant_append" in legs:
        extra["append_quantized"] = {name: quant_append_leg(torch, name) for name in ("c3", "c4")}
        log(f"quantize-on-append {extra['append_quantized']}")
    if "c5_step" in legs:
        extra["c5_step"] = c5_step_leg(torch)
        log(f"c5 step {extra['c5_step']}")
    if "prefill" in legs:
        extra["prefill_c5"] = prefill_leg(torch)
        log(f"prefill {extra['prefill_c5']['tflops']} TFLOP/s")
        extra["prefill_one_sequence_32k"] = prefill_leg(torch, iters=5, prefix=[32256])
        log(f"prefill one sequence {extra['prefill_one_sequence_32k']['tflops']} TFLOP/s")
        extra["prefill_c5_chunks_int8_70b"] = prefill_leg(torch, int8_70b=True)
        log(f"prefill int8 70B geometry {extra['prefill_c5_chunks_int8_70b']['tflops']} TFLOP/s")
    if "compress" in legs:
        extra["kv_compress_blocks"] = compress_leg(torch)
        log(f"compress blocks {extra['kv_compress_blocks']['gbps']} GB/s")
    if "blocks" in legs:
        extra["kv_blocks"] = blocks_leg(torch)
        log(f"block copy / wire {extra['kv_blocks']}")

    cpu = None
    if not args.no_cpu:
        q_last = step_q[-1].float().cpu().numpy()
        lens_final = (np.array(lens0) + n_steps).astype(np.int32)

        def bytes_of(lens, nseq):
            lens = np.asarray(lens, np.int64)
            return (int(lens.sum()) * kv_b + 4 * int(((lens + bs - 1) // bs).sum())
                    + nseq * cfg.n_q_heads * cfg.head_dim * (2 + 2))
        cpu = cpu_baseline(pool, w, tables_np, lens_final, q_last, args.cpu_seconds, bytes_of)
        log(f"cpu oracle {cpu['value']:.3f} GB/s ({cpu['cores']} threads), "
            f"{cpu['value_1core']:.3f} GB/s (1 thread)")
        cpu["pieces"] = cpu_append_gather(min(2.0, args.cpu_seconds), cpu["cores"])
        log(f"cpu oracle append / gather / quantize {cpu['pieces']}")

    result = {
        "metric": "paged decode attn HBM GB/s (% of peak); KV append+gather GB/s, 1 MI355X",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V/Q, seeded U[512,4096] contexts, shuffled pool)",
        "config": {
            "workload": "c2: append 1 token/seq + split-K paged decode (one fused launch), "
                        "Llama-3-8B shape",
            "batch": cfg.batch, "n_q_heads": cfg.n_q_heads, "n_kv_heads": cfg.n_kv_heads,
            "head_dim": cfg.head_dim, "block_size": cfg.block_size, "kv_dtype": "bf16",
            "q_dtype": "bf16", "out_dtype": "bf16", "ctx": "U[512,4096] seed 2",
            "pool_blocks": w.num_blocks, "max_splits": args.max_splits,
            "cached_tokens_final": int(np.sum(np.array(lens0) + n_steps)),
        },
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBPS, 2),
        "decode_gbps": round(dec_gbps, 1),
        "decode_us": round(ms_dec * 1e3, 2),
        "tokens_per_s": round(cfg.batch / (ms_step * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(dec_gbps, 1), "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": round(dec_gbps / PEAK_HBM_GBPS, 4),
                     "traffic": profiled_traffic(), "algorithmic_bytes": int(dec_bytes)},
        "cpu_baseline": cpu,
    }
    result.update(extra)
    print(json.dumps(result), flush=True)
    twin.close()
    pool.close()


if __name__ == "__main__":
    main()
