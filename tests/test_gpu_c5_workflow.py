"""configs[4] as a workflow: continuous batching over a fragmented pool,
checked against the oracle after every step.

Each step appends, in one launch, 512-token prefill chunks for the
sequences still prefilling plus one token for every decoding sequence; 5% of
the sequences are then freed and replaced by new ones, whose blocks come from
the FIFO free list that the frees have fragmented
(src/paged_attention.rs:115-135).  After the step every sequence is gathered
(bit-exact against the oracle's pool) and decoded (within 1e-3 of the
oracle).  The shape is configs[4]'s (32 q / 8 kv heads, head_dim 128, bf16
pages, block 32, lognormal contexts) at 64 sequences instead of 256, so the
oracle finishes in seconds; the full-size decode is a bench.py leg.
"""
import numpy as np
import pytest

import airkv
import oracle
from airkv import workloads
from gpu_helpers import log, rel_err, torch_mod

pytestmark = pytest.mark.gpu

NQ, NKV, D, BS = 32, 8, 128, 32
CHUNK = 512


def test_c5_continuous_batching_steps():
    torch = torch_mod()
    rng = np.random.default_rng(70)
    n_seq, cap = 64, 1600
    mgr = airkv.SequenceManager(cap, BS, free_order=workloads.lcg_permutation(cap, 71))
    pool = airkv.KvPool(cap, BS, NKV, D, airkv.BF16)
    host = oracle.HostPool(cap, BS, NKV, D, oracle.BF16)

    def new_target():
        return int(workloads.c5_lengths(1, median=256, sigma=1.0, lo=16, hi=1500,
                                        seed=int(rng.integers(1 << 30)))[0])

    seqs = [mgr.create_sequence() for _ in range(n_seq)]
    target = {s: new_target() for s in seqs}       # prefill length still to reach
    have = {s: 0 for s in seqs}
    # contexts exist before the measured steps: prefill every sequence
    while any(have[s] < target[s] for s in seqs):
        slots = []
        for s in seqs:
            n = min(CHUNK, target[s] - have[s])
            if n > 0:
                slots.append(mgr.append_slots(s, n))
                have[s] += n
        slots = np.concatenate(slots)
        k = rng.standard_normal((len(slots), NKV, D), dtype=np.float32)
        v = rng.standard_normal((len(slots), NKV, D), dtype=np.float32)
        pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                    torch.from_numpy(slots).cuda())
        assert host.append(k, v, slots) == 0
    freed_total = 0
    for step in range(5):
        # one append launch: prefill chunks (up to 8 sequences) + 1 token for the rest
        slots, prefill_n = [], 0
        for s in seqs:
            if have[s] < target[s] and prefill_n < 8:
                n = min(CHUNK, target[s] - have[s])
                prefill_n += 1
            elif have[s] >= target[s]:
                n = 1
            else:
                continue                            # waits for a prefill slot
            slots.append(mgr.append_slots(s, n))
            have[s] += n
        slots = np.concatenate(slots)
        k = rng.standard_normal((len(slots), NKV, D), dtype=np.float32)
        v = rng.standard_normal((len(slots), NKV, D), dtype=np.float32)
        pool.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                    torch.from_numpy(slots).cuda())
        assert host.append(k, v, slots) == 0

        # gather + decode every live sequence with some tokens
        live = [s for s in seqs if have[s] > 0]
        mb = max(-(-have[s] // BS) for s in live)
        tables, lens = mgr.export_tables(live, mb)
        tt, lt = torch.from_numpy(tables).cuda(), torch.from_numpy(lens).cuda()
        per = lens.astype(np.int64) * NKV * D
        offs = np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int64)
        gk = torch.empty(int(per.sum()), dtype=torch.bfloat16, device="cuda")
        gv = torch.empty_like(gk)
        pool.gather(tt, lt, torch.from_numpy(offs).cuda(), gk, gv)
        hk, hv, _, bad = host.gather(tables, lens, oracle.BF16)
        assert bad == 0
        assert np.array_equal(gk.cpu().view(torch.int16).numpy().view(np.uint16), hk)
        assert np.array_equal(gv.cpu().view(torch.int16).numpy().view(np.uint16), hv)
        q = torch.randn(len(live), NQ, D, device="cuda").to(torch.bfloat16)
        out = torch.empty(len(live), NQ, D, device="cuda")
        pool.paged_decode(q, tt, lt, out)
        want = host.paged_decode(q.float().cpu().numpy(), tables, lens)
        err = rel_err(out.cpu().numpy(), want)
        log(f"step {step}: {len(slots)} tokens appended ({prefill_n} prefill chunks), "
            f"{int(lens.sum())} cached, {mgr.allocator.num_free_blocks()} blocks free, decode err {err:.2e}")
        assert err <= 1e-3
        assert pool.error_count() == 0

        # 5% churn: free three sequences, start three new ones
        for s in rng.choice(seqs, size=3, replace=False).tolist():
            mgr.free_sequence(s)
            seqs.remove(s)
            del have[s], target[s]
            freed_total += 1
            t = mgr.create_sequence()
            seqs.append(t)
            have[t] = 0
            target[t] = new_target()
    assert freed_total == 15
