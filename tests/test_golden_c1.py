"""configs[0] (c1) against its committed digests (tests/golden/c1_digests.json):
the oracle's pages, scales and gathered views for every dtype, the inputs,
and the block tables of both the product's allocator and the oracle's
restatement of it (src/paged_attention.rs:89-381).  CPU only; the GPU side
is checked against the same file in test_gpu_append_gather.py."""
import json
import os
import sys

import numpy as np

from oracle import paged_attention_ref as ref

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import c1_digests as c1  # noqa: E402


def _fixture():
    with open(c1.JSON_PATH) as f:
        return json.load(f)


def test_fixture_describes_c1():
    doc = _fixture()
    assert doc["prefill"] == [37, 128, 200, 511] and doc["decode_steps"] == 16
    assert doc["final_lens"] == [53, 144, 216, 527]
    _, _, tables, lens, _, _ = c1.workload()
    assert lens.tolist() == doc["final_lens"]
    assert [int((t >= 0).sum()) for t in tables] == [4, 9, 14, 33]


def test_oracle_allocator_reproduces_the_slots():
    """The restated allocator, driven by the same calls, gives the slot
    batches whose digest the fixture holds."""
    doc = _fixture()
    w, batches, _, _, _, _ = c1.workload()
    mgr = ref.SequenceManager(c1.NUM_BLOCKS, c1.BS, free_order=w.free_order.tolist())
    seqs = [mgr.create_sequence() for _ in c1.PREFILL]
    got = []
    for s, n in zip(seqs, c1.PREFILL):
        got.append(np.array([mgr.slot_for_append(s) for _ in range(n)], np.int64))
    for _ in range(c1.STEPS):
        got.append(np.array([mgr.slot_for_append(s) for s in seqs], np.int64))
    assert c1.sha(np.concatenate(got)) == doc["digests"]["inputs"]["slots"]
    assert c1.sha(np.concatenate(batches)) == doc["digests"]["inputs"]["slots"]


def test_oracle_matches_the_digests():
    doc = _fixture()
    assert c1.oracle_digests() == doc["digests"]
