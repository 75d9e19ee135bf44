"""Device-side ingest (GlobalIndex.harvest_device, SuffixGPUDrafter.
harvest_finished with device row indices and lengths) against the oracle's
index with the same schedule: a rebuild that starts during an append is
still running at the appends' own polls (global_index.py:111,140) and
finishes at the caller's next poll_rebuild.  Every round compares the
whole index state -- corpus, suffix array, delta, lengths and both
doc-length lists -- after the caller's poll."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.global_index import GlobalIndexOracle
from suffixgpu_amd import synth
from tests.test_gpu_global import N, T, gpu_state_equal

pytestmark = pytest.mark.gpu

I32 = np.int32


def _pair(gpu, stream, **kw):
    from suffixgpu_amd.global_index import GlobalIndex
    side = torch.cuda.Stream(gpu) if stream else None
    g = GlobalIndex(device=gpu, rebuild_stream=side, **kw)
    g.blocking_poll = True
    o = GlobalIndexOracle(async_rebuild=True, finish_at_user_poll=True, **kw)
    return g, o


def _round(g, o, gpu, rng, b, s, vocab, idx64, lmax):
    tok = rng.integers(0, vocab, size=(b, s)).astype(I32)
    lengths = rng.integers(0, lmax, size=b)
    lengths[rng.integers(0, b)] = s  # longer than the delta
    lengths[rng.integers(0, b)] = 0
    rows = rng.permutation(b)[:max(1, b - 2)]
    dt = torch.int64 if idx64 else torch.int32
    g.harvest_device(T(rows, gpu).to(dt), T(lengths[rows], gpu).to(dt),
                     T(tok, gpu))
    o.append_documents([tok[r, :min(int(lengths[r]), s)] for r in rows
                        if lengths[r] > 0])


@pytest.mark.parametrize("stream", [False, True])
def test_device_harvest_matches_oracle(gpu, stream):
    """Rounds of harvests that truncate, make room, drop the oldest delta
    documents while a rebuild runs, stage snapshots that evict corpus
    documents, and end with maybe_rebuild."""
    rng = np.random.default_rng(31)
    g, o = _pair(gpu, stream, capacity=6000, delta_capacity=1500, k=4,
                 max_occurrences=8, rebuild_threshold=700)
    for rnd in range(14):
        # even rounds append more than twice the delta's capacity: the
        # second overflow finds the snapshot of the first still running
        b = 40 if rnd % 2 == 0 else 7
        _round(g, o, gpu, rng, b, 900, 7, rnd % 3 == 0, 200)
        g.poll_rebuild()
        o.poll_rebuild()
        g.sync_host_state()
        gpu_state_equal(g, o)
        assert g.ingest_counters["bad_rows"] == 0
    assert g.ingest_counters["docs_dropped"] > 0


def test_device_and_host_harvests_interleave(gpu):
    """Host-side appends, device harvests and a rebuild the host started
    running across the switch, in one sequence: the bookkeeping moves
    between the host lists and device memory without a difference.  A
    host-side append with blocking_poll waits for a running rebuild at its
    own polls, so the oracle takes that schedule for those calls."""
    rng = np.random.default_rng(32)
    g, o = _pair(gpu, True, capacity=8000, delta_capacity=2000, k=4,
                 max_occurrences=8, rebuild_threshold=900)
    tc = synth.TemplateCorpus(seed=33, n_templates=4)
    docs = [tc.sequence(lo=50, hi=400) for _ in range(12)]
    g.load_documents([T(d, gpu) for d in docs])
    o.load_documents(docs)
    for rnd in range(10):
        if rnd % 3 == 2:
            extra = [tc.sequence(lo=20, hi=300) for _ in range(5)]
            g.append_documents([T(d, gpu) for d in extra])
            o.finish_at_user_poll = False
            o.append_documents(extra)
            o.finish_at_user_poll = True
        else:
            _round(g, o, gpu, rng, 25, 700, 9, rnd % 2 == 0, 160)
        if rnd % 4 != 3:  # sometimes no poll between two harvests
            g.poll_rebuild()
            o.poll_rebuild()
            g.sync_host_state()
            gpu_state_equal(g, o)
    g.poll_rebuild()
    o.poll_rebuild()
    g.sync_host_state()
    gpu_state_equal(g, o)


def test_device_harvest_reads_nothing_back(gpu):
    """After the first device harvest (which uploads the host lists), a
    harvest and the drafter step run with no synchronising copy: torch's
    sync debug mode raises on any.  Bad rows are skipped and counted."""
    from suffixgpu_amd import SuffixGPUDrafter
    rng = np.random.default_rng(34)
    d = SuffixGPUDrafter(k=4, device=gpu, max_pattern_len=8,
                         max_occurrences=8, num_backoff=3,
                         enable_global=True, global_capacity=1 << 14,
                         delta_capacity=1 << 11, rebuild_threshold=800,
                         rebuild_stream=torch.cuda.Stream(gpu))
    tok = T(rng.integers(0, 11, size=(16, 300)).astype(I32), gpu)
    rows = torch.arange(16, device=gpu)
    lens = torch.full((16,), 120, dtype=torch.int64, device=gpu)
    d.harvest_finished(rows, lens, tok)
    torch.cuda.synchronize()
    prev = torch.cuda.get_sync_debug_mode()
    torch.cuda.set_sync_debug_mode("error")
    try:
        for _ in range(6):
            d.harvest_finished(rows, lens, tok)
    finally:
        torch.cuda.set_sync_debug_mode(prev)
    bad = torch.tensor([0, 16, -1, 3], device=gpu)
    d.harvest_finished(bad, torch.full((4,), 5, device=gpu), tok)
    d.global_index.blocking_poll = True
    d.poll()
    assert d.global_index.ingest_counters["bad_rows"] == 2
    assert d.global_index.ingest_counters["docs_in"] == 7 * 16 + 2


def test_device_harvest_argument_errors(gpu):
    from suffixgpu_amd.global_index import GlobalIndex
    g = GlobalIndex(capacity=1024, delta_capacity=256, k=4, device=gpu)
    tok = torch.zeros((4, 8), dtype=torch.int32, device=gpu)
    r = torch.arange(4, device=gpu)
    with pytest.raises(ValueError):
        g.harvest_device(r, r[:3], tok)
    with pytest.raises(TypeError):
        g.harvest_device(r.float(), r, tok)
    with pytest.raises(ValueError):
        g.harvest_device(r.cpu(), r, tok)
    with pytest.raises(ValueError):
        big = torch.zeros(5000, dtype=torch.int64, device=gpu)
        g.harvest_device(big, big, tok)
    assert int(g.delta_len_t.item()) == 0
    assert N(g.delta)[:4].tolist() == [0, 0, 0, 0]
