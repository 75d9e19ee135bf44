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
from tests.conftest import golden
from tests.test_gpu_global import N, T, gpu_state_equal
from tests.test_oracle_golden import (ACTIVE, HARVEST, INGEST_KW,
                                      ScriptedEvent, ingest_ops)

pytestmark = pytest.mark.gpu

I32 = np.int32


def device_state_equal(g, running: bool, active_len: int, live_len: int,
                       corpus_lens, delta_lens, corpus, sa, delta,
                       staging=None) -> None:
    """The index's device bookkeeping (read without handing it back to
    the host) and buffers against expected values: corpus_lens describes
    the corpus once a running rebuild is swapped in."""
    st = g.device_state()
    assert st["in_flight"] == int(running)
    assert st["active_len"] == active_len
    assert st["live_active_len"] == live_len
    assert st["corpus_doc_lens"] == list(corpus_lens)
    assert st["delta_doc_lens"] == list(delta_lens)
    assert st["delta_len"] == len(delta)
    assert int(g.delta_len_t.item()) == len(delta)
    np.testing.assert_array_equal(N(g.delta)[:len(delta)], delta)
    np.testing.assert_array_equal(N(g.corpus), corpus)
    np.testing.assert_array_equal(N(g.sa), sa)
    if staging is not None:
        np.testing.assert_array_equal(N(g.staging_corpus), staging)


def oracle_device_state_equal(g, o) -> None:
    running = o._rebuild_event is not None
    device_state_equal(
        g, running, o._pending[0] if running else o.active_len,
        o.active_len, o._pending[1] if running else o.active_doc_lens,
        o.delta_doc_lens, o.corpus, o.sa, o.delta[:o.delta_len],
        o.staging_corpus if running else None)


def test_ingest_trace_golden_on_device(gpu):
    """The reference's own harvest_finished / ingest_active trace (rebuilds
    finishing only at the script's polls marked done) replayed through
    the device paths: device row indices (negative ones count from the
    end), lengths <= 0 and past the row, documents longer than the delta,
    drops while a snapshot runs, evictions, and ingest_active's chunk /
    overlap / final rules with device slot keys.  After every operation
    the device bookkeeping, the buffers, the staged corpus and the slot
    progress table equal the reference's, with nothing handed back to the
    host in between."""
    from suffixgpu_amd import SuffixGPUDrafter
    z = golden("ingest_trace")
    d = SuffixGPUDrafter(device=gpu, rebuild_stream=torch.cuda.Stream(gpu),
                         **INGEST_KW)
    g = d.global_index
    g.blocking_poll = True
    i64 = torch.int64
    for i, kind, args in ingest_ops(z):
        if kind == HARVEST:
            tok, idx, lens = args
            d.harvest_finished(T(idx, gpu, i64), T(lens, gpu, i64),
                               T(tok, gpu))
        elif kind == ACTIVE:
            tok, keys, lens, final, chunk = args
            d.ingest_active(T(keys, gpu, i64), T(tok, gpu),
                            T(lens, gpu, i64), final=final, chunk=chunk)
        elif args[0]:  # a poll that finds the rebuild done
            d.poll()
        running = bool(z[f"in_flight_{i}"])
        device_state_equal(
            g, running, int(z[f"pend_n_new_{i}" if running
                              else f"active_len_{i}"]),
            int(z[f"active_len_{i}"]),
            z[f"pend_lens_{i}" if running else f"active_doc_lens_{i}"]
            .tolist(), z[f"delta_doc_lens_{i}"].tolist(), z[f"corpus_{i}"],
            z[f"sa_{i}"], z[f"delta_{i}"], z[f"staging_{i}"])
        if d._ingested_dev is not None:
            table = N(d._ingested_dev)
            want = np.zeros_like(table)
            want[z[f"ing_keys_{i}"]] = z[f"ing_vals_{i}"]
            np.testing.assert_array_equal(table, want, err_msg=f"op {i}")
    assert g._ing_live and g.ingest_counters.get("bad_rows", 0) == 0


@pytest.mark.parametrize("blocking", [True, False])
def test_device_ingest_long_run_wraps_rings(gpu, blocking):
    """Device-resident bookkeeping over 150 harvests and ingest_active
    calls with no sync_host_state in between: small capacities, so the
    corpus and delta doc-length rings wrap several times, compared with
    the oracle through device_state() every few calls.  blocking=False
    polls as the reference does (the event queried, never waited for);
    the oracle's rebuilds then complete at the polls where the GPU's
    swapped, and pinned header copies issued before a swap must not
    bring back the corpus length from before it."""
    from suffixgpu_amd.global_index import GlobalIndex
    rng = np.random.default_rng(35)
    kw = dict(capacity=600, delta_capacity=200, k=4, max_occurrences=8,
              rebuild_threshold=100)
    g = GlobalIndex(device=gpu, rebuild_stream=torch.cuda.Stream(gpu), **kw)
    g.blocking_poll = blocking
    o = GlobalIndexOracle(async_rebuild=True, finish_at_user_poll=True,
                          **kw)
    ev = ScriptedEvent()
    o.rebuild_event_factory = lambda: ev
    ingested = torch.zeros(64, dtype=torch.int64, device=gpu)
    o_ing: dict = {}
    swaps = 0
    for it in range(150):
        rows, seq = 12, 40
        tok = rng.integers(0, 9, size=(rows, seq)).astype(I32)
        if it % 5 == 4:  # ingest_active, chunk 8, overlap 6
            keys = rng.choice(64, size=6, replace=False)
            lens = rng.integers(0, seq + 3, size=6)
            final = bool(rng.random() < 0.3)
            g.ingest_active_device(T(keys, gpu), T(tok[:6], gpu),
                                   T(lens, gpu), ingested, final, 8, 6)
            docs = []
            for key, row, ln in zip(keys, tok[:6], lens):
                done = o_ing.get(int(key), 0)
                if ln - done >= 8 or (final and ln > done):
                    docs.append(row[max(0, done - 6):ln])
                    o_ing[int(key)] = int(ln)
                if final:
                    o_ing.pop(int(key), None)
            if docs:
                o.append_documents(docs)
        else:
            idx = rng.integers(-rows, rows, size=10)
            lens = rng.integers(-2, 30, size=10)
            g.harvest_device(T(idx, gpu), T(lens, gpu), T(tok, gpu))
            docs = [tok[r, :ln] for r, ln in zip(idx, lens) if ln > 0]
            if docs:  # harvest_rows calls append_documents only then
                o.append_documents(docs)
        if it % 3 == 2:
            before = g.swap_count
            g.poll_rebuild()
            ev.done = g.swap_count != before
            assert not ev.done or o._rebuild_event is not None
            o.poll_rebuild()
            ev.done = False
            swaps += g.swap_count != before
        if it % 10 == 9:
            oracle_device_state_equal(g, o)
            st = g.device_state()
            assert g._ing_live
            want = np.zeros(64, np.int64)
            for key, v in o_ing.items():
                want[key] = v
            np.testing.assert_array_equal(N(ingested), want)
    st = g.device_state()
    _, acap, dcap = g._ing_layout[:3]
    # the rings wrapped: more documents passed through than they hold (the
    # corpus ring with a swap at every third call; without waiting, fewer
    # swaps and more drops)
    assert st["bad_rows"] == 0
    assert st["docs_in"] > 3 * dcap
    if blocking:
        assert st["docs_in"] - st["docs_dropped"] - st["delta_docs"] > acap
    assert swaps >= 5
    g.blocking_poll = True
    before = g.swap_count
    g.poll_rebuild()
    ev.done = g.swap_count != before
    o.poll_rebuild()
    g.sync_host_state()
    gpu_state_equal(g, o)


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
    docs = [tok[r, :min(int(lengths[r]), s)] for r in rows if lengths[r] > 0]
    if docs:
        o.append_documents(docs)


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
    # -1 is the last row (Python indexing); 16 and -17 are outside
    bad = torch.tensor([0, 16, -1, 3, -17], device=gpu)
    d.harvest_finished(bad, torch.full((5,), 5, device=gpu), tok)
    d.global_index.blocking_poll = True
    d.poll()
    assert d.global_index.ingest_counters["bad_rows"] == 2
    assert d.global_index.ingest_counters["docs_in"] == 7 * 16 + 3


def test_device_harvest_argument_errors(gpu):
    from suffixgpu_amd.global_index import GlobalIndex
    g = GlobalIndex(capacity=1024, delta_capacity=256, k=4, device=gpu)
    tok = torch.zeros((4, 8), dtype=torch.int32, device=gpu)
    r = torch.arange(4, device=gpu)
    with pytest.raises(TypeError):
        g.harvest_device(r.float(), r, tok)
    with pytest.raises(TypeError):
        g.harvest_device(r, r, tok.float())
    with pytest.raises(TypeError):
        g.harvest_device(r, r, tok[0])
    with pytest.raises(ValueError):
        g.harvest_device(r.cpu(), r, tok)
    with pytest.raises(ValueError):
        big = torch.zeros(5000, dtype=torch.int64, device=gpu)
        g.harvest_device(big, big, tok)
    assert int(g.delta_len_t.item()) == 0
    assert N(g.delta)[:4].tolist() == [0, 0, 0, 0]


def test_ingest_active_at_scale_reads_nothing_back(gpu):
    """ingest_active with device slot keys, rows and lengths over 256
    in-flight responses of up to 4096 tokens: 24 calls (chunk 64, overlap
    P + k, every sixth call final) into a 2^20 index with a 2^16 delta,
    polls that query the rebuild without waiting, and no synchronising
    call from the second call on (torch's sync debug mode raises on any;
    every call's lengths and rows were uploaded before).  The oracle runs
    the reference's ingest_active on the same sequence, its rebuilds
    completing at the polls where the GPU's swapped; at the end the index
    state and the per-slot progress equal the oracle's."""
    from oracle.drafter import DrafterOracle
    from suffixgpu_amd import SuffixGPUDrafter
    rng = np.random.default_rng(36)
    kw = dict(k=16, max_pattern_len=32, max_occurrences=32, num_backoff=4,
              enable_global=True, global_capacity=1 << 20,
              delta_capacity=1 << 16)
    d = SuffixGPUDrafter(device=gpu, rebuild_stream=torch.cuda.Stream(gpu),
                         **kw)
    g = d.global_index
    o = DrafterOracle(async_rebuild=True, finish_at_user_poll=True, **kw)
    ev = ScriptedEvent()
    o.global_index.rebuild_event_factory = lambda: ev
    b, s, calls = 256, 4096, 24
    tc = synth.TemplateCorpus(seed=37, n_templates=16)
    resp = np.stack([np.resize(tc.sequence(lo=s, hi=s + 1), s)
                     for _ in range(b)]).astype(I32)
    keys = np.arange(b, dtype=np.int64) * 3  # slots need not be rows
    lens_all = np.zeros((calls, b), np.int64)
    final_at = [c % 6 == 5 for c in range(calls)]
    lens = np.zeros(b, np.int64)
    for c in range(calls):
        lens = np.minimum(lens + rng.integers(0, 300, size=b), s)
        lens_all[c] = lens
        if final_at[c]:
            lens = np.zeros(b, np.int64)
    versions = [np.roll(resp, 7 * v, axis=1) for v in range(calls // 6 + 1)]
    rows_d = T(np.stack(versions), gpu)
    keys_d, lens_d = T(keys, gpu), T(lens_all, gpu)
    torch.cuda.synchronize()
    swaps = 0
    prev = torch.cuda.get_sync_debug_mode()
    try:
        for c in range(calls):
            if c == 1:
                torch.cuda.synchronize()
                torch.cuda.set_sync_debug_mode("error")
            ver = c // 6
            d.ingest_active(keys_d, rows_d[ver], lens_d[c],
                            final=final_at[c], chunk=64)
            before = g.swap_count
            d.poll()
            o.ingest_active([int(x) for x in keys], list(versions[ver]),
                            [int(x) for x in lens_all[c]],
                            final=final_at[c], chunk=64)
            ev.done = g.swap_count != before
            assert not ev.done or o.global_index._rebuild_event is not None
            o.poll()
            ev.done = False
            swaps += g.swap_count != before
    finally:
        torch.cuda.set_sync_debug_mode(prev)
    g.blocking_poll = True
    before = g.swap_count
    d.poll()
    ev.done = g.swap_count != before
    o.poll()
    g.sync_host_state()
    gpu_state_equal(g, o.global_index)
    want = np.zeros(d._ingested_dev.numel(), np.int64)
    for key, v in o._ingested.items():
        want[key] = v
    np.testing.assert_array_equal(N(d._ingested_dev), want)
    assert g.ingest_counters["docs_in"] > 1000 and swaps >= 2
