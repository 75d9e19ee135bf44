"""The drafter at the full sizes of its benchmark workloads, against the
oracle (which sorts its own suffix arrays; nothing the GPU built is handed
to it):

* a 2^22-token template corpus with a half-full 2^16 delta, B=64, S=8192
  (the measured step): index, key rows, one propose_with_update, the
  global query of the same tails, and graph replays of the step;
* suffix-array builds of that 4,193,511-token corpus and of 2^22 uniform
  tokens (V=128256), adaptive and fixed-sequence, plus the corpus
  snapshot rebuilt in the background while local-only B=64 S=8192 steps
  run on the main stream, swapped in, and stepped again;
* the B=256, S=16384 decode loop: 70 captured steps with the step-63
  harvest of 16 rows, background rebuilds and swaps (blocking poll), the
  oracle stepping every update and the full step on chosen steps.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from oracle import sa as osa
from oracle.drafter import DrafterOracle
from suffixgpu_amd import synth
from tests.conftest import keys_by_definition

pytestmark = pytest.mark.gpu

I32 = np.int32
CFG = dict(k=16, max_pattern_len=32, max_occurrences=128, num_backoff=8,
           max_spec_factor=2.0, min_token_prob=0.1)
N22 = 1 << 22
D16 = 1 << 16


def T(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def N(t):
    return t.cpu().numpy()


def index_equal(gi, og) -> None:
    assert gi.active_len == og.active_len
    assert gi.delta_len == og.delta_len
    assert list(gi.active_doc_lens) == list(og.active_doc_lens)
    assert list(gi.delta_doc_lens) == list(og.delta_doc_lens)
    np.testing.assert_array_equal(N(gi.corpus), og.corpus)
    np.testing.assert_array_equal(N(gi.sa), og.sa)
    np.testing.assert_array_equal(N(gi.delta)[:gi.delta_len],
                                  og.delta[:og.delta_len])
    assert int(gi.delta_len_t.item()) == gi.delta_len
    gi.poll_tables(wait=True)  # rows of a swap built on the rebuild stream
    keys_by_definition(gi.corpus, gi.sa, gi.sa_key)


# ------------------------------------------------------------ 2^22 corpus
@pytest.fixture(scope="module")
def c3(gpu):
    """The template workload, the oracle's index over it, and the GPU
    drafter loaded with the same documents (rebuild stream attached,
    rebuilds held off until a test asks for one)."""
    from suffixgpu_amd import SuffixGPUDrafter
    w = synth.global_corpus(seed=3, capacity=N22, delta_fill=1 << 15,
                            n_docs=1024, b=64, s=8192)
    kw = dict(enable_global=True, global_capacity=N22, delta_capacity=D16,
              rebuild_threshold=1 << 30, **CFG)
    o = DrafterOracle(**kw)
    o.global_index.load_documents(w.active_docs)
    o.global_index.append_documents(w.delta_docs)
    side = torch.cuda.Stream(gpu)
    d = SuffixGPUDrafter(device=gpu, rebuild_stream=side, **kw)
    d.global_index.blocking_poll = True
    d.global_index.load_documents([T(x, gpu) for x in w.active_docs])
    d.global_index.append_documents([T(x, gpu) for x in w.delta_docs])
    torch.cuda.synchronize()
    return w, o, d


def test_c3_index_matches_oracle(c3):
    """Corpus, suffix array (4,193,511 sorted positions + identity tail),
    delta and key rows of the 2^22 index."""
    w, o, d = c3
    gi, og = d.global_index, o.global_index
    assert gi.active_len == sum(len(x) + 1 for x in w.active_docs)
    assert gi.active_len + 1 == 4_193_511
    index_equal(gi, og)


def _c3_step_check(w, o, d, gpu):
    bt = w.batch
    tg = T(bt.tokens, gpu)
    draft, nv, new = d.propose_with_update(T(bt.num_tokens, gpu), tg,
                                           T(bt.sampled, gpu))
    to = bt.tokens.copy()
    ed, env, enew = o.propose_with_update(bt.num_tokens, to, bt.sampled)
    np.testing.assert_array_equal(N(tg), to)
    np.testing.assert_array_equal(N(new), enew)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)
    return tg, to, enew, env


def test_c3_step_matches_oracle(c3, gpu):
    """One B=64, S=8192 propose_with_update with global memory on, the
    query of the same tails (SA + delta lengths, continuations and
    occurrence counts per cap), and three graph replays of the step."""
    from oracle.local import gather_tails
    w, o, d = c3
    tg, to, enew, env = _c3_step_check(w, o, d, gpu)
    assert (env > 0).sum() >= 48
    tails, tl = gather_tails(enew, to, 32)
    caps = np.asarray(o._global_caps)
    got = d.global_index._query_backoff(T(tails.astype(I32), gpu),
                                        T(tl.astype(np.int64), gpu), 32,
                                        T(caps, gpu))
    exp = o.global_index._query_backoff(tails.astype(I32), tl, 32, caps)
    for a, e in zip(got, exp):
        np.testing.assert_array_equal(N(a), e)
    # the step as the benchmark replays it
    bt = w.batch
    tok = T(bt.tokens, gpu)
    nt = T(bt.num_tokens, gpu)
    samp = T(bt.sampled, gpu)
    for _ in range(2):
        d.propose_with_update(nt, tok, samp)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = d.propose_with_update(nt, tok, samp)
    for _ in range(3):
        tok.copy_(T(bt.tokens, gpu))
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(N(out[0]), N(d.propose_with_update(
            nt, T(bt.tokens, gpu), samp)[0]))
        np.testing.assert_array_equal(N(out[1]), env)
        np.testing.assert_array_equal(N(tok), to)


# ------------------------------------------------------------ SA builds
def test_c4_from_scratch_builds(c3, gpu):
    """The 4,193,511-token corpus and 2^22 uniform tokens, built from
    scratch by the adaptive and the fixed-sequence form, against the
    oracle's own builds; key rows of the uniform build by definition, and
    the compact first-four-token array beside them."""
    from suffixgpu_amd.suffix_array import build_suffix_array_into
    from suffixgpu_amd.global_index import PAD_TOKEN
    w, o, d = c3
    og = o.global_index
    m = og.active_len + 1
    text = torch.full((N22,), PAD_TOKEN, dtype=torch.int32, device=gpu)
    text[:og.active_len].copy_(T(og.corpus[:og.active_len], gpu))
    out = torch.empty(N22, dtype=torch.int32, device=gpu)
    for adaptive in (True, False):
        out.fill_(-7)
        build_suffix_array_into(text, m, out, adaptive=adaptive)
        np.testing.assert_array_equal(N(out), og.sa)
    rng = np.random.default_rng(4)
    uni = rng.integers(0, synth.VOCAB_LARGE, size=N22).astype(I32)
    exp = osa.build_suffix_array(uni).astype(I32)
    tu = T(uni, gpu)
    for adaptive in (True, False):
        out.fill_(-7)
        build_suffix_array_into(tu, N22, out, adaptive=adaptive)
        np.testing.assert_array_equal(N(out), exp)
    from suffixgpu_amd import _lib
    keys = torch.empty(N22 * 32, dtype=torch.int32, device=gpu)
    first4 = torch.empty(N22 * 4, dtype=torch.int32, device=gpu)
    _lib.check(_lib.lib().sfx_sa_keys(tu.data_ptr(), out.data_ptr(), N22,
                                      N22, 32, keys.data_ptr(),
                                      first4.data_ptr(),
                                      _lib.stream_of(gpu)), "keys")
    keys_by_definition(tu, out, keys)
    # the compact first-token output of the same launch
    assert torch.equal(first4.view(N22, 4), keys.view(N22, 32)[:, :4])


def test_c2_b64_local_matches_oracle(gpu):
    """Local-only propose_with_update and propose at B=64, S=8192."""
    from suffixgpu_amd import SuffixGPUDrafter
    w = synth.local_zipf(seed=2, b=64, s=8192)
    d = SuffixGPUDrafter(device=gpu, **CFG)
    o = DrafterOracle(**CFG)
    tg = T(w.tokens, gpu)
    draft, nv, new = d.propose_with_update(T(w.num_tokens, gpu), tg,
                                           T(w.sampled, gpu))
    to = w.tokens.copy()
    ed, env, enew = o.propose_with_update(w.num_tokens, to, w.sampled)
    np.testing.assert_array_equal(N(tg), to)
    np.testing.assert_array_equal(N(new), enew)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)
    draft, nv = d.propose(new, tg)
    ed, env = o.propose(enew, to)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)


def test_c4_steps_overlap_the_background_rebuild(c3, gpu):
    """The snapshot rebuild of the 2^22 index (oldest documents evicted so
    that the corpus and the delta's whole documents fit) on the rebuild
    stream, with global-on B=64 S=8192 steps of the rebuilding drafter
    itself on another stream meanwhile -- 40 replays of the captured step
    and 4 eager calls, no poll in between -- each equal to the oracle's
    step on the index as it stands before the swap (the snapshot staged,
    the delta compacted).  HIP events on both streams show the replays ran
    while the build did.  Then the swap, the index against the oracle's,
    and a step on the new index.  Runs last on the shared index: it
    changes it."""
    w, o, d = c3
    o = copy.deepcopy(o)
    gi, og = d.global_index, o.global_index
    bt = w.batch
    tok = T(bt.tokens, gpu)
    nt, samp = T(bt.num_tokens, gpu), T(bt.sampled, gpu)
    d.propose_with_update(nt, tok, samp)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = d.propose_with_update(nt, tok, samp)
    torch.cuda.synchronize()
    # HIP maps streams onto a few hardware queues, and two streams on one
    # queue run one after the other: the steps and the build get a fresh
    # pair of streams, created one after the other (different queues).
    side = torch.cuda.Stream(gpu)
    run = torch.cuda.Stream(gpu)
    gi.rebuild_stream = side
    with torch.cuda.stream(side):  # the streams' first use
        torch.zeros(1, device=gpu)
    with torch.cuda.stream(run):  # and the eager step's workspace on `run`
        d.propose_with_update(nt, tok.clone(), samp)
    torch.cuda.synchronize()
    gi.rebuild_threshold = og.rebuild_threshold = 1
    gi.blocking_poll = False
    outs, ends = [], []
    with torch.cuda.stream(run):
        # The build waits for the staging copies on `run`; holding `run`
        # first (about 20 ms) lets the host enqueue the rebuild and every
        # step below before any of it runs, so the steps start with the
        # build however long the host takes to enqueue them.
        t0 = torch.cuda.Event(enable_timing=True)
        t0.record(run)
        torch.cuda._sleep(40_000_000)
        gi.maybe_rebuild()
        assert gi._rebuild_event is not None
        side_end = torch.cuda.Event(enable_timing=True)
        side_end.record(side)
        for i in range(44):
            if i % 11 == 10:  # an eager call
                res = d.propose_with_update(nt, tok, samp)
            else:
                graph.replay()
                res = out
            outs.append([t.clone() for t in res])
            e = torch.cuda.Event(enable_timing=True)
            e.record(run)
            ends.append(e)
    side_end.synchronize()
    run.synchronize()
    # steps that ended before the build did ran beside it: the build was
    # enqueued, behind the staging copies, before them all
    overlapped = sum(e.elapsed_time(side_end) > 0 for e in ends)
    assert overlapped >= 8, (overlapped, t0.elapsed_time(side_end),
                             [round(t0.elapsed_time(e), 3) for e in ends])
    og.async_rebuild = True
    og.maybe_rebuild()  # staged: pending until the oracle's next poll
    assert og._rebuild_event is not None
    to = bt.tokens.copy()
    ed, env, enew = o.propose_with_update(bt.num_tokens, to, bt.sampled)
    assert (env > 0).sum() >= 48
    for i, got in enumerate(outs):
        for a, e in zip(got, (ed, env, enew)):
            np.testing.assert_array_equal(N(a), e, err_msg=f"step {i}")
    np.testing.assert_array_equal(N(tok), to)
    gi.blocking_poll = True
    gi.poll_rebuild()
    og.poll_rebuild()
    torch.cuda.synchronize()
    assert gi._rebuild_event is None and og._rebuild_event is None
    index_equal(gi, og)
    assert gi.active_len + gi.delta_len > 0 and gi.delta_len == 0
    gi.rebuild_threshold = og.rebuild_threshold = 1 << 30
    _c3_step_check(w, o, d, gpu)


# ------------------------------------------------------------ decode loop
C5_CHECK = (0, 1, 2, 3, 62, 63, 64, 65, 69)


@pytest.mark.parametrize("device_harvest", [False, True])
def test_c5_decode_loop_matches_oracle(gpu, device_harvest):
    """B=256, S=16384: 70 replays of a captured propose_with_update with
    the sampled block and counts fed back on the device, the step-63
    harvest of the 16 longest rows into global memory (background
    rebuilds at delta_capacity/2, blocking poll every step) and the rows
    reset; new counts every step, the full step and token rows on the
    chosen steps, and the index after the harvest.  device_harvest: the
    rows and lengths are device tensors (device-side ingest; the oracle's
    rebuilds then finish at the caller's poll)."""
    from suffixgpu_amd import SuffixGPUDrafter
    steps = 70
    lp = synth.decode_loop(seed=5, b=256, s=16384, steps=steps)
    assert 63 in lp.harvests
    kw = dict(enable_global=True, global_capacity=N22, delta_capacity=D16,
              rebuild_threshold=D16 // 2, **CFG)
    side = torch.cuda.Stream(gpu)
    d = SuffixGPUDrafter(device=gpu, rebuild_stream=side, **kw)
    gi = d.global_index
    gi.blocking_poll = True
    o = DrafterOracle(async_rebuild=True, finish_at_user_poll=device_harvest,
                      **kw)
    tok = T(lp.tokens, gpu)
    nt = T(lp.num_tokens, gpu)
    samp_all = T(lp.sampled, gpu)
    samp = samp_all[0].clone()
    for _ in range(3):
        d.propose_with_update(nt, tok, samp)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = d.propose_with_update(nt, tok, samp)
    torch.cuda.synchronize()
    to = lp.tokens.copy()
    ont = lp.num_tokens.copy()
    swaps = 0
    for i in range(steps):
        samp.copy_(samp_all[i])
        graph.replay()
        nt.copy_(out[2])
        if i in C5_CHECK:
            ed, env, enew = o.propose_with_update(ont, to, lp.sampled[i])
            torch.cuda.synchronize()
            np.testing.assert_array_equal(N(out[0]), ed, err_msg=f"step {i}")
            np.testing.assert_array_equal(N(out[1]), env, err_msg=f"step {i}")
            np.testing.assert_array_equal(N(tok), to, err_msg=f"step {i}")
        else:
            enew = o.update_state(ont, to, lp.sampled[i])
        np.testing.assert_array_equal(N(out[2]), enew, err_msg=f"step {i}")
        ont = enew
        hv = lp.harvests.get(i)
        before = gi.active_len
        if hv is not None:
            rows, lengths, new_rows, new_q = hv
            idx = torch.tensor(rows, dtype=torch.int64, device=gpu)
            if device_harvest:
                d.harvest_finished(idx, T(np.asarray(lengths), gpu), tok)
            else:
                d.harvest_finished(rows, lengths, tok)
            o.harvest_finished(rows, lengths, to)
            tok.index_copy_(0, idx, T(new_rows, gpu))
            nt.index_copy_(0, idx, T(new_q, gpu))
            to[rows] = new_rows
            ont = ont.copy()
            ont[rows] = new_q
        d.poll()
        o.poll()
        swaps += int(gi.active_len != before)
        if hv is not None:
            torch.cuda.synchronize()
            gi.sync_host_state()
            index_equal(gi, o.global_index)
    assert swaps >= 1 and gi.active_len > 0


def test_c5_nonblocking_loop_follows_gpu_swaps(gpu):
    """B=256, S=16384: 200 replays of the captured step with device-side
    harvests of the 16 longest rows at steps 63, 127 and 191, and a poll
    every step that queries the rebuild's event without waiting (the
    reference's poll_rebuild): rebuilds run on the side stream while the
    steps replay, and swap in at whichever poll finds them done.  The
    oracle's rebuilds complete at the polls where the GPU's swapped.  New
    counts every step; the full step and token rows right after every
    harvest (while its snapshot is staged or building) and every swap,
    and at the first and last step; the device bookkeeping and buffers
    after every harvest and every swap."""
    from suffixgpu_amd import SuffixGPUDrafter
    from tests.test_gpu_ingest import oracle_device_state_equal
    from tests.test_oracle_golden import ScriptedEvent
    steps = 200
    lp = synth.decode_loop(seed=5, b=256, s=16384, steps=steps)
    assert sorted(lp.harvests) == [63, 127, 191]
    kw = dict(enable_global=True, global_capacity=N22, delta_capacity=D16,
              rebuild_threshold=D16 // 2, **CFG)
    d = SuffixGPUDrafter(device=gpu, rebuild_stream=torch.cuda.Stream(gpu),
                         **kw)
    gi = d.global_index
    assert not gi.blocking_poll
    o = DrafterOracle(async_rebuild=True, finish_at_user_poll=True, **kw)
    og = o.global_index
    ev = ScriptedEvent()
    og.rebuild_event_factory = lambda: ev
    tok = T(lp.tokens, gpu)
    nt = T(lp.num_tokens, gpu)
    samp_all = T(lp.sampled, gpu)
    samp = samp_all[0].clone()
    for _ in range(3):
        d.propose_with_update(nt, tok, samp)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = d.propose_with_update(nt, tok, samp)
    torch.cuda.synchronize()
    to = lp.tokens.copy()
    ont = lp.num_tokens.copy()
    swap_polls, full_in_flight = [], 0
    check_next = {0, steps - 1}
    for i in range(steps):
        samp.copy_(samp_all[i])
        graph.replay()
        nt.copy_(out[2])
        if i in check_next:
            in_flight = og._rebuild_event is not None
            ed, env, enew = o.propose_with_update(ont, to, lp.sampled[i])
            np.testing.assert_array_equal(N(out[0]), ed, err_msg=f"step {i}")
            np.testing.assert_array_equal(N(out[1]), env, err_msg=f"step {i}")
            np.testing.assert_array_equal(N(tok), to, err_msg=f"step {i}")
            full_in_flight += in_flight
        else:
            enew = o.update_state(ont, to, lp.sampled[i])
        np.testing.assert_array_equal(N(out[2]), enew, err_msg=f"step {i}")
        ont = enew
        hv = lp.harvests.get(i)
        if hv is not None:
            rows, lengths, new_rows, new_q = hv
            idx = torch.tensor(rows, dtype=torch.int64, device=gpu)
            d.harvest_finished(idx, T(np.asarray(lengths), gpu), tok)
            o.harvest_finished(rows, lengths, to)
            assert og._rebuild_event is not None  # a snapshot is staged
            oracle_device_state_equal(gi, og)
            tok.index_copy_(0, idx, T(new_rows, gpu))
            nt.index_copy_(0, idx, T(new_q, gpu))
            to[rows] = new_rows
            ont = ont.copy()
            ont[rows] = new_q
            check_next.update((i + 1, i + 2, i + 3))
        before = gi.swap_count
        d.poll()
        ev.done = gi.swap_count != before
        assert not ev.done or og._rebuild_event is not None, f"poll {i}"
        o.poll()
        ev.done = False
        if gi.swap_count != before:
            swap_polls.append(i)
            assert og._rebuild_event is None
            oracle_device_state_equal(gi, og)
            check_next.add(i + 1)
    print(f"swaps at polls {swap_polls}; full steps checked {len(check_next)},"
          f" {full_in_flight} with a rebuild staged or running")
    assert len(swap_polls) >= 2
    assert full_in_flight >= 3
    assert gi.active_len > 0
