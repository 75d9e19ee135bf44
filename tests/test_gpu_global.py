"""Global index on gfx950 vs the oracle and the reference's goldens/KATs:
write path state machine (append, rebuild, eviction, compaction, in-flight
drops), SA rebuild, capped SA + delta queries, merge and draft."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import naive
from oracle.global_index import GlobalIndexOracle
from suffixgpu_amd import synth
from tests.conftest import golden, keys_by_definition
from tests.test_oracle_golden import _docs, trace_ops

pytestmark = pytest.mark.gpu

I32 = np.int32


def T(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def N(t):
    return t.cpu().numpy()


def key_arrays_equal(gi):
    """Key rows are the suffixes' first 32 tokens by rank, -1 past the end
    of the corpus (an index without search tables has none)."""
    if gi.sa_key is None:
        assert not gi.search_tables
        return
    gi.poll_tables(wait=True)  # rows of a swap built on the rebuild stream
    assert not gi.tables_pending
    corpus, sa = N(gi.corpus), N(gi.sa).astype(np.int64)
    n, kw = corpus.shape[0], 32
    pos = sa[:, None] + np.arange(kw)[None, :]
    want = np.where(pos < n, corpus[np.minimum(pos, n - 1)], -1)
    np.testing.assert_array_equal(N(gi.sa_key).reshape(n, kw), want)


def gpu_state_equal(gi, ref):
    """ref: oracle index or a dict of golden arrays."""
    key_arrays_equal(gi)
    if isinstance(ref, dict):
        g = ref
        assert gi.active_len == int(g["active_len"])
        assert gi.delta_len == int(g["delta_len"])
        assert list(gi.active_doc_lens) == g["active_doc_lens"].tolist()
        assert list(gi.delta_doc_lens) == g["delta_doc_lens"].tolist()
        np.testing.assert_array_equal(N(gi.corpus), g["corpus"])
        np.testing.assert_array_equal(N(gi.sa), g["sa"])
        np.testing.assert_array_equal(N(gi.delta)[:gi.delta_len], g["delta"])
        assert int(gi.delta_len_t.item()) == gi.delta_len
        return
    assert gi.active_len == ref.active_len
    assert gi.delta_len == ref.delta_len
    assert list(gi.active_doc_lens) == list(ref.active_doc_lens)
    assert list(gi.delta_doc_lens) == list(ref.delta_doc_lens)
    np.testing.assert_array_equal(N(gi.corpus), ref.corpus)
    np.testing.assert_array_equal(N(gi.sa), ref.sa)
    np.testing.assert_array_equal(N(gi.delta)[:gi.delta_len],
                                  ref.delta[:ref.delta_len])


def _sub(z, suffix):
    return {k: z[k + suffix] for k in ("active_len", "delta_len",
                                       "active_doc_lens", "delta_doc_lens",
                                       "corpus", "sa", "delta")}


class _NeverDone:
    def query(self) -> bool:
        return False


def test_index_trace_golden(gpu):
    from suffixgpu_amd.global_index import GlobalIndex
    z = golden("index_trace")
    gi = GlobalIndex(capacity=96, delta_capacity=40, k=4, max_occurrences=8,
                     rebuild_threshold=25, device=gpu)
    for step, docs, infl in trace_ops(z):
        if infl and gi._rebuild_event is None:
            gi._rebuild_event = _NeverDone()
            gi._pending = (gi.active_len, gi.active_doc_lens)
        gi.append_documents([T(d, gpu) for d in docs])
        if step in (14, 27):
            gi._rebuild_event = None
            gi._pending = None
        gpu_state_equal(gi, _sub(z, f"_{step}"))


def _ties_index(gpu):
    from suffixgpu_amd import SuffixGPUDrafter
    z = golden("global_ties")
    docs = _docs(z)
    d = SuffixGPUDrafter(k=6, device=gpu, max_pattern_len=10,
                         max_occurrences=8, num_backoff=5, enable_global=True,
                         global_capacity=2048, delta_capacity=300,
                         rebuild_threshold=200)
    d.harvest_rows([T(x, gpu) for x in docs[:20]], [len(x) for x in docs[:20]])
    d.harvest_rows([T(x, gpu) for x in docs[20:]], [len(x) for x in docs[20:]])
    return z, d


def test_global_ties_golden(gpu):
    z, d = _ties_index(gpu)
    gi = d.global_index
    gpu_state_equal(gi, _sub(z, ""))
    q, ql, caps = T(z["query"], gpu), T(z["query_len"], gpu), T(z["caps"], gpu)
    ml, cont, occ = gi._query_backoff(q, ql, 10, caps)
    np.testing.assert_array_equal(N(ml), z["q_len"])
    np.testing.assert_array_equal(N(occ), z["q_occ"])
    np.testing.assert_array_equal(N(cont), z["q_cont"])
    dl, dp, dc = gi._delta_match_backoff(q, ql, 10, caps)
    np.testing.assert_array_equal(N(dl), z["d_len"])
    np.testing.assert_array_equal(N(dp), z["d_pos"])
    np.testing.assert_array_equal(N(dc), z["d_cnt"])
    dr = gi.draft(q, ql, 10, 6, min_token_prob=0.05, max_spec_factor=1.5,
                  max_spec_offset=1.0, caps=caps)
    for g, key in zip(dr, ("dr_chain", "dr_emit", "dr_len", "dr_occ",
                           "dr_score")):
        np.testing.assert_array_equal(N(g), z[key], err_msg=key)
    draft, nv = d.propose(T(z["query_len"].astype(I32), gpu),
                          T(z["rows"], gpu))
    np.testing.assert_array_equal(N(draft), z["draft"])
    np.testing.assert_array_equal(N(nv), z["num_valid"])


@pytest.mark.parametrize("tables", [True, False])
def test_global_drafter_golden(gpu, tables):
    """The reference's drafter trace, with the search tables (key rows and
    n-gram table) and without them."""
    from suffixgpu_amd import SuffixGPUDrafter
    z = golden("global_drafter")
    docs = _docs(z)
    d = SuffixGPUDrafter(k=16, device=gpu, max_pattern_len=32,
                         max_occurrences=128, num_backoff=8,
                         max_spec_factor=2.0, min_token_prob=0.1,
                         enable_global=True, global_capacity=1 << 13,
                         delta_capacity=1 << 10, rebuild_threshold=700,
                         global_search_tables=tables)
    for step, lo in enumerate(range(0, len(docs), 8)):
        chunk = docs[lo:lo + 8]
        d.harvest_rows([T(x, gpu) for x in chunk], [len(x) for x in chunk])
        d.poll()
        tok = T(z["rows"], gpu)
        draft, nv, _ = d.propose_with_update(T(z["num_tokens"], gpu), tok,
                                             T(z["sampled"], gpu))
        np.testing.assert_array_equal(N(draft), z[f"draft_{step}"])
        np.testing.assert_array_equal(N(nv), z[f"nv_{step}"])
        gpu_state_equal(d.global_index, _sub(z, f"_{step}"))


# ---------------------------------------------------------------- KATs
def _query(gi, query, gpu, p=8):
    ml, cont, occ = gi.query(T(np.array([query], I32), gpu),
                             T(np.array([len(query)]), gpu), p)
    chain, nv = gi.expand(cont, occ)
    return (N(chain)[0, :int(nv[0])].tolist(), int(ml[0]), int(occ[0]))


def _gi(gpu, **kw):
    from suffixgpu_amd.global_index import GlobalIndex
    base = dict(capacity=1024, delta_capacity=256, k=4, max_occurrences=8,
                rebuild_threshold=100000, device=gpu)
    base.update(kw)
    return GlobalIndex(**base)


def _append(gi, docs, gpu):
    gi.append_documents([T(np.array(d, I32), gpu) for d in docs])


def test_kat_delta_sa_consistency(gpu):
    doc = [5, 6, 7, 8, 9, 5, 6, 7, 8, 10]
    for thr in (100000, 1):
        gi = _gi(gpu, rebuild_threshold=thr)
        _append(gi, [doc], gpu)
        if thr == 1:
            assert gi.active_len == len(doc) + 1 and gi.delta_len == 0
        exp_chain, exp_len = naive.global_chain([doc], [5, 6, 7, 8], 4, 8, 8)
        assert _query(gi, [5, 6, 7, 8], gpu) == (exp_chain, exp_len, 2)
    docs = [[1, 2, 3, 4, 1, 2, 3, 9], [7, 1, 2, 3, 4, 8, 1, 2]]
    res = []
    for thr in (100000, 1):
        gi = _gi(gpu, rebuild_threshold=thr)
        _append(gi, docs, gpu)
        res.append(_query(gi, [1, 2, 3, 4], gpu)[:2])
    assert res[0] == res[1] == naive.global_chain(docs, [1, 2, 3, 4], 4, 8, 8)


def test_kat_rebuilds_eviction_empty(gpu):
    gi = _gi(gpu, rebuild_threshold=1)
    docs = [[1, 1, 2], [1, 1, 3], [1, 1, 4], [1, 1, 5]]
    for d in docs:
        _append(gi, [d], gpu)
    assert gi.active_len == sum(len(d) + 1 for d in docs)
    assert _query(gi, [1, 1], gpu)[:2] == naive.global_chain(docs, [1, 1], 4,
                                                             8, 8)
    gi = _gi(gpu, capacity=12, delta_capacity=64, rebuild_threshold=1)
    for t in (1, 2, 3, 4):
        _append(gi, [[t] * 4], gpu)
    assert gi.active_len <= 12
    assert _query(gi, [4, 4], gpu)[1] == 2
    assert _query(gi, [1, 1, 1, 1], gpu)[1] == 0
    gi = _gi(gpu, capacity=64, delta_capacity=16, rebuild_threshold=None)
    assert _query(gi, [1, 2, 3], gpu) == ([], 0, 0)


def test_kat_regressions(gpu):
    gi = _gi(gpu)
    doc = [9, 7, 7, 101, 5, 5, 5, 5, 5, 3, 7, 7, 101, 6, 6, 6, 6, 6, 6, 7, 7,
           101, 4]
    _append(gi, [doc], gpu)
    dl, dp, dc = gi._delta_match_backoff(
        T(np.array([[7, 7] + [0] * 6], I32), gpu), T(np.array([2]), gpu), 8,
        T(np.array([8]), gpu))
    assert int(dl[0, 0]) == 2 and int(dc[0, 0]) == 3
    assert N(dp)[0, 0, :3].tolist() == [1, 10, 19]
    chain, ml, occ = _query(gi, [7, 7], gpu)
    assert (ml, occ, chain[0]) == (2, 3, 101)
    gi = _gi(gpu, max_occurrences=4)
    _append(gi, [[1, 9] * 10 + [1, 2, 3, 4, 6]], gpu)
    assert _query(gi, [1, 2, 3, 4], gpu) == ([6], 4, 1)


def test_kat_overflow(gpu):
    gi = _gi(gpu, capacity=64, delta_capacity=18)
    _append(gi, [[1] * 6, [2] * 6], gpu)
    gi._rebuild_event = _NeverDone()
    gi._pending = (gi.active_len, gi.active_doc_lens)
    _append(gi, [[3] * 10], gpu)
    assert gi.delta_len <= gi.delta_capacity
    assert _query(gi, [3, 3], gpu)[1] == 2
    assert _query(gi, [2, 2], gpu)[1] == 2
    assert _query(gi, [1, 1], gpu)[1] == 0
    gi._rebuild_event = None
    gi._pending = None
    gi = _gi(gpu, capacity=64, delta_capacity=16)
    _append(gi, [[1] * 12], gpu)
    _append(gi, [[2] * 12], gpu)
    assert gi.active_len == 13 and gi.delta_len == 13
    assert _query(gi, [1, 1], gpu)[1] == 2
    assert _query(gi, [2, 2], gpu)[1] == 2


def test_kat_no_cross_document(gpu):
    for thr in (100000, 1):
        gi = _gi(gpu, capacity=256, delta_capacity=64, rebuild_threshold=thr)
        _append(gi, [[1, 2, 3, 7, 8, 9], [100, 101, 102, 55, 56]], gpu)
        assert _query(gi, [7, 8, 9], gpu) == ([], 3, 1)
        assert _query(gi, [8, 9, 100], gpu) == ([101, 102, 55, 56], 1, 1)


# ------------------------------------------------------ random vs oracle
def _load_pair(gpu, docs, delta_docs, cap, dcap, r, k=16, delta_index=True):
    from suffixgpu_amd.global_index import GlobalIndex
    g = GlobalIndex(capacity=cap, delta_capacity=dcap, k=k,
                    max_occurrences=r, rebuild_threshold=10 ** 9, device=gpu,
                    delta_index=delta_index)
    o = GlobalIndexOracle(capacity=cap, delta_capacity=dcap, k=k,
                          max_occurrences=r, rebuild_threshold=10 ** 9)
    g.load_documents([T(d, gpu) for d in docs])
    o.load_documents(docs)
    g.append_documents([T(d, gpu) for d in delta_docs])
    o.append_documents(delta_docs)
    gpu_state_equal(g, o)
    return g, o


@pytest.mark.parametrize("kind", ["periodic", "runs"])
def test_sa_interval_search_long_repeats(gpu, kind):
    """The key-row k-ary search (32-token rows, lower and upper bounds that
    share probes until they split) on texts whose suffixes share long
    prefixes: wide intervals at every length, matches past the row."""
    from suffixgpu_amd.sa_search import suffix_match_backoff
    from oracle.sa import suffix_match_backoff as o_smb
    rng = np.random.default_rng(77 if kind == "periodic" else 78)
    if kind == "periodic":
        docs = [np.tile(np.array([3, 1, 4, 1, 5], I32), 400)[:int(n)]
                for n in rng.integers(50, 2000, size=12)]
        docs += [rng.integers(0, 6, size=300).astype(I32) for _ in range(4)]
    else:
        docs = [np.repeat(rng.integers(0, 3, size=60), rng.integers(1, 40,
                                                              size=60))
                .astype(I32) for _ in range(16)]
    cap = sum(len(d) + 1 for d in docs) + 5
    g, o = _load_pair(gpu, docs, [], cap, 64, 16, k=4)
    b, p = 64, 32
    q = np.zeros((b, p), I32)
    ql = np.zeros(b, np.int64)
    for i in range(b):
        src = docs[i % len(docs)]
        n = int(rng.integers(1, min(len(src), p) + 1))
        st = int(rng.integers(0, len(src) - n + 1))
        q[i, :n] = src[st:st + n]
        ql[i] = n
        if i % 9 == 0 and n > 2:
            q[i, n - 1] = 9  # diverges at the last token
    caps = np.array([32, 16, 8, 4, 2], np.int64)
    tq, tl, tc_ = T(q, gpu), T(ql, gpu), T(caps, gpu)
    for got, exp in zip(suffix_match_backoff(g.sa, g.corpus, tq, tl, p, tc_),
                        o_smb(o.sa, o.corpus, q, ql, p, caps)):
        np.testing.assert_array_equal(N(got), exp)
    for got, exp in zip(g._query_backoff(tq, tl, p, tc_),
                        o._query_backoff(q, ql, p, caps)):
        np.testing.assert_array_equal(N(got), exp)


@pytest.mark.parametrize("vocab", [4, 0])
def test_queries_vs_oracle(gpu, vocab):
    rng = np.random.default_rng(31 + vocab)
    if vocab:
        docs = [rng.integers(0, vocab, size=int(rng.integers(1, 200))).astype(
            I32) for _ in range(60)]
        dd = [rng.integers(0, vocab, size=int(rng.integers(1, 90))).astype(I32)
              for _ in range(6)]
    else:
        tc = synth.TemplateCorpus(seed=5, n_templates=12)
        docs = [tc.sequence(lo=64, hi=500) for _ in range(40)]
        dd = [tc.sequence(lo=64, hi=300) for _ in range(4)]
    cap = sum(len(d) + 1 for d in docs) + 37
    g, o = _load_pair(gpu, docs, dd, cap, 2048, 16, k=8)
    b, p = 48, 12
    q = np.zeros((b, p), I32)
    ql = np.zeros(b, np.int64)
    for i in range(b):
        src = docs[i % len(docs)] if i % 3 else dd[i % len(dd)]
        n = int(rng.integers(0, min(len(src), p) + 1))
        st = int(rng.integers(0, len(src) - n + 1))
        q[i, :n] = src[st:st + n]
        ql[i] = n
        if i % 7 == 0:
            q[i, :n] = rng.integers(0, max(vocab, 50), size=n)
    ql[0] = 0
    ql[1] = p + 5   # longer than the query width: clamped gathers
    caps = np.array([12, 6, 3, 2], np.int64)
    tq, tl, tc_ = T(q, gpu), T(ql, gpu), T(caps, gpu)
    for got, exp in zip(g._query_backoff(tq, tl, p, tc_),
                        o._query_backoff(q, ql, p, caps)):
        np.testing.assert_array_equal(N(got), exp)
    for got, exp in zip(g._delta_match_backoff(tq, tl, p, tc_),
                        o._delta_match_backoff(q, ql, p, caps)):
        np.testing.assert_array_equal(N(got), exp)
    for got, exp in zip(g.draft(tq, tl, p, 8, min_token_prob=0.05,
                                max_spec_factor=0.7, max_spec_offset=0.3,
                                caps=tc_, alpha=0.25),
                        o.draft(q, ql, p, 8, min_token_prob=0.05,
                                max_spec_factor=0.7, max_spec_offset=0.3,
                                caps=caps, alpha=0.25)):
        np.testing.assert_array_equal(N(got), exp)
    from suffixgpu_amd.sa_search import suffix_match_backoff
    from oracle.sa import suffix_match_backoff as o_smb
    for got, exp in zip(suffix_match_backoff(g.sa, g.corpus, tq, tl, p, tc_),
                        o_smb(o.sa, o.corpus, q, ql, p, caps)):
        np.testing.assert_array_equal(N(got), exp)


@pytest.mark.parametrize("delta_index", [False, True])
@pytest.mark.parametrize("mode", ["small_vocab", "templates", "short"])
def test_split_delta_vs_oracle(gpu, mode, delta_index):
    """A 2^16-token delta, without the delta token index, is scanned by
    several workgroups per row; their lists are combined in part order.
    Queries whose longest delta match lies in a late part exercise the
    per-part threshold check.  With the index each row visits its newest
    token's bucket (over a 5-token vocabulary: buckets of thousands of
    positions, longer than the LDS chunk)."""
    rng = np.random.default_rng({"small_vocab": 1, "templates": 2,
                                 "short": 3}[mode])
    tc = synth.TemplateCorpus(seed=9, n_templates=10)
    docs = [tc.sequence(lo=64, hi=400) for _ in range(30)]
    if mode == "small_vocab":
        dd = [rng.integers(0, 5, size=int(rng.integers(200, 4000))).astype(I32)
              for _ in range(14)]
    elif mode == "templates":
        dd = [tc.sequence(lo=1024, hi=6000) for _ in range(10)]
    else:
        dd = [tc.sequence(lo=20, hi=60) for _ in range(2)]
    cap = sum(len(d) + 1 for d in docs) + 11
    g, o = _load_pair(gpu, docs, dd, cap, 1 << 16, 32, k=8,
                      delta_index=delta_index)
    assert g.delta_len == o.delta_len
    assert (g.delta_buckets > 0) == delta_index
    b, p = 40, 24
    q = np.zeros((b, p), I32)
    ql = np.zeros(b, np.int64)
    for i in range(b):
        # late delta docs first: their longest matches sit in the last parts
        src = dd[-1 - (i % len(dd))] if i % 4 else docs[i % len(docs)]
        n = int(rng.integers(1, min(len(src), p) + 1))
        st = int(rng.integers(0, len(src) - n + 1))
        q[i, :n] = src[st:st + n]
        ql[i] = n
    caps = np.array([24, 12, 6, 3, 2], np.int64)
    tq, tl, tc_ = T(q, gpu), T(ql, gpu), T(caps, gpu)
    for got, exp in zip(g._delta_match_backoff(tq, tl, p, tc_),
                        o._delta_match_backoff(q, ql, p, caps)):
        np.testing.assert_array_equal(N(got), exp)
    for got, exp in zip(g._query_backoff(tq, tl, p, tc_),
                        o._query_backoff(q, ql, p, caps)):
        np.testing.assert_array_equal(N(got), exp)
    for got, exp in zip(g.draft(tq, tl, p, 8, min_token_prob=0.05,
                                caps=tc_),
                        o.draft(q, ql, p, 8, min_token_prob=0.05,
                                caps=caps)):
        np.testing.assert_array_equal(N(got), exp)


def delta_bucket(t, hbits):
    """The index's bucket of token t (Fibonacci hashing of its 32 bits)."""
    return ((int(t) & 0xFFFFFFFF) * 0x9E3779B1 & 0xFFFFFFFF) >> (32 - hbits)


def check_delta_index(g):
    """The delta token index of g by its definition: bucket b lists the
    positions p < delta_len with delta_bucket(delta[p]) == b, ascending,
    each with the tokens x(p), x(p - 1), x(p - 2) (-1 before position 0);
    the positions from delta_len on follow in order, and start[b] is each
    bucket's first index."""
    hb = g.delta_buckets.bit_length() - 1
    dl = g.delta_len
    delta = N(g.delta)
    ent = N(g._dix_ent).astype(np.int64)
    pos = ent[:, 0]
    padded = np.concatenate([[-1, -1], delta.astype(np.int64)])
    for k in range(3):
        np.testing.assert_array_equal(ent[:, 1 + k], padded[pos + 2 - k])
    start = N(g._dix_start).view(np.uint32).astype(np.int64)
    keys = np.array([delta_bucket(t, hb) for t in delta[:dl]], np.int64)
    order = np.lexsort((np.arange(dl), keys))
    np.testing.assert_array_equal(pos[:dl], order)
    np.testing.assert_array_equal(pos[dl:], np.arange(dl, g.delta_capacity))
    exp = np.searchsorted(keys[order], np.arange(g.delta_buckets + 1),
                          side="left")
    np.testing.assert_array_equal(start, exp)


@pytest.mark.parametrize("kind", ["repeated", "colliding", "edges"])
def test_delta_index_rows_vs_scan(gpu, kind):
    """Queries and drafts through the delta token index equal the delta
    scan's and the oracle's, and the index matches its definition after
    appends and a compaction: a delta of one repeated token (a bucket
    covering the whole delta, compacted in chunks); tokens chosen to share
    one bucket (each row's entries mostly of other tokens); query tails
    holding -1 (end 0 reads x(-1) = -1), separators and padding, and an
    empty delta."""
    from suffixgpu_amd.global_index import GlobalIndex
    rng = np.random.default_rng({"repeated": 31, "colliding": 32,
                                 "edges": 33}[kind])
    tc = synth.TemplateCorpus(seed=19, n_templates=6)
    docs = [tc.sequence(lo=64, hi=300) for _ in range(20)]
    dcap = 1 << 15
    hb = 13  # delta_buckets_for(2^15) = 2^13
    if kind == "repeated":
        dd = [np.full(int(rng.integers(3000, 9000)), 7, I32)
              for _ in range(4)]
        dd.append(np.concatenate([np.full(50, 7, I32),
                                  np.array([3, 7, 7, 9], I32)]))
    elif kind == "colliding":
        pool = [t for t in range(1, 400000)
                if delta_bucket(t, hb) == delta_bucket(11, hb)][:6] + [11]
        assert len(pool) == 7
        dd = [rng.choice(np.array(pool, I32), size=int(rng.integers(500,
                         3000))).astype(I32) for _ in range(8)]
    else:
        dd = [tc.sequence(lo=100, hi=900) for _ in range(6)]
    cap = sum(len(d) + 1 for d in docs) + 11
    pairs = [_load_pair(gpu, docs, dd if kind != "edges" else [], cap, dcap,
                        32, k=8, delta_index=x) for x in (True, False)]
    (gi, o), (gs, _) = pairs
    assert gi.delta_buckets == 1 << hb and gs.delta_buckets == 0
    check_delta_index(gi)
    b, p = 48, 20
    q = np.zeros((b, p), I32)
    ql = np.zeros(b, np.int64)
    src_all = dd if dd else docs
    for i in range(b):
        src = src_all[i % len(src_all)]
        n = int(rng.integers(1, min(len(src), p) + 1))
        st = int(rng.integers(0, len(src) - n + 1))
        q[i, :n] = src[st:st + n]
        ql[i] = n
        if kind == "edges" and i % 3 == 0:
            q[i, n - 1 - int(rng.integers(0, min(n, 3)))] = (-1, -2, PAD)[
                (i // 3) % 3]
        if kind == "edges" and i % 12 == 0:
            q[i, :n] = -1  # a tail of -1s matches before position 0
    caps = np.array([20, 10, 5, 3, 2, 1], np.int64)
    for step in range(2):
        if step == 1:
            # more documents, then drop the oldest: both rebuild the index
            more = [tc.sequence(lo=200, hi=600) for _ in range(3)]
            for g in (gi, gs):
                g.append_documents([T(d, gpu) for d in more])
                g._drop_oldest_docs(1)
            o.append_documents(more)
            o._drop_oldest_docs(1)
            gpu_state_equal(gi, o)
            check_delta_index(gi)
        tq, tl, tc_ = T(q, gpu), T(ql, gpu), T(caps, gpu)
        exp = o._query_backoff(q, ql, p, caps)
        for g in (gi, gs):
            for got, e in zip(g._query_backoff(tq, tl, p, tc_), exp):
                np.testing.assert_array_equal(N(got), e)
        exp = o.draft(q, ql, p, 8, min_token_prob=0.05, caps=caps)
        for g in (gi, gs):
            for got, e in zip(g.draft(tq, tl, p, 8, min_token_prob=0.05,
                                      caps=tc_), exp):
                np.testing.assert_array_equal(N(got), e)


@pytest.mark.parametrize("hint", [12, 1, 3])
def test_async_rebuild_blocking_poll(gpu, hint):
    """Side-stream rebuilds swapped at deterministic points match the
    oracle's done-at-next-poll schedule.  The build runs its doubling
    rounds in two chunks; a small first chunk (hint) forces the second."""
    from suffixgpu_amd.global_index import GlobalIndex
    rng = np.random.default_rng(8)
    side = torch.cuda.Stream(gpu)
    g = GlobalIndex(capacity=3000, delta_capacity=400, k=4,
                    max_occurrences=8, rebuild_threshold=150, device=gpu,
                    rebuild_stream=side)
    g.blocking_poll = True
    g.sa_round_hint = hint
    o = GlobalIndexOracle(capacity=3000, delta_capacity=400, k=4,
                          max_occurrences=8, rebuild_threshold=150,
                          async_rebuild=True)
    for step in range(40):
        docs = [rng.integers(0, 6, size=int(rng.integers(1, 120))).astype(I32)
                for _ in range(int(rng.integers(1, 4)))]
        if hint < 12:
            g.sa_round_hint = hint  # every build starts with a short chunk
        g.append_documents([T(d, gpu) for d in docs])
        o.append_documents(docs)
        if step % 3 == 0:
            g.poll_rebuild()
            o.poll_rebuild()
        assert (g._rebuild_event is None) == (o._rebuild_event is None)
        assert g.delta_len == o.delta_len
        assert list(g.delta_doc_lens) == list(o.delta_doc_lens)
    g.poll_rebuild()
    o.poll_rebuild()
    torch.cuda.synchronize()
    gpu_state_equal(g, o)


def test_queries_while_the_swapped_tables_are_built(gpu):
    """After a background rebuild swaps in, the steps before the next poll
    find the selector set (the swap sets it on their stream) and search
    without key rows and table; the poll after the tables' event clears it.
    Queries and drafts equal the oracle's in both windows, and the rebuilt
    key rows and table equal their definition."""
    from suffixgpu_amd.global_index import GlobalIndex
    rng = np.random.default_rng(41)
    tc = synth.TemplateCorpus(seed=23, n_templates=6)
    side = torch.cuda.Stream(gpu)
    kw = dict(capacity=1 << 15, delta_capacity=1 << 13, k=8,
              max_occurrences=16, rebuild_threshold=1 << 30)
    g = GlobalIndex(device=gpu, rebuild_stream=side, **kw)
    o = GlobalIndexOracle(async_rebuild=True, **kw)
    docs = [tc.sequence(lo=200, hi=600) for _ in range(20)]
    g.load_documents([T(d, gpu) for d in docs])
    o.load_documents(docs)
    dd = [tc.sequence(lo=200, hi=900) for _ in range(8)]
    g.append_documents([T(d, gpu) for d in dd])
    o.append_documents(dd)
    g.rebuild_threshold = o.rebuild_threshold = 1
    g.blocking_poll = True
    g.maybe_rebuild()
    o.maybe_rebuild()
    g.poll_rebuild()  # swaps; the tables are built on `side`
    o.poll_rebuild()
    assert g._rebuild_event is None and o._rebuild_event is None
    assert g.tables_pending and int(g.key_select.item()) == 1
    b, p = 32, 24
    q = np.zeros((b, p), I32)
    ql = np.zeros(b, np.int64)
    src_all = docs + dd
    for i in range(b):
        src = src_all[int(rng.integers(0, len(src_all)))]
        n = int(rng.integers(1, min(len(src), p) + 1))
        st = int(rng.integers(0, len(src) - n + 1))
        q[i, :n] = src[st:st + n]
        ql[i] = n
    caps = np.array([24, 12, 6, 3, 2], np.int64)
    tq, tl, tc_ = T(q, gpu), T(ql, gpu), T(caps, gpu)
    for pending in (True, False):
        if not pending:
            g.poll_rebuild()  # waits for the tables' event, clears the word
            assert not g.tables_pending and int(g.key_select.item()) == 0
        for got, e in zip(g._query_backoff(tq, tl, p, tc_),
                          o._query_backoff(q, ql, p, caps)):
            np.testing.assert_array_equal(N(got), e)
        for got, e in zip(g.draft(tq, tl, p, 8, min_token_prob=0.05,
                                  caps=tc_),
                          o.draft(q, ql, p, 8, min_token_prob=0.05,
                                  caps=caps)):
            np.testing.assert_array_equal(N(got), e)
    gpu_state_equal(g, o)
    kmax, tab = gpu_gram_table(g)
    assert kmax == 4
    assert tab == gram_runs(N(g.corpus), N(g.sa))


@pytest.mark.parametrize("dcap", [400, 4097])
def test_delta_index_at_odd_capacities(gpu, dcap):
    """The delta token index by its definition at a capacity below the
    smallest bucket count (400: 1024 buckets) and one just past a radix
    tile (4097), after appends, a drop and a rebuild's compaction."""
    from suffixgpu_amd.global_index import GlobalIndex
    rng = np.random.default_rng(dcap)
    g = GlobalIndex(capacity=1 << 14, delta_capacity=dcap, k=4,
                    max_occurrences=8, rebuild_threshold=1 << 30,
                    device=gpu)
    for step in range(6):
        docs = [rng.integers(0, 50, size=int(rng.integers(1, dcap // 3)))
                .astype(I32) for _ in range(3)]
        g.append_documents([T(d, gpu) for d in docs])
        torch.cuda.synchronize()
        check_delta_index(g)
        if step == 3:
            g.rebuild_threshold = 1
            g.maybe_rebuild()  # synchronous: the delta is compacted
            g.rebuild_threshold = 1 << 30
            torch.cuda.synchronize()
            check_delta_index(g)


def test_round_hint_follows_the_last_build(gpu):
    """The background rebuild's first chunk of doubling rounds is sized
    from the rounds the previous build needed, with the radix path for the
    rounds that took it: a long exact repeat (one token 6000 times) raises
    the hint past the default; once that document is evicted, a build over
    short-repeat documents lowers it again (the state copy is read even
    when the first chunk held every round)."""
    from suffixgpu_amd.global_index import GlobalIndex
    rng = np.random.default_rng(31)
    side = torch.cuda.Stream(gpu)
    kw = dict(capacity=8000, delta_capacity=7000, k=4, max_occurrences=8,
              rebuild_threshold=4000)
    g = GlobalIndex(device=gpu, rebuild_stream=side, **kw)
    g.blocking_poll = True
    o = GlobalIndexOracle(async_rebuild=True, **kw)
    rep = np.full(6000, 3, I32)
    g.append_documents([T(rep, gpu)])
    o.append_documents([rep])
    g.poll_rebuild()
    o.poll_rebuild()
    gpu_state_equal(g, o)
    high = g.sa_round_hint
    assert high > 12
    # rounds over the repeat's groups of up to 6000 suffixes took the radix
    # path, and the next build enqueues it for them
    assert g.sa_radix_hint & 2
    docs = [rng.integers(0, 1000, size=900).astype(I32) for _ in range(5)]
    g.append_documents([T(d, gpu) for d in docs])
    o.append_documents(docs)
    g.poll_rebuild()
    o.poll_rebuild()
    torch.cuda.synchronize()
    gpu_state_equal(g, o)
    assert list(g.active_doc_lens) == [901] * 5
    assert g.sa_round_hint < 8 < high
    assert g.sa_radix_hint == 0


def test_save_restore_bit_exact(gpu, tmp_path):
    """A saved index restores to the same corpus, SA, delta, key rows and
    host state (into a new index and in place), and answers queries
    bit-exactly; an in-flight rebuild is completed before saving."""
    from suffixgpu_amd.global_index import GlobalIndex
    rng = np.random.default_rng(21)
    side = torch.cuda.Stream(gpu)
    g = GlobalIndex(capacity=5000, delta_capacity=600, k=6,
                    max_occurrences=16, rebuild_threshold=250, device=gpu,
                    rebuild_stream=side)
    # a rebuild swaps in at the next poll, as the oracle's does
    g.blocking_poll = True
    o = GlobalIndexOracle(capacity=5000, delta_capacity=600, k=6,
                          max_occurrences=16, rebuild_threshold=250,
                          async_rebuild=True)
    for _ in range(12):
        docs = [rng.integers(0, 9, size=int(rng.integers(5, 150))).astype(I32)
                for _ in range(3)]
        g.append_documents([T(d, gpu) for d in docs])
        o.append_documents(docs)
    path = tmp_path / "index.sfx"
    g.save(path)  # completes the pending rebuild, if any
    o.poll_rebuild()
    gpu_state_equal(g, o)
    h = GlobalIndex.from_file(path, device=gpu)
    gpu_state_equal(h, o)
    np.testing.assert_array_equal(N(h.sa_key), N(g.sa_key))
    # in place into an index that holds other data
    e = GlobalIndex(capacity=5000, delta_capacity=600, k=6,
                    max_occurrences=16, rebuild_threshold=250, device=gpu)
    e.append_documents([T(rng.integers(0, 9, size=100).astype(I32), gpu)])
    ptrs = (e.corpus.data_ptr(), e.sa.data_ptr(), e.sa_key.data_ptr())
    e.restore(path)
    assert ptrs == (e.corpus.data_ptr(), e.sa.data_ptr(), e.sa_key.data_ptr())
    gpu_state_equal(e, o)
    q = np.zeros((16, 10), I32)
    ql = np.zeros(16, np.int64)
    for i in range(16):
        n = int(rng.integers(1, 11))
        q[i, :n] = rng.integers(0, 9, size=n)
        ql[i] = n
    caps = np.array([10, 5, 2], np.int64)
    for idx in (h, e):
        for got, exp in zip(idx._query_backoff(T(q, gpu), T(ql, gpu), 10,
                                               T(caps, gpu)),
                            o._query_backoff(q, ql, 10, caps)):
            np.testing.assert_array_equal(N(got), exp)
    with pytest.raises(ValueError):
        GlobalIndex(capacity=4096, delta_capacity=600, k=6,
                    device=gpu).restore(path)


def test_batched_appends_match_oracle(gpu):
    """Harvests of many rows at once: runs of more than 64 documents (two
    append launches), documents longer than the delta (kept tail), drops of
    the oldest documents while a rebuild is in flight, compactions at
    rebuild launch, and lengths given as a device tensor."""
    from suffixgpu_amd import SuffixGPUDrafter
    from oracle.drafter import DrafterOracle
    rng = np.random.default_rng(21)
    kw = dict(k=4, max_pattern_len=8, max_occurrences=8, num_backoff=3,
              enable_global=True, global_capacity=20000, delta_capacity=3000,
              rebuild_threshold=1500)
    d = SuffixGPUDrafter(device=gpu, **kw)
    o = DrafterOracle(**kw)
    s = 4000
    for rnd in range(6):
        b = 70 if rnd % 2 == 0 else 9
        tok = rng.integers(0, 7, size=(b, s)).astype(I32)
        lengths = rng.integers(0, 60, size=b)
        lengths[rng.integers(0, b)] = s        # longer than the delta
        lengths[rng.integers(0, b)] = 0
        rows = list(range(b))
        if rnd == 3:
            d.global_index._rebuild_event = _NeverDone()
            d.global_index._pending = (d.global_index.active_len,
                                       d.global_index.active_doc_lens)
            o.global_index._rebuild_event = _NeverDone()
            o.global_index._pending = (o.global_index.active_len,
                                       o.global_index.active_doc_lens)
        lens = T(lengths, gpu) if rnd % 3 == 1 else lengths.tolist()
        d.harvest_finished(rows, lens, T(tok, gpu))
        o.harvest_finished(rows, lengths.tolist(), tok)
        gpu_state_equal(d.global_index, o.global_index)
        assert int(d.global_index.delta_len_t.item()) == o.global_index.delta_len
        if rnd == 3:
            for gi in (d.global_index, o.global_index):
                gi._rebuild_event = None
                gi._pending = None


@pytest.mark.parametrize("keys", [True, False])
def test_patterns_longer_than_key_rows(gpu, keys):
    """P = 48 on long-repeat text: interval searches that compare past the
    32-token key rows (in the corpus), and the same queries on an index
    passed without key rows (sa[] and corpus compares only)."""
    from suffixgpu_amd import _lib
    tc = synth.TemplateCorpus(seed=9, n_templates=6)
    docs = [tc.sequence(lo=200, hi=900) for _ in range(30)]
    dd = [tc.sequence(lo=64, hi=300) for _ in range(3)]
    cap = sum(len(d) + 1 for d in docs) + 11
    g, o = _load_pair(gpu, docs, dd, cap, 2048, 32, k=16)
    if not keys:
        full = g.index_struct()
        g.index_struct = lambda: _lib.SfxIndex(
            full.corpus, full.sa, full.capacity, full.delta,
            full.delta_capacity, full.delta_len, None, 0)
    rng = np.random.default_rng(10)
    b, p = 40, 48
    q = np.zeros((b, p), I32)
    ql = np.zeros(b, np.int64)
    for i in range(b):
        src = docs[i % len(docs)]
        n = int(rng.integers(1, p + 1))
        st = int(rng.integers(0, len(src) - n + 1))
        q[i, :n] = src[st:st + n]
        ql[i] = n
    caps = np.array([48, 24, 12, 6, 3, 2], np.int64)
    tq, tl, tc_ = T(q, gpu), T(ql, gpu), T(caps, gpu)
    got = g._query_backoff(tq, tl, p, tc_)
    exp = o._query_backoff(q, ql, p, caps)
    for a, e in zip(got, exp):
        np.testing.assert_array_equal(N(a), e)
    assert (exp[0] > 32).sum() > 5
    for a, e in zip(g.draft(tq, tl, p, 16, min_token_prob=0.05,
                            max_spec_factor=1.0, caps=tc_),
                    o.draft(q, ql, p, 16, min_token_prob=0.05,
                            max_spec_factor=1.0, caps=caps)):
        np.testing.assert_array_equal(N(a), e)


PAD = np.iinfo(np.int32).max


def gram_runs(corpus, sa):
    """{(k, t0, t1, t2, t3): (lo, hi)}: every maximal run of ranks whose
    suffixes start with the same k real tokens (k = 1..4; tokens past k
    are 0), from the suffix array by its definition."""
    n = corpus.shape[0]
    pos = sa.astype(np.int64)
    idx = pos[:, None] + np.arange(4)[None, :]
    tok = np.where(idx < n, corpus[np.minimum(idx, n - 1)], -1).astype(
        np.int64)
    real = (tok >= 0) & (tok != PAD)
    out = {}
    for k in range(1, 5):
        key = np.where(np.arange(4)[None, :] < k, tok, 0)
        ok = real[:, :k].all(axis=1)
        new = np.ones(n, bool)
        new[1:] = (key[1:] != key[:-1]).any(axis=1) | (ok[1:] != ok[:-1])
        starts = np.flatnonzero(new)
        ends = np.append(starts[1:], n)
        for a, z in zip(starts, ends):
            if ok[a]:
                out[(k, *key[a].tolist())] = (int(a), int(z))
    return out


def runs_capacity_kmax(exp, slots):
    """The longest run length k whose runs of 1..k tokens together fill at
    most 3/4 of the table's slots: the lengths a build stores."""
    n, kmax = 0, 0
    for k in range(1, 5):
        n += sum(1 for key in exp if key[0] == k)
        if 4 * n > 3 * slots:
            break
        kmax = k
    return kmax


def gpu_gram_table(g):
    """(kmax, entries) of the live table: a 256-byte header {kmax, pad,
    runs[4] u64}, one u32 fill count per bucket of 16 slots (padded to
    256 bytes), then the buckets of 384 bytes: 16 keys {t0..t3} (-1 past
    the run's length k) and their 16 ranges {lo, hi}; a bucket's first
    min(count, 16) slots are filled.  Entries are keyed (k, t0, t1, t2,
    t3), tokens past k 0; kmax is the longest length whose runs are all
    stored."""
    raw = N(g._gram)
    slots_n = g.gram_slots
    nb = slots_n // 16
    cbytes = (nb * 4 + 255) // 256 * 256
    kmax = int(raw[:4].view(np.uint32)[0])
    counts = raw[256:256 + nb * 4].view(np.uint32)
    buckets = raw[256 + cbytes:256 + cbytes + nb * 384].view(
        np.int32).reshape(nb, 96)
    tab = {}
    for b in np.flatnonzero(counts):
        keys = buckets[b, :64].reshape(16, 4)
        ranges = buckets[b, 64:].reshape(16, 2)
        for key4, rng in zip(keys[:min(int(counts[b]), 16)],
                             ranges[:min(int(counts[b]), 16)]):
            k = int((key4 != -1).sum())
            assert (key4[:k] >= 0).all() and (key4[k:] == -1).all(), key4
            key = (k, *[int(x) if j < k else 0 for j, x in enumerate(key4)])
            assert key not in tab, key
            tab[key] = (int(np.uint32(rng[0])), int(np.uint32(rng[1])))
    return kmax, tab


def test_gram_table_matches_runs(gpu):
    """The n-gram range table after a rebuild holds exactly the runs of
    1..4 real tokens of the sorted suffixes with their rank ranges, also
    after later rebuilds reuse both buffers (a shorter corpus after a
    longer one, so stale rows and slots are left behind)."""
    from suffixgpu_amd.global_index import GlobalIndex
    tc = synth.TemplateCorpus(seed=13, n_templates=5)
    g = GlobalIndex(capacity=1 << 14, delta_capacity=1 << 12, k=8,
                    max_occurrences=16, rebuild_threshold=1 << 30,
                    device=gpu)
    for rep, nd in enumerate((12, 17, 4, 3, 15)):
        docs = [tc.sequence(lo=100 + 50 * (rep % 2), hi=700)
                for _ in range(nd)]
        g.load_documents([T(d, gpu) for d in docs])
        torch.cuda.synchronize()
        kmax, tab = gpu_gram_table(g)
        assert kmax == 4
        exp = gram_runs(N(g.corpus), N(g.sa))
        assert len(exp) > 200
        assert tab == exp
        keys_by_definition(g.corpus, g.sa, g.sa_key)


def test_gram_table_keeps_the_lengths_that_fit(gpu):
    """Uniform random tokens over a 2^17 vocabulary hold about 3 distinct
    runs of 1-4 tokens per position, more than the 3 slots per position
    hold at 3/4 load: the table keeps every run of the lengths that fit
    (the 1- and 2-token runs here) and exactly those, and capped queries
    and drafts still equal the oracle's (searches start from the first
    two tokens' range)."""
    from suffixgpu_amd.global_index import GlobalIndex
    from oracle.global_index import GlobalIndexOracle
    rng = np.random.default_rng(21)
    # 48 documents, 59,182 tokens: 47,684 distinct tokens, then 59,086,
    # 59,038 and 58,990 runs of 2, 3 and 4 tokens, against 147,456 slots
    # at 3/4 of 3 x 2^16
    docs = [rng.integers(0, 1 << 17, size=int(rng.integers(1150, 1300)))
            .astype(I32) for _ in range(48)]
    kw = dict(capacity=1 << 16, delta_capacity=1 << 12, k=12,
              max_occurrences=32, rebuild_threshold=1 << 30)
    g = GlobalIndex(device=gpu, **kw)
    o = GlobalIndexOracle(**kw)
    g.load_documents([T(d, gpu) for d in docs])
    o.load_documents(docs)
    torch.cuda.synchronize()
    kmax, tab = gpu_gram_table(g)
    exp = gram_runs(N(g.corpus), N(g.sa))
    assert runs_capacity_kmax(exp, g.gram_slots) == 2
    assert kmax == 2
    assert tab == {key: v for key, v in exp.items() if key[0] <= kmax}
    b, p = 48, 24
    q = np.zeros((b, p), I32)
    ql = np.zeros(b, np.int64)
    for i in range(b):
        n = int(rng.integers(1, p + 1))
        if i % 3 == 2:  # absent patterns
            q[i, :n] = rng.integers(0, 1 << 17, size=n)
        else:
            src = docs[i % len(docs)]
            st = int(rng.integers(0, len(src) - n + 1))
            q[i, :n] = src[st:st + n]
        ql[i] = n
    caps = np.array([24, 12, 6, 3, 2, 1], np.int64)
    tq, tl, tc_ = T(q, gpu), T(ql, gpu), T(caps, gpu)
    for got, e in zip(g._query_backoff(tq, tl, p, tc_),
                      o._query_backoff(q, ql, p, caps)):
        np.testing.assert_array_equal(N(got), e)
    for got, e in zip(g.draft(tq, tl, p, 12, min_token_prob=0.05,
                              caps=tc_),
                      o.draft(q, ql, p, 12, min_token_prob=0.05,
                              caps=caps)):
        np.testing.assert_array_equal(N(got), e)


@pytest.mark.parametrize("slots", [None, 1024, 0])
def test_queries_with_and_without_gram_table(gpu, slots):
    """Capped SA + delta queries and drafts agree with the oracle with the
    table in use and with a table too small for the corpus (it keeps the
    run lengths that fit, possibly none, and searches start from those);
    queries holding separator, padding or -1 tokens skip the table.
    slots=0: no key rows and no table at all (search_tables=False); every
    comparison reads the suffix array and the corpus."""
    from suffixgpu_amd.global_index import GlobalIndex
    from oracle.global_index import GlobalIndexOracle
    tc = synth.TemplateCorpus(seed=14, n_templates=6)
    docs = [tc.sequence(lo=200, hi=900) for _ in range(30)]
    kw = dict(capacity=1 << 15, delta_capacity=1 << 12, k=12,
              max_occurrences=32, rebuild_threshold=1 << 30)
    g = GlobalIndex(device=gpu, gram_slots=slots or None,
                    search_tables=slots != 0, **kw)
    o = GlobalIndexOracle(**kw)
    g.load_documents([T(d, gpu) for d in docs])
    o.load_documents(docs)
    dd = [tc.sequence(lo=64, hi=300) for _ in range(4)]
    g.append_documents([T(d, gpu) for d in dd])
    o.append_documents(dd)
    torch.cuda.synchronize()
    if slots != 0:
        kmax, tab = gpu_gram_table(g)
        exp = gram_runs(N(g.corpus), N(g.sa))
        if slots is None:
            assert kmax == 4
        else:
            kcap = runs_capacity_kmax(exp, slots)
            assert kmax <= kcap < 4
            # only runs of the lengths that fit were inserted; an insert
            # that found no room lowered kmax below its own length
            assert all(key[0] <= kcap for key in tab)
        assert {key: v for key, v in tab.items() if key[0] <= kmax} == \
            {key: v for key, v in exp.items() if key[0] <= kmax}
    else:
        assert g.sa_key is None and g.device_bytes()["key_rows"] == 0
    rng = np.random.default_rng(15)
    b, p = 48, 40
    q = np.zeros((b, p), I32)
    ql = np.zeros(b, np.int64)
    for i in range(b):
        src = docs[i % len(docs)]
        n = int(rng.integers(1, p + 1))
        st = int(rng.integers(0, len(src) - n + 1))
        q[i, :n] = src[st:st + n]
        ql[i] = n
        if i % 8 == 7:  # tokens a query never holds by contract
            q[i, int(rng.integers(0, n))] = (-2, PAD, -1)[i % 3]
    caps = np.array([40, 20, 10, 5, 3, 2, 1], np.int64)
    tq, tl, tc_ = T(q, gpu), T(ql, gpu), T(caps, gpu)
    for got, exp in zip(g._query_backoff(tq, tl, p, tc_),
                        o._query_backoff(q, ql, p, caps)):
        np.testing.assert_array_equal(N(got), exp)
    for got, exp in zip(g.draft(tq, tl, p, 12, min_token_prob=0.05,
                                caps=tc_),
                        o.draft(q, ql, p, 12, min_token_prob=0.05,
                                caps=caps)):
        np.testing.assert_array_equal(N(got), exp)
