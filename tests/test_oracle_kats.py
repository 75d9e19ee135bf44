"""The oracle against the reference's known-answer tests and brute force.

Re-expresses tests/test_expand.py, test_suffix_array.py, test_sa_search.py,
test_local_matcher.py, test_global_index.py and test_proposer_glue.py of
zip95297/SuffixGPU against the numpy restatement, plus brute-force checks
built from the textbook definitions in oracle/naive.py.
"""

from __future__ import annotations

import random

import numpy as np
import pytest

from oracle import naive
from oracle.drafter import DrafterOracle, backoff_thresholds, global_caps
from oracle.expand import expand_chain, expand_chain_pairwise, majority_token
from oracle.global_index import GlobalIndexOracle
from oracle.local import LocalMatcher, match_back, newest_first_pattern
from oracle.sa import (build_suffix_array, longest_suffix_match,
                       search_interval)

I32 = np.int32


# ---------------------------------------------------------------- expand
def test_majority_kats():
    v = np.array([[5, 5, 7, 7, 7], [1, 2, 1, -1, -1]], I32)
    a = np.array([[True] * 5, [True, True, True, False, False]])
    tok, cnt = majority_token(v, a, -1)
    assert tok.tolist() == [7, 1] and cnt.tolist() == [3, 2]
    tok, cnt = majority_token(np.array([[5, 7, 5, 5, -1]], I32),
                              np.ones((1, 5), bool), -1)
    assert tok.tolist() == [5] and cnt.tolist() == [3]
    tok, cnt = majority_token(np.array([[9, 9, 3, 3, -1]], I32),
                              np.ones((1, 5), bool), -1)
    assert tok.tolist() == [3] and cnt.tolist() == [2]
    tok, cnt = majority_token(np.zeros((1, 4), I32), np.zeros((1, 4), bool),
                              -1)
    assert tok.tolist() == [-1] and cnt.tolist() == [0]


def test_expand_kats():
    one = np.array([2], np.int64)
    ch, nv, _, _ = expand_chain(np.array([[[4, 5, 6], [4, 7, 8]]], I32), one, 3)
    assert ch.tolist() == [[4, 5, 6]] and nv.tolist() == [3]
    ch, nv, _, _ = expand_chain(np.array([[[4, 5, -1], [3, 9, 2]]], I32), one,
                                3)
    assert ch.tolist() == [[3, 9, 2]] and nv.tolist() == [3]
    ch, nv, _, _ = expand_chain(np.array([[[4, -1, -1], [4, 1, -1]]], I32),
                                one, 3)
    assert ch.tolist() == [[4, 1, -1]] and nv.tolist() == [2]
    ch, nv, _, _ = expand_chain(np.full((2, 3, 4), -1, I32),
                                np.zeros(2, np.int64), 4)
    assert (ch == -1).all() and nv.tolist() == [0, 0]


def test_weighted_vote_and_alpha_kats():
    cont = np.array([[[7, 1], [7, 1], [3, 2]]], I32)
    ch, nv, _, _ = expand_chain(cont, np.array([3]), 2,
                                weights=np.array([[1.0, 1.0, 5.0]]))
    assert ch[0].tolist() == [3, 2] and nv.item() == 2
    cont = np.array([[[5, 6, 7, 8]]], I32)
    _, nv, _, _ = expand_chain(cont, np.array([1]), 4, min_token_prob=0.2,
                               alpha=1.0)
    assert nv.item() == 2
    _, nv, _, _ = expand_chain(cont, np.array([1]), 4, min_token_prob=0.2,
                               alpha=0.0)
    assert nv.item() == 4


def _rand_expand_case(rng, b, r, k):
    cont = rng.integers(0, 9, size=(b, r, k)).astype(I32)
    tail = rng.integers(0, k + 1, size=(b, r))
    cont = np.where(np.arange(k)[None, None, :] < tail[:, :, None], cont, -1)
    occ = rng.integers(0, r + 1, size=b).astype(np.int64)
    cap = rng.integers(0, k + 1, size=b).astype(np.int64)
    return cont.astype(I32), occ, cap


@pytest.mark.parametrize("r", [4, 32])
@pytest.mark.parametrize("minp", [0.0, 0.1])
def test_sort_vote_equals_pairwise_vote(r, minp):
    """The reference's v2 == pairwise property (test_expand_v2.py:28-43)."""
    rng = np.random.default_rng(1234 + r)
    cont, occ, cap = _rand_expand_case(rng, 17, r, 8)
    a = expand_chain(cont, occ, 8, min_token_prob=minp, cap=cap)
    b = expand_chain_pairwise(cont, occ, 8, minp, cap)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(np.asarray(x), np.asarray(y))


def test_prob_is_fp32_div_then_mul():
    """cum = fl32(cum * fl32(v / n)), each step rounded (expand.py:130)."""
    cont = np.zeros((1, 3, 2), I32)
    cont[0, :, 0] = [4, 4, 5]
    cont[0, :2, 1] = [6, 7]
    cont[0, 2, 1] = -1
    _, _, _, score = expand_chain(cont, np.array([3]), 2)
    p0 = np.float32(2) / np.float32(3)
    p1 = np.float32(p0 * (np.float32(1) / np.float32(2)))
    assert score.item() == np.float32(p0 + p1)


# ----------------------------------------------------------- suffix array
STRUCTURED = [[1, 2, 3, 1, 2, 3, 1, 2], [5, 5, 5, 5, 5], [0], [2, 1],
              [1, 2, 1, 2, 1, 2, 1], [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5]]


@pytest.mark.parametrize("tokens", STRUCTURED)
def test_suffix_array_structured(tokens):
    assert build_suffix_array(np.array(tokens)).tolist() == \
        naive.suffix_array(tokens)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("n,vocab", [(31, 3), (64, 8), (200, 16), (7, 2)])
def test_suffix_array_random(seed, n, vocab):
    rng = np.random.default_rng(seed)
    t = rng.integers(0, vocab, size=n).tolist()
    assert build_suffix_array(np.array(t)).tolist() == naive.suffix_array(t)


def test_suffix_array_signed_order_and_edges():
    t = [3, -2, 2147483647, 3, -2, 0, 2147483647]
    assert build_suffix_array(np.array(t)).tolist() == naive.suffix_array(t)
    assert build_suffix_array(np.zeros(0, I32)).shape == (0,)
    assert build_suffix_array(np.array([7])).tolist() == [0]


# ------------------------------------------------------------- SA search
CORPUS = [1, 2, 3, 1, 2, 4, 1, 2, 3, 9, 1, 2, 3, 1, 5]


@pytest.mark.parametrize("pattern", [[1], [1, 2], [1, 2, 3], [1, 2, 4], [9],
                                     [5], [1, 2, 3, 1], [7],
                                     [1, 2, 3, 1, 2, 3], [3, 1], [2, 4, 1]])
def test_search_interval_kat(pattern):
    sa = build_suffix_array(np.array(CORPUS))
    s, e = search_interval(sa, np.array(CORPUS, I32),
                           np.array([pattern], I32),
                           np.array([len(pattern)]))
    exp = naive.search_interval(naive.suffix_array(CORPUS), CORPUS, pattern)
    assert (int(s[0]), int(e[0])) == exp
    assert sorted(sa[int(s[0]):int(e[0])].tolist()) == \
        naive.occurrences(CORPUS, pattern)


@pytest.mark.parametrize("seed", range(4))
def test_search_interval_random(seed):
    rng = np.random.default_rng(seed)
    toks = rng.integers(0, 4, size=128).tolist()
    sa = build_suffix_array(np.array(toks))
    pats, lens = [], []
    for _ in range(20):
        m = int(rng.integers(1, 8))
        st = int(rng.integers(0, 128 - m + 1))
        pats.append(toks[st:st + m] + [0] * (8 - m))
        lens.append(m)
    s, e = search_interval(sa, np.array(toks, I32), np.array(pats, I32),
                           np.array(lens))
    for i in range(20):
        assert (int(s[i]), int(e[i])) == naive.search_interval(
            sa.tolist(), toks, pats[i][:lens[i]])


@pytest.mark.parametrize("query,max_len", [([1, 2, 3, 1, 2], 8),
                                           ([9, 9, 1, 2, 3], 8),
                                           ([4, 4, 4], 4),
                                           ([1, 2, 3, 1, 5, 1, 2, 3], 10)])
def test_longest_suffix_match_kat(query, max_len):
    sa = build_suffix_array(np.array(CORPUS))
    ml, s, e = longest_suffix_match(sa, np.array(CORPUS, I32),
                                    np.array([query], I32),
                                    np.array([len(query)]), max_len)
    exp = naive.longest_suffix_match(CORPUS, query, max_len)
    assert int(ml[0]) == exp
    if exp:
        assert sorted(sa[int(s[0]):int(e[0])].tolist()) == \
            naive.occurrences(CORPUS, query[-exp:])


# ----------------------------------------------------------- local match
LOCAL_CASES = [[1, 2, 3, 1, 2, 3, 4, 5, 1, 2, 3], [7, 7, 7, 7, 7, 7],
               [1, 2, 1, 2, 1, 2, 9, 1, 2], [5, 6, 7, 8, 5, 6, 7, 8, 5, 6],
               [1], [1, 2], [3, 1, 4, 1, 5, 9, 2, 6],
               [2, 2, 3, 2, 2, 4, 2, 2, 3]]


def _run_local(lm, seqs, mask=None):
    w = max(len(s) for s in seqs)
    buf = np.zeros((len(seqs), w), I32)
    lens = np.zeros(len(seqs), I32)
    for i, s in enumerate(seqs):
        buf[i, :len(s)] = s
        lens[i] = len(s)
    if mask is None:
        mask = np.ones(len(seqs), bool)
    return lm.forward(lens, buf, mask)


def test_local_match_vs_naive():
    lm = LocalMatcher(k=4, max_pattern_len=8, max_occurrences=16)
    draft, nv, mlen, _, _ = _run_local(lm, LOCAL_CASES)
    for i, seq in enumerate(LOCAL_CASES):
        exp_chain, exp_len = naive.local_match(seq, 4, 8, 1, 16)
        assert mlen[i] == exp_len
        assert draft[i, :nv[i]].tolist() == exp_chain


def test_local_match_random_vs_naive():
    lm = LocalMatcher(k=4, max_pattern_len=6, max_occurrences=8)
    rng = np.random.default_rng(0)
    seqs = [rng.integers(0, 4, size=int(rng.integers(8, 48))).tolist()
            for _ in range(24)]
    draft, nv, mlen, _, _ = _run_local(lm, seqs)
    for i, seq in enumerate(seqs):
        exp_chain, exp_len = naive.local_match(seq, 4, 6, 1, 8)
        assert mlen[i] == exp_len, seq
        assert draft[i, :nv[i]].tolist() == exp_chain[:nv[i]], seq


def test_local_mask():
    lm = LocalMatcher(k=4, max_pattern_len=8, max_occurrences=16)
    seq = [1, 2, 3, 1, 2, 3, 4, 1, 2, 3]
    draft, nv, *_ = _run_local(lm, [seq, seq], mask=np.array([False, True]))
    assert nv[0] == 0 and (draft[0] == -1).all()
    assert draft[1, :nv[1]].tolist() == naive.local_match(seq, 4, 8, 1, 16)[0]


def test_match_back_brute_force():
    rng = np.random.default_rng(5)
    tok = rng.integers(0, 3, size=(4, 50)).astype(I32)
    q = np.array([50, 37, 5, 0])
    pat = newest_first_pattern(tok, q, 6, -2)
    mb = match_back(tok, pat, 50)
    for b in range(4):
        for i in range(50):
            m = 0
            while m < 6:
                j = i - 1 - m
                x = tok[b, j] if j >= 0 else -1
                if x != pat[b, m]:
                    break
                m += 1
            assert mb[b, i] == m


def test_candidates_closed_form():
    """cand_t = largest L with #{i < q: mb[i] >= L} >= t."""
    rng = np.random.default_rng(9)
    lm = LocalMatcher(k=4, max_pattern_len=10, max_occurrences=8,
                      support_thresholds=(1, 2, 4, 8, 16))
    tok = rng.integers(0, 3, size=(6, 120)).astype(I32)
    q = rng.integers(1, 121, size=6)
    mb = lm.match(q, tok)
    cand, _, _ = lm.gather_candidates(q, tok, np.ones(6, bool))
    for b in range(6):
        prev = None
        for c, t in enumerate((1, 2, 4, 8, 16)):
            best = max([L for L in range(1, 11) if (mb[b] >= L).sum() >= t],
                       default=0)
            exp = 0 if best == prev else best
            prev = best
            assert cand[b, c] == exp


# ------------------------------------------------------------ proposer glue
def _drafter(enable_global=False, **kw):
    return DrafterOracle(k=4, max_pattern_len=8, max_occurrences=8,
                         enable_global=enable_global, global_capacity=1024,
                         delta_capacity=256, rebuild_threshold=100000, **kw)


def test_caps_and_thresholds():
    assert backoff_thresholds(8) == (1, 2, 4, 8, 16, 32, 64, 128)
    assert global_caps(32, 8) == [32, 16, 8, 4, 2]
    assert global_caps(32, 1) == [32]
    assert global_caps(10, 5) == [10, 5, 2]


def test_update_state_kats():
    d = _drafter()
    buf = np.zeros((2, 10), I32)
    buf[0, :3] = [1, 2, 3]
    buf[1, :5] = 9
    new = d.update_state(np.array([3, 5], I32), buf,
                         np.array([[7, 8, -1], [4, -1, -1]], I32))
    assert new.tolist() == [5, 6]
    assert buf[0, :5].tolist() == [1, 2, 3, 7, 8]
    assert buf[1, :6].tolist() == [9, 9, 9, 9, 9, 4]
    buf = np.zeros((1, 4), I32)
    new = d.update_state(np.array([3], I32), buf, np.array([[5, 6]], I32))
    assert buf[0, 3] == 5 and new.tolist() == [5]


def test_propose_with_update_kats():
    d = _drafter()
    buf = np.zeros((1, 32), I32)
    buf[0, :7] = [5, 6, 7, 8, 5, 6, 7]
    draft, nv, new = d.propose_with_update(
        np.array([7], I32), buf, np.array([[8, 5, -1, -1, -1]], I32))
    assert new.tolist() == [9] and nv[0] >= 1
    assert draft[0, :nv[0]].tolist() == [6, 7, 8, 5][:nv[0]]
    buf = np.zeros((2, 16), I32)
    buf[:, :5] = [3, 4, 3, 4, 3]
    draft, nv, _ = d.propose_with_update(np.array([5, 5], I32), buf,
                                         np.array([[4, -1], [-1, -1]], I32))
    assert nv[0] > 0 and nv[1] == 0 and (draft[1] == -1).all()
    buf = np.zeros((1, 16), I32)
    buf[0, :6] = [3, 4, 3, 4, 3, 4]
    _, nv, new = d.propose_with_update(np.array([6], I32), buf,
                                       np.array([[3, -1]], I32),
                                       max_model_len=7)
    assert new.tolist() == [7] and nv[0] == 0


def test_adaptive_cap_and_min_prob_kats():
    seq = [1, 2, 7, 8, 9, 1, 2]
    buf = np.zeros((1, 16), I32)
    buf[0, :7] = seq
    n = np.array([7], I32)
    base = DrafterOracle(k=4, max_pattern_len=8, max_occurrences=16)
    draft, nv = base.propose(n, buf)
    assert nv[0] == 4 and draft[0].tolist() == [7, 8, 9, 1]
    clamped = DrafterOracle(k=4, max_pattern_len=8, max_occurrences=16,
                            max_spec_factor=1.0)
    draft, nv = clamped.propose(n, buf)
    assert nv[0] == 2 and draft[0].tolist() == [7, 8, -1, -1]
    seq = [5, 6, 0, 5, 6, 1, 5, 7, 2, 5]
    buf = np.zeros((1, 16), I32)
    buf[0, :10] = seq
    n = np.array([10], I32)
    mid = DrafterOracle(k=4, max_pattern_len=8, max_occurrences=16,
                        min_token_prob=0.5)
    draft, nv = mid.propose(n, buf)
    assert nv[0] == 1 and draft[0].tolist() == [6, -1, -1, -1]
    strict = DrafterOracle(k=4, max_pattern_len=8, max_occurrences=16,
                           min_token_prob=0.7)
    draft, nv = strict.propose(n, buf)
    assert nv[0] == 0


def test_ingest_active_kats():
    d = _drafter(enable_global=True)
    gi = d.global_index
    row = np.arange(100, 200, dtype=I32)
    d.ingest_active(["r0"], [row], [10], chunk=16)
    assert gi.delta_len == 0
    d.ingest_active(["r0"], [row], [20], chunk=16)
    assert gi.delta_len == 21
    d.ingest_active(["r0"], [row], [30], chunk=16)
    assert gi.delta_len == 21
    d.ingest_active(["r0"], [row], [30], final=True, chunk=16)
    assert gi.delta_len > 21 and "r0" not in d._ingested
    d = _drafter(enable_global=True)
    row = np.arange(500, 564, dtype=I32)
    d.ingest_active(["r"], [row], [32], chunk=32)
    d.ingest_active(["r"], [row], [64], chunk=32)
    ml, cont, occ = d.global_index.query(row[28:36][None, :],
                                         np.array([8]), 8)
    assert ml[0] == 8
    chain, nv = d.global_index.expand(cont, occ)
    assert nv[0] > 0 and chain[0, :nv[0]].tolist() == \
        row[36:36 + nv[0]].tolist()


# ----------------------------------------------------------- global index
def _q(gi, query, p=8):
    ml, cont, occ = gi.query(np.array([query], I32), np.array([len(query)]),
                             p)
    chain, nv = gi.expand(cont, occ)
    return chain[0, :nv[0]].tolist(), int(ml[0]), int(occ[0])


def _gi(**kw):
    base = dict(capacity=1024, delta_capacity=256, k=4, max_occurrences=8,
                rebuild_threshold=100000)
    base.update(kw)
    return GlobalIndexOracle(**base)


def test_global_delta_sa_and_consistency():
    doc = [5, 6, 7, 8, 9, 5, 6, 7, 8, 10]
    for thr in (100000, 1):
        gi = _gi(rebuild_threshold=thr)
        gi.append_documents([np.array(doc)])
        chain, ml, occ = _q(gi, [5, 6, 7, 8])
        exp_chain, exp_len = naive.global_chain([doc], [5, 6, 7, 8], 4, 8, 8)
        assert (chain, ml, occ) == (exp_chain, exp_len, 2)
    docs = [[1, 2, 3, 4, 1, 2, 3, 9], [7, 1, 2, 3, 4, 8, 1, 2]]
    res = []
    for thr in (100000, 1):
        gi = _gi(rebuild_threshold=thr)
        gi.append_documents([np.array(x) for x in docs])
        res.append(_q(gi, [1, 2, 3, 4]))
    exp_chain, exp_len = naive.global_chain(docs, [1, 2, 3, 4], 4, 8, 8)
    assert res[0][:2] == res[1][:2] == (exp_chain, exp_len)


def test_global_multiple_rebuilds_eviction_empty():
    gi = _gi(rebuild_threshold=1)
    docs = [[1, 1, 2], [1, 1, 3], [1, 1, 4], [1, 1, 5]]
    for x in docs:
        gi.append_documents([np.array(x)])
    assert gi.active_len == sum(len(x) + 1 for x in docs)
    chain, ml, _ = _q(gi, [1, 1])
    assert (chain, ml) == naive.global_chain(docs, [1, 1], 4, 8, 8)
    gi = _gi(capacity=12, delta_capacity=64, rebuild_threshold=1)
    for t in (1, 2, 3, 4):
        gi.append_documents([np.array([t] * 4)])
    assert gi.active_len <= 12
    assert _q(gi, [4, 4])[1] == 2 and _q(gi, [1, 1, 1, 1])[1] == 0
    gi = GlobalIndexOracle(capacity=64, delta_capacity=16, k=4,
                           max_occurrences=8)
    assert _q(gi, [1, 2, 3]) == ([], 0, 0)


def test_global_regressions():
    gi = _gi()
    doc = [9, 7, 7, 101, 5, 5, 5, 5, 5, 3, 7, 7, 101, 6, 6, 6, 6, 6, 6, 7, 7,
           101, 4]
    gi.append_documents([np.array(doc)])
    dl, dp, dc = gi._delta_match_backoff(
        np.array([[7, 7] + [0] * 6], I32), np.array([2]), 8,
        np.array([8]))
    assert dl[0, 0] == 2 and dc[0, 0] == 3 and dp[0, 0, :3].tolist() == \
        [1, 10, 19]
    chain, ml, occ = _q(gi, [7, 7])
    assert (ml, occ, chain[0]) == (2, 3, 101)
    gi = _gi(max_occurrences=4)
    gi.max_occurrences = 4
    doc = [1, 9] * 10 + [1, 2, 3, 4, 6]
    gi.append_documents([np.array(doc)])
    assert _q(gi, [1, 2, 3, 4]) == ([6], 4, 1)


class _NeverDone:
    def query(self):
        return False


def test_global_overflow_paths():
    gi = GlobalIndexOracle(capacity=64, delta_capacity=18, k=4,
                           max_occurrences=8, rebuild_threshold=100000)
    gi.append_documents([np.array([1] * 6), np.array([2] * 6)])
    gi._rebuild_event = _NeverDone()
    gi._pending = (gi.active_len, gi.active_doc_lens)
    gi.append_documents([np.array([3] * 10)])
    assert gi.delta_len <= gi.delta_capacity
    assert _q(gi, [3, 3])[1] == 2 and _q(gi, [2, 2])[1] == 2
    assert _q(gi, [1, 1])[1] == 0
    gi = GlobalIndexOracle(capacity=64, delta_capacity=16, k=4,
                           max_occurrences=8, rebuild_threshold=100000)
    gi.append_documents([np.array([1] * 12)])
    gi.append_documents([np.array([2] * 12)])
    assert gi.active_len == 13 and gi.delta_len == 13
    assert _q(gi, [1, 1])[1] == 2 and _q(gi, [2, 2])[1] == 2


def test_no_cross_document_match():
    for thr in (100000, 1):
        gi = _gi(capacity=256, delta_capacity=64, rebuild_threshold=thr)
        gi.append_documents([np.array([1, 2, 3, 7, 8, 9]),
                             np.array([100, 101, 102, 55, 56])])
        assert _q(gi, [7, 8, 9]) == ([], 3, 1)
        assert _q(gi, [8, 9, 100]) == ([101, 102, 55, 56], 1, 1)


def test_query_consistency_across_rebuilds():
    d = DrafterOracle(k=4, max_pattern_len=8, max_occurrences=16,
                      enable_global=True, global_capacity=1 << 16,
                      delta_capacity=1 << 12, rebuild_threshold=1 << 10)
    gi = d.global_index
    gi.rebuild_threshold = 16
    g = random.Random(3)
    corpus: list[int] = []
    for _ in range(8):
        doc = [g.randint(0, 4) for _ in range(24)]
        gi.append_documents([np.array(doc)])
        corpus.extend(doc)
        query = doc[-6:]
        ml, _, occ = gi.query(np.array([query + [0, 0]], I32), np.array([6]),
                              8)
        exp = naive.longest_suffix_match(corpus, query, 8)
        assert ml[0] == exp
        if exp:
            assert 1 <= occ[0] <= min(len(naive.occurrences(
                corpus, query[-exp:])), 16)


def test_proposer_global_harvest():
    d = DrafterOracle(k=4, max_pattern_len=8, max_occurrences=8,
                      enable_global=True, global_capacity=1024,
                      delta_capacity=256, rebuild_threshold=1)
    buf = np.zeros((2, 32), I32)
    done = [9, 8, 7, 6, 5, 9, 8, 7, 6, 4]
    buf[0, :10] = done
    d.harvest_finished([0], [10], buf)
    buf[1, :4] = [9, 8, 7, 6]
    draft, nv = d.propose(np.array([0, 4], I32), buf,
                          np.array([False, True]))
    exp_chain, _ = naive.global_chain([done], [9, 8, 7, 6], 4, 8, 8)
    assert nv[1] == len(exp_chain) and draft[1, :nv[1]].tolist() == exp_chain
    assert nv[0] == 0


def test_row_pool_matches_single_process():
    """The row-parallel oracle (the benchmark's multi-core CPU baseline)
    returns exactly the single-process step, local-only and with a global
    index, and updates the token rows the same way."""
    from oracle.pool import RowPool
    from suffixgpu_amd import synth
    kw = dict(k=8, max_pattern_len=16, max_occurrences=32, num_backoff=6,
              max_spec_factor=2.0, min_token_prob=0.05)
    w = synth.local_zipf(seed=9, b=13, s=600, lo=100)
    o = DrafterOracle(**kw)
    tok = w.tokens.copy()
    exp = o.propose_with_update(w.num_tokens, tok, w.sampled)
    with RowPool(kw, workers=3) as pool:
        tp = w.tokens.copy()
        got = pool.propose_with_update(w.num_tokens, tp, w.sampled)
        np.testing.assert_array_equal(tp, tok)
        for a, e in zip(got, exp):
            np.testing.assert_array_equal(a, e)
        for a, e in zip(pool.propose(exp[2], tp), o.propose(exp[2], tok)):
            np.testing.assert_array_equal(a, e)
    gkw = dict(kw, enable_global=True, global_capacity=1 << 14,
               delta_capacity=1 << 12, rebuild_threshold=1 << 20)
    gw = synth.global_corpus(seed=4, capacity=1 << 14, delta_fill=2100,
                             n_docs=12, b=11, s=1600, seq_hi=1300)
    o = DrafterOracle(**gkw)
    o.global_index.load_documents(gw.active_docs)
    o.global_index.append_documents(gw.delta_docs)
    g = o.global_index
    index = {"corpus": g.corpus, "sa": g.sa, "delta": g.delta[:g.delta_len],
             "active_len": g.active_len, "delta_len": g.delta_len}
    tok = gw.batch.tokens.copy()
    exp = o.propose_with_update(gw.batch.num_tokens, tok, gw.batch.sampled)
    assert (exp[1] > 0).any()
    with RowPool(gkw, index=index, workers=4) as pool:
        tp = gw.batch.tokens.copy()
        got = pool.propose_with_update(gw.batch.num_tokens, tp,
                                       gw.batch.sampled)
    np.testing.assert_array_equal(tp, tok)
    for a, e in zip(got, exp):
        np.testing.assert_array_equal(a, e)


def test_rebuild_finishing_at_the_callers_poll():
    """finish_at_user_poll: a rebuild that an append starts is still
    running at that append's later room-making, so the oldest delta
    document is dropped (global_index.py:110-118) instead of a second
    rebuild starting; the caller's poll swaps the first one in.  Worked by
    hand: delta capacity 20, documents of 10, 10, 5, 15 and 3 tokens
    (separator included)."""
    docs = [np.arange(1, 10), np.arange(11, 20), np.arange(21, 25),
            np.arange(31, 45), np.arange(51, 53)]
    kw = dict(capacity=100, delta_capacity=20, k=4, rebuild_threshold=1000)
    u = GlobalIndexOracle(async_rebuild=True, finish_at_user_poll=True, **kw)
    u.append_documents(docs)
    # the 5-token document made room by staging the first two; the
    # 3-token one found that rebuild running and dropped the 5-token one
    assert u.delta_doc_lens == [15, 3] and u.delta_len == 18
    assert u.active_len == 0 and u._rebuild_event is not None
    np.testing.assert_array_equal(
        u.delta[:18], np.concatenate([docs[3], [-2], docs[4], [-2]]))
    u.poll_rebuild()
    assert u.active_len == 20 and list(u.active_doc_lens) == [10, 10]
    np.testing.assert_array_equal(
        u.corpus[:20], np.concatenate([docs[0], [-2], docs[1], [-2]]))
    assert u._rebuild_event is None
    # the schedule where a build is done by the next poll: the 3-token
    # document's room-making swaps the first one in and stages the 5- and
    # 15-token documents, which maybe_rebuild's poll swaps in too
    a = GlobalIndexOracle(async_rebuild=True, **kw)
    a.append_documents(docs)
    assert a.delta_doc_lens == [3] and a.active_len == 40
    assert list(a.active_doc_lens) == [10, 10, 5, 15]


def test_user_poll_schedule_equals_next_poll_without_midcall_room():
    """Without room-making inside a call, the two schedules leave the same
    index after every caller poll (the only rebuilds start at the end of
    a call, in maybe_rebuild)."""
    rng = np.random.default_rng(35)
    kw = dict(capacity=3000, delta_capacity=400, k=4, rebuild_threshold=150)
    u = GlobalIndexOracle(async_rebuild=True, finish_at_user_poll=True, **kw)
    a = GlobalIndexOracle(async_rebuild=True, **kw)
    for _ in range(30):
        docs = [rng.integers(0, 9, size=int(n))
                for n in rng.integers(1, 40, size=3)]
        for gi in (u, a):
            gi.append_documents(docs)
            gi.poll_rebuild()
        assert u.delta_doc_lens == a.delta_doc_lens
        assert list(u.active_doc_lens) == list(a.active_doc_lens)
        np.testing.assert_array_equal(u.corpus, a.corpus)
        np.testing.assert_array_equal(u.sa, a.sa)
        np.testing.assert_array_equal(u.delta[:u.delta_len],
                                      a.delta[:a.delta_len])


def test_expand_other_sentinel_kat():
    """expand.py:107-147 with sentinel -7: -1 is a real token.  Depth 0:
    -1 holds 2 of 3 votes; depth 1: the two rows on the chain agree on 5;
    depth 2: both are padding.  Worked by hand."""
    from oracle.expand import expand_chain
    cont = np.array([[[-1, 5, -7], [-1, 5, -7], [3, -7, -7]]], np.int32)
    chain, nv, emit, score = expand_chain(cont, np.array([3]), 3,
                                          sentinel=-7)
    assert chain.tolist() == [[-1, 5, -7]]
    assert nv.tolist() == [2] and emit.tolist() == [2]
    p = np.float32(2) / np.float32(3)
    assert score[0] == np.float32(p + np.float32(p * np.float32(1)))
