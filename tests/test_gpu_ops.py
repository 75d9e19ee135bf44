"""HIP operators vs the oracle: scatter, match_back, first occurrences,
SA build and search, majority-vote expansion (bit-exact; weighted-vote
scores within rtol 1e-5, the tolerance the path is held to; the
reference's own test allows 1e-4)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import naive
from oracle.drafter import DrafterOracle
from oracle.expand import expand_chain as o_expand
from oracle.local import first_occurrences as o_first_occ
from oracle.local import match_back as o_match_back
from oracle.local import newest_first_pattern
from oracle.sa import build_suffix_array as o_build_sa
from oracle.sa import search_interval as o_search
from tests.conftest import golden

pytestmark = pytest.mark.gpu

I32 = np.int32


def T(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def N(t):
    return t.cpu().numpy()


def test_scatter_append(gpu):
    from suffixgpu_amd import SuffixGPUDrafter
    rng = np.random.default_rng(0)
    b, s, t = 33, 64, 9
    tok = rng.integers(0, 50, size=(b, s)).astype(I32)
    nt = rng.integers(0, s + 5, size=b).astype(I32)
    samp = rng.integers(-1, 50, size=(b, t)).astype(I32)
    samp[3] = -1
    d = SuffixGPUDrafter(k=4, device=gpu, max_pattern_len=8)
    o = DrafterOracle(k=4, max_pattern_len=8)
    for vc in (None, rng.integers(0, t + 1, size=b).astype(np.int64)):
        tg = T(tok, gpu)
        new = d.update_state(T(nt, gpu), tg, T(samp, gpu),
                             None if vc is None else T(vc, gpu))
        to = tok.copy()
        exp = o.update_state(nt, to, samp, vc)
        np.testing.assert_array_equal(N(tg), to)
        np.testing.assert_array_equal(N(new), exp)


def test_match_back_rows_and_shared(gpu):
    from suffixgpu_amd import kernels
    rng = np.random.default_rng(1)
    tok = rng.integers(0, 3, size=(7, 300)).astype(I32)
    q = rng.integers(0, 320, size=7)
    pat = newest_first_pattern(tok, q, 12, -2)
    got = kernels.match_back(T(tok, gpu), T(pat, gpu), 300)
    np.testing.assert_array_equal(N(got), o_match_back(tok, pat, 300))
    delta = rng.integers(-2, 3, size=500).astype(I32)
    got = kernels.match_back(T(delta, gpu), T(pat, gpu), 501)
    np.testing.assert_array_equal(N(got), o_match_back(delta, pat, 501))


def test_first_occurrences(gpu):
    from suffixgpu_amd import kernels
    rng = np.random.default_rng(2)
    mb = rng.integers(0, 6, size=(5, 3000)).astype(I32)
    thr = rng.integers(0, 7, size=(5, 4)).astype(np.int64)
    for r in (1, 7, 128, 600):
        pos, cnt = kernels.first_occurrences(T(mb, gpu), T(thr.reshape(-1),
                                                           gpu), 4, r)
        ep, ec = o_first_occ(mb, thr, r)
        np.testing.assert_array_equal(N(pos), ep.reshape(-1, r))
        np.testing.assert_array_equal(N(cnt), ec.reshape(-1))


@pytest.mark.parametrize("n,vocab", [(1, 3), (2, 2), (7, 2), (64, 3),
                                     (4095, 4), (4097, 50), (20000, 3),
                                     (70000, 30000)])
def test_build_suffix_array(gpu, n, vocab):
    from suffixgpu_amd.suffix_array import build_suffix_array
    rng = np.random.default_rng(n)
    t = rng.integers(-2, vocab, size=n).astype(I32)
    got = build_suffix_array(T(t, gpu))
    np.testing.assert_array_equal(N(got), o_build_sa(t))


@pytest.mark.parametrize("n", [5000, 70000])
def test_build_suffix_array_wide_tokens(gpu, n):
    """Tokens spanning 2^31 values (no pair keys: the token round keys
    each position by its own token, signed order), over several radix
    tiles, with runs that need several doubling rounds."""
    from suffixgpu_amd.suffix_array import build_suffix_array
    rng = np.random.default_rng(n)
    vals = np.array([-2 ** 31, -5, 0, 7, 2 ** 30, 2 ** 31 - 2], np.int64)
    t = vals[rng.integers(0, len(vals), size=n)].astype(I32)
    t[n // 3:n // 3 + 900] = np.tile(t[:30], 30)  # a long repeat
    got = build_suffix_array(T(t, gpu))
    np.testing.assert_array_equal(N(got), o_build_sa(t))


def test_build_suffix_array_structured(gpu):
    from suffixgpu_amd.suffix_array import build_suffix_array
    for toks in ([1, 2, 3, 1, 2, 3, 1, 2], [5] * 5000, [0],
                 [3, -2, 2147483647, 3, -2, 0, 2147483647],
                 [-2147483648, 0, -2147483648, 5, -2147483648],
                 [1, 2] * 3000 + [1]):
        got = build_suffix_array(T(np.array(toks, I32), gpu))
        if len(toks) <= 64:
            assert N(got).tolist() == naive.suffix_array(toks)
        np.testing.assert_array_equal(N(got), o_build_sa(np.array(toks)))


def test_build_suffix_array_template_corpus(gpu):
    """Sequences sharing template spans: long repeats, many rounds, most
    suffixes finished early (the active set shrinks round by round)."""
    from suffixgpu_amd import synth
    from suffixgpu_amd.suffix_array import build_suffix_array
    tc = synth.TemplateCorpus(seed=11)
    docs = [np.append(tc.sequence(lo=1024, hi=4096), -2) for _ in range(90)]
    t = np.concatenate(docs + [np.array([2147483647])]).astype(I32)
    t = np.concatenate([t, t[:5000]])  # one 5000-token exact repeat
    got = build_suffix_array(T(t, gpu))
    np.testing.assert_array_equal(N(got), o_build_sa(t))


def _planted_bigram_text(count: int, seed: int) -> np.ndarray:
    """Random large-alphabet text where the bigram (1, 2) occurs exactly
    `count` times, after the suffixes starting with 0: the group of
    suffixes starting with (1, 2) -- the largest after the token round --
    occupies SA positions from there to there + count, across a
    4096-position tile boundary (asserted)."""
    rng = np.random.default_rng(seed)
    n = 3 * count + 6000
    t = rng.integers(3, 60000, size=n).astype(I32)
    t[rng.choice(n, 4000, replace=False)] = 0
    slots = rng.choice(n // 3 - 1, count, replace=False) * 3
    t[slots] = 1
    t[slots + 1] = 2
    zeros = int(np.sum(t == 0))
    assert zeros < 4096 < zeros + count
    return t


@pytest.mark.parametrize("extra", [0, 1])
def test_build_suffix_array_group_cap(gpu, extra):
    """A round whose largest group has sfx_sa_group_cap() suffixes sorts it
    inside one workgroup (following it into the next tile); one more takes
    the radix path.  The state's radix mask records which path round 1
    took."""
    from suffixgpu_amd import _lib
    from suffixgpu_amd.suffix_array import (build_suffix_array_into,
                                            read_build_state,
                                            sa_workspace_bytes)
    cap = int(_lib.lib().sfx_sa_group_cap())
    count = cap + extra
    t = _planted_bigram_text(count, count)
    exp = o_build_sa(t)
    assert np.sum((t[:-1] == 1) & (t[1:] == 2)) == count
    for adaptive in (True, False):
        ws = torch.empty(sa_workspace_bytes(t.shape[0]), dtype=torch.uint8,
                         device=gpu)
        out = torch.empty(t.shape[0], dtype=torch.int32, device=gpu)
        build_suffix_array_into(T(t, gpu), t.shape[0], out, ws,
                                adaptive=adaptive)
        np.testing.assert_array_equal(N(out), exp)
        st = read_build_state(ws, t.shape[0])
        assert st.done and not st.stalled
        assert bool(st.radix_mask & 2) == (count > cap)


def test_build_suffix_array_stall_and_resume(gpu):
    """Rounds enqueued without the radix path stop at the first round that
    needs it (the state names the round, the rest return at once); the
    same rounds enqueued again from there with the radix path finish the
    array."""
    from suffixgpu_amd import _lib
    from suffixgpu_amd.suffix_array import (build_suffix_array_rounds,
                                            enqueue_rounds, read_build_state,
                                            sa_workspace_bytes)
    t = _planted_bigram_text(5000, 3)
    m = t.shape[0]
    ws = torch.empty(sa_workspace_bytes(m), dtype=torch.uint8, device=gpu)
    out = torch.empty(m, dtype=torch.int32, device=gpu)
    L = _lib.lib()
    total = int(L.sfx_sa_build_rounds_total(m))
    build_suffix_array_rounds(T(t, gpu), m, out, ws, total, radix_mask=0)
    st = read_build_state(ws, m)
    assert not st.done and st.stalled == 1 and st.radix_mask == 1
    enqueue_rounds(m, 1, total, 1 << 1, ws.data_ptr(), ws.numel(),
                   _lib.stream_of(gpu))
    _lib.check(L.sfx_sa_build_finish(m, m, out.data_ptr(), 0, ws.data_ptr(),
                                     ws.numel(), _lib.stream_of(gpu)), "sa")
    st = read_build_state(ws, m)
    assert st.done and not st.stalled and st.radix_mask == 3
    np.testing.assert_array_equal(N(out), o_build_sa(t))


@pytest.mark.parametrize("final_from", [1, 2, 4])
def test_build_suffix_array_expect_final_flag(gpu, final_from):
    """Rounds flagged as expected to find the array final (a rebuild's
    margin rounds) give the same array whether the flag is right or wrong:
    from round 1 every round is flagged, including the token pairs' radix
    round and the rounds that still have groups to sort."""
    from suffixgpu_amd.suffix_array import (build_suffix_array_rounds,
                                            read_build_state,
                                            sa_workspace_bytes)
    rng = np.random.default_rng(11)
    period = rng.integers(0, 5, size=37).astype(I32)
    texts = [_planted_bigram_text(5000, 3),
             np.concatenate([np.tile(period, 300),
                             rng.integers(0, 5, size=900).astype(I32)])]
    for t in texts:
        m = t.shape[0]
        ws = torch.empty(sa_workspace_bytes(m), dtype=torch.uint8,
                         device=gpu)
        out = torch.empty(m, dtype=torch.int32, device=gpu)
        build_suffix_array_rounds(T(t, gpu), m, out, ws, 40,
                                  radix_mask=(1 << 40) - 2,
                                  final_from=final_from)
        st = read_build_state(ws, m)
        assert st.done and not st.stalled
        np.testing.assert_array_equal(N(out), o_build_sa(t))


def test_build_suffix_array_identity_tail(gpu):
    from suffixgpu_amd.suffix_array import build_suffix_array_into
    rng = np.random.default_rng(4)
    t = rng.integers(0, 9, size=1000).astype(I32)
    out = torch.empty(1500, dtype=torch.int32, device=gpu)
    build_suffix_array_into(T(t, gpu), 600, out)
    exp = np.concatenate([o_build_sa(t[:600]), np.arange(600, 1500)])
    np.testing.assert_array_equal(N(out), exp)


@pytest.mark.parametrize("seed", range(3))
def test_sa_search(gpu, seed):
    from suffixgpu_amd.sa_search import search_interval
    rng = np.random.default_rng(seed)
    n = 3000
    toks = rng.integers(0, 4, size=n).astype(I32)
    sa = o_build_sa(toks).astype(I32)
    pats = np.zeros((200, 10), I32)
    lens = np.zeros(200, np.int64)
    for i in range(200):
        m = int(rng.integers(0, 11))
        st = int(rng.integers(0, n - m + 1))
        pats[i, :m] = toks[st:st + m]
        if i % 5 == 0:
            pats[i, :m] = rng.integers(0, 5, size=m)
        lens[i] = m
    s, e = search_interval(T(sa, gpu), T(toks, gpu), T(pats, gpu),
                           T(lens, gpu))
    es, ee = o_search(sa, toks, pats, lens)
    np.testing.assert_array_equal(N(s), es)
    np.testing.assert_array_equal(N(e), ee)


def _rand_expand(rng, b, r, k, vocab=9):
    cont = rng.integers(0, vocab, size=(b, r, k)).astype(I32)
    tail = rng.integers(0, k + 1, size=(b, r))
    cont = np.where(np.arange(k)[None, None, :] < tail[:, :, None], cont, -1)
    occ = rng.integers(0, r + 1, size=b).astype(np.int64)
    cap = rng.integers(-1, k + 2, size=b).astype(np.int64)
    return cont.astype(I32), occ, cap


@pytest.mark.parametrize("r", [1, 4, 30, 128, 256, 700])
@pytest.mark.parametrize("minp", [0.0, 0.1])
def test_expand_chain(gpu, r, minp):
    from suffixgpu_amd.expand import expand_chain
    rng = np.random.default_rng(1234 + r)
    for k, vocab in ((16, 9), (5, 3), (12, 2000)):
        cont, occ, cap = _rand_expand(rng, 37, r, k, vocab)
        got = expand_chain(T(cont, gpu), T(occ, gpu), k,
                           min_token_prob=minp, cap=T(cap, gpu))
        exp = o_expand(cont, occ, k, min_token_prob=minp, cap=cap)
        for g, e in zip(got, exp):
            np.testing.assert_array_equal(N(g), e)


@pytest.mark.parametrize("sentinel", [-7, -2, 0, 4])
def test_expand_chain_other_sentinels(gpu, sentinel):
    """A sentinel other than -1 pads the continuations and -1 is then a
    real token (expand.py:59-66, 107-147): the chain, counts and scores
    equal the oracle's, with and without weights, and int64 blocks keep
    their dtype."""
    from suffixgpu_amd.expand import expand_chain
    rng = np.random.default_rng(77 + sentinel)
    b, r, k = 41, 48, 10
    for lo, hi in ((-3, 6), (sentinel - 2, sentinel + 3)):
        cont = rng.integers(lo, hi, size=(b, r, k))
        tail = rng.integers(0, k + 1, size=(b, r))
        cont = np.where(np.arange(k)[None, None, :] < tail[:, :, None], cont,
                        sentinel)
        occ = rng.integers(0, r + 1, size=b).astype(np.int64)
        cap = rng.integers(-1, k + 2, size=b).astype(np.int64)
        w = rng.random((b, r)).astype(np.float32) + 0.05
        for dt, weights in ((I32, None), (np.int64, None), (I32, w)):
            c = cont.astype(dt)
            got = expand_chain(T(c, gpu), T(occ, gpu), k, sentinel=sentinel,
                               min_token_prob=0.05, cap=T(cap, gpu),
                               weights=None if weights is None
                               else T(weights, gpu))
            exp = o_expand(c, occ, k, sentinel=sentinel, min_token_prob=0.05,
                           cap=cap, weights=weights)
            assert got[0].dtype == T(c, gpu).dtype
            for g, e in zip(got[:3], exp[:3]):
                np.testing.assert_array_equal(N(g), e)
            if weights is None:
                np.testing.assert_array_equal(N(got[3]), exp[3])
            else:
                np.testing.assert_allclose(N(got[3]), exp[3], rtol=1e-5,
                                           atol=0)


@pytest.mark.parametrize("i", range(4))
def test_expand_alpha_weights_golden(gpu, i):
    from suffixgpu_amd.expand import expand_chain
    z = golden("expand_alpha_weights")
    cont, occ, cap = z[f"cont_{i}"], z[f"occ_{i}"], z[f"cap_{i}"]
    k = cont.shape[2]
    got = expand_chain(T(cont, gpu), T(occ, gpu), k, min_token_prob=0.05,
                       cap=T(cap, gpu), alpha=float(z[f"alpha_{i}"]))
    for g, key in zip(got, ("chain", "nv", "emit", "score")):
        np.testing.assert_array_equal(N(g), z[f"{key}_{i}"], err_msg=key)
    got = expand_chain(T(cont, gpu), T(occ, gpu), k, min_token_prob=0.05,
                       cap=T(cap, gpu), weights=T(z[f"w_{i}"], gpu))
    for g, key in zip(got[:3], ("wchain", "wnv", "wemit")):
        np.testing.assert_array_equal(N(g), z[f"{key}_{i}"], err_msg=key)
    np.testing.assert_allclose(N(got[3]), z[f"wscore_{i}"], rtol=1e-5,
                               atol=0)


def test_expand_division_table(gpu):
    """Every vote fraction v/n, 1 <= v <= n <= 128, is the IEEE fp32
    quotient: a one-depth chain of n occurrences with v equal tokens."""
    from suffixgpu_amd.expand import expand_chain
    rows = [(v, n) for n in range(1, 129) for v in range(1, n + 1)]
    b = len(rows)
    cont = np.full((b, 128, 1), -1, I32)
    occ = np.zeros(b, np.int64)
    for i, (v, n) in enumerate(rows):
        cont[i, :n, 0] = np.arange(1000, 1000 + n)
        cont[i, :v, 0] = 7
        occ[i] = n
    for alpha in (0.0, 0.5):
        _, _, _, score = expand_chain(T(cont, gpu), T(occ, gpu), 1,
                                      alpha=alpha)
        exp = np.array([np.float32(v) / (np.float32(max(n, 1)) +
                                         np.float32(alpha))
                        for v, n in rows], np.float32)
        np.testing.assert_array_equal(N(score), exp)


@pytest.mark.parametrize("start,n", [(1, 39999), (100, 30000), (8191, 8192),
                                     (20000, 20000), (0, 123), (5, 0)])
def test_delta_shift_in_place(gpu, start, n):
    """delta[:n] = delta[start:start + n] in place, overlapping windows
    included, and the device length set to n; the rest is untouched."""
    from suffixgpu_amd import _lib
    rng = np.random.default_rng(start + n)
    cap = 40000
    host = rng.integers(0, 1 << 30, size=cap).astype(I32)
    dl = torch.full((), -7, dtype=torch.int64, device=gpu)
    d = torch.from_numpy(host).to(gpu)
    rc = _lib.lib().sfx_delta_shift(d.data_ptr(), cap, start, n,
                                    dl.data_ptr(),
                                    torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == 0
    want = host.copy()
    want[:n] = host[start:start + n]
    np.testing.assert_array_equal(d.cpu().numpy(), want)
    assert int(dl.item()) == n


def test_delta_append_groups(gpu):
    """150 documents (three launches of at most 64) at host-chosen offsets,
    a zero-length one among them; each followed by SEP, length set."""
    from suffixgpu_amd import _lib
    rng = np.random.default_rng(3)
    cap = 30000
    d = torch.full((cap,), 77, dtype=torch.int32, device=gpu)
    dl = torch.zeros((), dtype=torch.int64, device=gpu)
    want = np.full(cap, 77, dtype=I32)
    srcs, descs, off = [], [], 0
    for i in range(150):
        n = 0 if i == 17 else int(rng.integers(1, 150))
        x = rng.integers(0, 1000, size=n).astype(I32)
        t = torch.from_numpy(x).to(gpu)
        srcs.append(t)
        descs.append(_lib.SfxAppendDoc(t.data_ptr(), n, off))
        want[off:off + n] = x
        want[off + n] = -2
        off += n + 1
    arr = (_lib.SfxAppendDoc * len(descs))(*descs)
    rc = _lib.lib().sfx_delta_append(arr, len(descs), d.data_ptr(), cap,
                                     dl.data_ptr(), off,
                                     torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == 0
    np.testing.assert_array_equal(d.cpu().numpy(), want)
    assert int(dl.item()) == off


@pytest.mark.parametrize("weighted", [False, True])
def test_majority_token_vs_oracle(gpu, weighted):
    """expand._majority_token (a one-depth expansion) against the oracle's
    pairwise vote.  Weights are multiples of 1/8, so every weight sum is
    exact in fp32 whatever the summation order, and tokens and counts
    compare exactly."""
    from oracle.expand import majority_token as o_major
    from suffixgpu_amd.expand import _majority_token
    rng = np.random.default_rng(17)
    b, r = 96, 40
    vals = rng.integers(0, 6, size=(b, r)).astype(np.int64)
    act = rng.random((b, r)) < 0.7
    act[:4] = False  # rows with no active entry
    w = ((rng.integers(1, 9, size=(b, r)) / 8).astype(np.float32)
         if weighted else None)
    tok, cnt = _majority_token(T(vals, gpu), T(act, gpu), -5,
                               None if w is None else T(w, gpu))
    etok, ecnt = o_major(vals, act, -5, w)
    np.testing.assert_array_equal(N(tok), etok)
    np.testing.assert_array_equal(N(cnt), ecnt)
