"""Local matcher on gfx950 vs the oracle (and the reference's goldens)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.drafter import DrafterOracle, backoff_thresholds
from oracle.local import LocalMatcher
from suffixgpu_amd import synth
from tests.conftest import golden

pytestmark = pytest.mark.gpu

I32 = np.int32


def T(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def N(t):
    return t.cpu().numpy()


def _pair(gpu, **kw):
    from suffixgpu_amd.local_matcher import LocalMatchKernel
    return LocalMatchKernel(**kw), LocalMatcher(**kw)


def _check(gpu, g, o, nt, tok, mask):
    cand, cont, occ = g.gather_candidates(T(nt, gpu), T(tok, gpu),
                                          T(mask, gpu))
    ec, econt, eocc = o.gather_candidates(nt, tok, mask)
    np.testing.assert_array_equal(N(cand), ec)
    np.testing.assert_array_equal(N(occ), eocc)
    np.testing.assert_array_equal(N(cont), econt)
    fw = g(T(nt, gpu), T(tok, gpu), T(mask, gpu))
    efw = o.forward(nt, tok, mask)
    for a, b, name in zip(fw, efw, ("draft", "nv", "len", "occ", "score")):
        np.testing.assert_array_equal(N(a), b, err_msg=name)


def test_local_uniform_golden(gpu):
    z = golden("local_uniform")
    from suffixgpu_amd.local_matcher import LocalMatchKernel
    g = LocalMatchKernel(k=16, max_pattern_len=32, max_occurrences=128,
                         support_thresholds=(1,))
    cand, cont, occ = g.gather_candidates(
        T(z["num_tokens"], gpu), T(z["tokens"], gpu),
        torch.ones(8, dtype=torch.bool, device=gpu))
    np.testing.assert_array_equal(N(cand), z["cand"])
    np.testing.assert_array_equal(N(occ), z["occ"])
    np.testing.assert_array_equal(N(cont), z["cont"])


def test_local_zipf_forward_golden(gpu):
    z = golden("local_zipf_update")
    from suffixgpu_amd.local_matcher import LocalMatchKernel
    g = LocalMatchKernel(k=16, max_pattern_len=32, max_occurrences=128,
                         max_spec_factor=2.0, min_token_prob=0.1,
                         support_thresholds=backoff_thresholds(8))
    fw = g(T(z["new_counts"], gpu), T(z["tokens_after"], gpu),
           torch.ones(12, dtype=torch.bool, device=gpu))
    for a, key in zip(fw, ("fw_draft", "fw_nv", "fw_len", "fw_occ",
                           "fw_score")):
        np.testing.assert_array_equal(N(a), z[key], err_msg=key)


def test_local_ties_golden(gpu):
    z = golden("local_ties")
    kw = dict(k=8, max_pattern_len=12, max_occurrences=16,
              max_spec_factor=0.7, max_spec_offset=0.3, min_token_prob=0.05,
              support_thresholds=backoff_thresholds(6),
              vote_smoothing_alpha=0.5)
    g, o = _pair(gpu, **kw)
    fw = g(T(z["num_tokens"], gpu), T(z["tokens"], gpu), T(z["mask"], gpu))
    np.testing.assert_array_equal(N(fw[2]), z["fw_len"])
    np.testing.assert_array_equal(N(fw[3]), z["fw_occ"])
    np.testing.assert_array_equal(N(fw[4]), z["fw_score"])
    _check(gpu, g, o, z["num_tokens"], z["tokens"], z["mask"])


@pytest.mark.parametrize("vocab,s,r,p", [(3, 200, 8, 6), (5, 1000, 16, 12),
                                         (50, 3000, 128, 32),
                                         (2, 257, 300, 40), (4, 999, 16, 2),
                                         (60, 20000, 64, 70),
                                         (3, 20001, 32, 100)])
def test_local_random(gpu, vocab, s, r, p):
    rng = np.random.default_rng(vocab * 1000 + s)
    b = 9
    tok = rng.integers(0, vocab, size=(b, s)).astype(I32)
    nt = rng.integers(0, s + 1, size=b).astype(np.int64)
    nt[0], nt[1], nt[2] = 0, 1, s + 7   # empty, one token, past the buffer
    mask = rng.random(b) < 0.85
    g, o = _pair(gpu, k=7, max_pattern_len=p, max_occurrences=r,
                 max_spec_factor=1.5, max_spec_offset=0.5,
                 min_token_prob=0.02,
                 support_thresholds=(1, 2, 3, 8, 64, 1 << 20))
    _check(gpu, g, o, nt, tok, mask)


def test_local_synth_workloads(gpu):
    for w, nb, f, minp in ((synth.local_uniform(seed=1), 1, None, 0.0),
                           (synth.local_zipf(seed=2, b=16), 8, 2.0, 0.1)):
        g, o = _pair(gpu, k=16, max_pattern_len=32, max_occurrences=128,
                     max_spec_factor=f, min_token_prob=minp,
                     support_thresholds=backoff_thresholds(nb))
        _check(gpu, g, o, w.num_tokens, w.tokens,
               np.ones(w.tokens.shape[0], bool))


def test_local_drafter_propose_matches_oracle(gpu):
    from suffixgpu_amd import SuffixGPUDrafter
    w = synth.local_zipf(seed=2, b=32, s=8192)
    kw = dict(k=16, max_pattern_len=32, max_occurrences=128, num_backoff=8,
              max_spec_factor=2.0, min_token_prob=0.1)
    d = SuffixGPUDrafter(device=gpu, **kw)
    o = DrafterOracle(**kw)
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


def _long_rows(seed, s, vocab, q_list, p):
    """Rows longer than fit in LDS.  Suffixes of each row's last p tokens
    are planted so that match ends fall on both sides of the 16384- and
    8192-position chunk boundaries and at the first position, with varied
    match lengths."""
    rng = np.random.default_rng(seed)
    b = len(q_list)
    tok = rng.integers(0, vocab, size=(b, s)).astype(I32)
    nt = np.array(q_list, dtype=np.int64)
    for i in range(b):
        q = int(min(nt[i], s))
        if q < 4 * p:
            continue
        tail = tok[i, q - p:q].copy()
        for j, end in enumerate((p, 8192, 8193, 16384, 16385, 16384 + p // 2,
                                 24575, 32768 - 3, 32768 + 1, q - p - 1)):
            ln = (p, p // 2, 3, p - 1)[j % 4]
            if ln <= end <= q - p:
                tok[i, end - ln:end] = tail[p - ln:]
    return tok, nt


@pytest.mark.parametrize("vocab", [3, 1000])
@pytest.mark.parametrize("s", [40000, 70001])
def test_local_long_rows_streamed(gpu, vocab, s):
    """Rows of 40K-70K tokens take the streamed path (chunks of 16384 or
    8192 positions, the whole row's match lengths kept in LDS):
    committed lengths of 0, 1, inside the first chunk, on and just past a
    chunk boundary, full and past the buffer."""
    q_list = [0, 1, 5000, 16384, 16385, 16400, 32769, s, s + 7]
    tok, nt = _long_rows(vocab * 7 + s, s, vocab, q_list, 32)
    mask = np.ones(len(q_list), bool)
    mask[2] = False
    g, o = _pair(gpu, k=16, max_pattern_len=32, max_occurrences=128,
                 max_spec_factor=2.0, min_token_prob=0.1,
                 support_thresholds=backoff_thresholds(8))
    _check(gpu, g, o, nt, tok, mask)


def test_local_rows_beyond_the_match_array(gpu):
    """Rows of 140,000 tokens: their match lengths do not fit in LDS beside
    the smallest chunk, so the chunks are staged twice (histogram pass,
    then the ordered compaction with counts carried between chunks)."""
    s = 140_000
    q_list = [16383, 16385, 70000, s]
    tok, nt = _long_rows(s + 11, s, 40, q_list, 32)
    g, o = _pair(gpu, k=16, max_pattern_len=32, max_occurrences=128,
                 max_spec_factor=2.0, min_token_prob=0.1,
                 support_thresholds=backoff_thresholds(8))
    _check(gpu, g, o, nt, tok, np.ones(len(q_list), bool))


def test_local_long_rows_small_chunks(gpu):
    """k = 2048 with eight thresholds leaves room for 8192-position chunks
    only: a 20000-token row is streamed in three chunks (five at
    S = 40000)."""
    for s in (20000, 40000):
        q_list = [8191, 8192, 8193, 12000, s]
        tok, nt = _long_rows(s, s, 50, q_list, 24)
        g, o = _pair(gpu, k=2048, max_pattern_len=24, max_occurrences=64,
                     max_spec_factor=None, min_token_prob=0.0,
                     support_thresholds=(1, 2, 3, 5, 8, 16, 64, 1000))
        _check(gpu, g, o, nt, tok, np.ones(len(q_list), bool))


@pytest.mark.parametrize("s,t,vocab,p,holes", [(8192, 17, 1000, 32, False),
                                                (20000, 17, 4, 32, False),
                                                (20001, 80, 50, 100, True),
                                                (16384, 17, 3, 3, True)])
def test_step_resident_rows_vs_oracle(gpu, s, t, vocab, p, holes):
    """Local-only propose_with_update on rows that fit in LDS (each thread
    matches 16, 32 or 48 consecutive ends): committed lengths at 16-end
    chunk edges, the row start and past the buffer; copy-span rows over
    small vocabularies (long matches that walk past the first four
    pattern tokens); more sampled ids than a wave has lanes; an explicit
    valid count with -1 holes among the counted ids; S not a multiple of 4;
    patterns longer than 64 and shorter than 4."""
    from suffixgpu_amd import SuffixGPUDrafter
    rng = np.random.default_rng(s + t + vocab)
    q_list = [0, 1, 15, 16, 17, 4095, 8191, 8192, 12000, s - t - 1, s - 3, s,
              s + 5]
    b = len(q_list)
    draw = synth.uniform_draw(vocab)
    hidden = np.stack([synth.build_row(rng, s + t, draw) for _ in range(b)])
    rows = hidden[:, :s].copy()
    nt = np.array([min(q, s) if q >= 0 else 0 for q in q_list], dtype=I32)
    nt[-1] = s + 5
    sampled = np.full((b, t), -1, dtype=I32)
    cnt = np.zeros(b, dtype=I32)
    for i in range(b):
        acc = int(rng.integers(0, t + 1)) if i % 4 else t
        st = int(min(nt[i], s))
        seg = hidden[i, st:st + acc]
        sampled[i, :seg.shape[0]] = seg
        cnt[i] = acc
        if holes and acc > 2:
            sampled[i, acc // 2] = -1
    kw = dict(k=16, max_pattern_len=p, max_occurrences=128, num_backoff=8,
              max_spec_factor=2.0, min_token_prob=0.1)
    d = SuffixGPUDrafter(device=gpu, **kw)
    o = DrafterOracle(**kw)
    tg = T(rows, gpu)
    vc = T(cnt, gpu) if holes else None
    draft, nv, new = d.propose_with_update(T(nt, gpu), tg, T(sampled, gpu),
                                           vc)
    to = rows.copy()
    ed, env, enew = o.propose_with_update(nt, to, sampled,
                                          cnt if holes else None)
    np.testing.assert_array_equal(N(tg), to)
    np.testing.assert_array_equal(N(new), enew)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)
    assert (env > 0).sum() > 0
