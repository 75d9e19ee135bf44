"""Local (per-request) multi-length suffix matcher -- numpy restatement.

Follows suffix_gpu/local_matcher.py:76-263 and the tail gather of
suffix_gpu/proposer.py:110-125.
"""

from __future__ import annotations

import numpy as np

from oracle.expand import F32, expand_chain


def spec_cap(match_len: np.ndarray, k: int, factor: float | None,
             offset: float) -> np.ndarray:
    """local_matcher.py:76-81: max(0, floor(fl32(f)*fl32(L) + fl32(off)))."""
    if factor is None:
        return np.full(match_len.shape, k, dtype=np.int64)
    v = (F32(factor) * match_len.astype(F32)).astype(F32)
    v = (v + F32(offset)).astype(F32)
    return np.maximum(np.floor(v).astype(np.int64), 0)


def gather_tails(num_tokens: np.ndarray, tok: np.ndarray, p: int
                 ) -> tuple[np.ndarray, np.ndarray]:
    """proposer.py:110-125: last min(q, P) tokens, left-aligned, 0 padded."""
    b, s = tok.shape
    q = num_tokens.astype(np.int64)
    tail_len = np.minimum(q, p)
    offs = np.arange(p, dtype=np.int64)
    idx = q[:, None] - tail_len[:, None] + offs[None, :]
    valid = offs[None, :] < tail_len[:, None]
    vals = np.take_along_axis(tok, np.clip(idx, 0, s - 1), axis=1)
    return np.where(valid, vals, 0).astype(tok.dtype), tail_len


def newest_first_pattern(src: np.ndarray, src_len: np.ndarray, p: int,
                         fill: int) -> np.ndarray:
    """pat[b,t] = src[b, clamp(len-1-t)] if len-1-t >= 0 else fill.

    Local pattern with fill -2 (local_matcher.py:103-112) and delta pattern
    with fill -3 over the query tails (global_index.py:493-501).
    """
    w = src.shape[1]
    offs = np.arange(p, dtype=np.int64)
    idx = src_len.astype(np.int64)[:, None] - 1 - offs[None, :]
    vals = np.take_along_axis(src, np.clip(idx, 0, w - 1), axis=1)
    return np.where(idx >= 0, vals, fill).astype(np.int32)


def match_back(src: np.ndarray, pat: np.ndarray, n_out: int) -> np.ndarray:
    """mb[b,i] = #leading t with x(i-1-t) == pat[b,t]; x(j<0) = -1.

    local_matcher.py:114-126 (rows [B,S]) and global_index.py:503-515 (the
    shared 1-D delta).  Rolling AND over the P pattern offsets.
    """
    b, p = pat.shape
    rows = src if src.ndim == 2 else src[None, :]
    lp = np.concatenate(
        [np.full((rows.shape[0], p), -1, dtype=rows.dtype), rows], axis=1)
    acc = np.ones((b, n_out), dtype=bool)
    mb = np.zeros((b, n_out), dtype=np.int32)
    for t in range(p):
        seg = lp[:, p - 1 - t:p - 1 - t + n_out]
        acc &= seg == pat[:, t:t + 1]
        mb += acc
    return mb


def first_occurrences(mb: np.ndarray, thr: np.ndarray, r: int
                      ) -> tuple[np.ndarray, np.ndarray]:
    """First r ascending i with mb[b,i] >= thr[b,c] (thr>0), zero padded.

    local_matcher.py:160-184 / triton_kernels.py:217-243.  ``mb`` must be
    zeroed at invalid positions.  Returns (pos [B,C,r] i64, count [B,C] i64).
    """
    b, c = thr.shape
    pos = np.zeros((b, c, r), dtype=np.int64)
    cnt = np.zeros((b, c), dtype=np.int64)
    for i in range(b):
        for j in range(c):
            t = int(thr[i, j])
            if t <= 0:
                continue
            hits = np.flatnonzero(mb[i] >= t)[:r]
            pos[i, j, :hits.shape[0]] = hits
            cnt[i, j] = hits.shape[0]
    return pos, cnt


def candidates(mb: np.ndarray, thresholds: np.ndarray, min_match_len: int,
               mask: np.ndarray) -> np.ndarray:
    """local_matcher.py:134-157: thr-th largest mb, zeroed and deduped."""
    b, s = mb.shape
    thr = thresholds.astype(np.int64)
    w = min(int(thr.max()), s)
    top = -np.sort(-mb, axis=1)[:, :w]
    tidx = np.clip(thr - 1, 0, w - 1)
    cand = top[:, tidx].astype(np.int64)
    cand = np.where(thr[None, :] > w, 0, cand)
    cand = np.where((cand >= max(1, min_match_len)) & mask[:, None], cand, 0)
    if cand.shape[1] > 1:
        dup = np.zeros_like(cand, dtype=bool)
        dup[:, 1:] = cand[:, 1:] == cand[:, :-1]
        cand = np.where(dup, 0, cand)
    return cand


class LocalMatcher:
    """Restatement of LocalMatchKernel (local_matcher.py:49-242)."""

    def __init__(self, k: int, max_pattern_len: int = 32,
                 min_match_len: int = 1, max_occurrences: int = 32,
                 min_token_prob: float = 0.0,
                 max_spec_factor: float | None = None,
                 max_spec_offset: float = 0.0,
                 support_thresholds=(1, 2, 4, 8),
                 vote_smoothing_alpha: float = 0.0):
        self.k = k
        self.max_pattern_len = max_pattern_len
        self.min_match_len = max(1, min_match_len)
        self.max_occurrences = max_occurrences
        self.min_token_prob = min_token_prob
        self.max_spec_factor = max_spec_factor
        self.max_spec_offset = max_spec_offset
        self.vote_smoothing_alpha = vote_smoothing_alpha
        self.support_thresholds = tuple(int(t) for t in support_thresholds)
        if not self.support_thresholds:
            raise ValueError("support_thresholds must be non-empty")
        self.thresholds = np.array(self.support_thresholds, dtype=np.int64)

    def spec_cap(self, match_len: np.ndarray) -> np.ndarray:
        return spec_cap(match_len, self.k, self.max_spec_factor,
                        self.max_spec_offset)

    def match(self, num_tokens: np.ndarray, tok: np.ndarray) -> np.ndarray:
        """match_back zeroed past the committed length (:103-132)."""
        b, s = tok.shape
        q = num_tokens.astype(np.int64)
        pat = newest_first_pattern(tok, q, self.max_pattern_len, -2)
        mb = match_back(tok, pat, s)
        valid = np.arange(s, dtype=np.int64)[None, :] < q[:, None]
        return np.where(valid, mb, 0).astype(np.int32)

    def gather_candidates(self, num_tokens: np.ndarray, tok: np.ndarray,
                          mask: np.ndarray):
        """(cand [B,C] i64, cont [B,C,R,K] i32, occ_count [B,C] i64)."""
        b, s = tok.shape
        k, r = self.k, self.max_occurrences
        q = num_tokens.astype(np.int64)
        mb = self.match(num_tokens, tok)
        cand = candidates(mb, self.thresholds, self.min_match_len,
                          mask.astype(bool))
        occ_end, occ_count = first_occurrences(mb, cand, r)
        idx = occ_end[:, :, :, None] + np.arange(k, dtype=np.int64)
        row_active = (np.arange(r)[None, None, :] < occ_count[:, :, None])
        valid = (idx < q[:, None, None, None]) & row_active[:, :, :, None]
        flat = np.clip(idx, 0, s - 1).reshape(b, -1)
        vals = np.take_along_axis(tok, flat, axis=1).reshape(idx.shape)
        cont = np.where(valid, vals, -1).astype(np.int32)
        return cand, cont, occ_count

    def forward(self, num_tokens: np.ndarray, tok: np.ndarray,
                mask: np.ndarray):
        """(draft [B,K] i32, nv [B] i32, len i64, occ i64, score f32)."""
        b = tok.shape[0]
        k, r = self.k, self.max_occurrences
        cand, cont, occ = self.gather_candidates(num_tokens, tok, mask)
        c = cand.shape[1]
        cap = self.spec_cap(cand.reshape(-1))
        chain, _, emit, score = expand_chain(
            cont.reshape(b * c, r, k), occ.reshape(-1), k,
            min_token_prob=self.min_token_prob, cap=cap,
            alpha=self.vote_smoothing_alpha)
        sel = select_local_best(cand, chain.reshape(b, c, k),
                                emit.reshape(b, c), occ, score.reshape(b, c))
        ch, em, ln, oc, sc = sel
        slot = np.arange(k)[None, :]
        ch = np.where(slot < em[:, None], ch, -1)
        return (ch.astype(np.int32), em.astype(np.int32), ln, oc, sc)


def select_local_best(cand, chain, emit, occ, score):
    """local_matcher.py:245-263: first argmax of score + fl32(len)*fl32(1e-6)."""
    b = cand.shape[0]
    tie = (cand.astype(F32) * F32(1e-6)).astype(F32)
    best = (score.astype(F32) + tie).astype(F32).argmax(axis=1)
    i = np.arange(b)
    return chain[i, best], emit[i, best], cand[i, best], occ[i, best], \
        score[i, best]
