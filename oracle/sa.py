"""Suffix array construction and interval search -- numpy restatement.

* ``build_suffix_array`` follows suffix_gpu/suffix_array.py:15-63 (prefix
  doubling over dense ranks of the signed int64 token order, the
  out-of-range second key sorting first).  The result is the unique suffix
  array, so the early exit once every rank is distinct changes nothing.
* ``search_interval`` follows sa_search.py:66-107 with the comparison of
  sa_search.py:25-63: fixed ceil(log2(n+1)) iterations, merged lower/upper
  bound, corpus reads at or past n compare as -1.
* ``suffix_match_backoff`` / ``longest_suffix_match`` follow
  sa_search.py:110-185.
"""

from __future__ import annotations

import math

import numpy as np


def build_suffix_array(tokens: np.ndarray) -> np.ndarray:
    tokens = np.asarray(tokens).reshape(-1)
    n = tokens.shape[0]
    if n == 0:
        return np.empty(0, dtype=np.int64)
    if n == 1:
        return np.zeros(1, dtype=np.int64)
    rank = np.unique(tokens.astype(np.int64), return_inverse=True)[1]
    rank = rank.reshape(-1).astype(np.int64)
    base = n + 1
    k = 1
    sa = np.argsort(rank, kind="stable")
    rounds = max(1, math.ceil(math.log2(n)))
    for _ in range(rounds):
        second = np.zeros(n, dtype=np.int64)
        if k < n:
            second[:-k] = rank[k:] + 1
        key = rank * base + second
        sa = np.argsort(key, kind="stable")
        sk = key[sa]
        distinct = np.ones(n, dtype=np.int64)
        distinct[1:] = sk[1:] != sk[:-1]
        new_sorted = np.cumsum(distinct) - 1
        rank = np.empty_like(rank)
        rank[sa] = new_sorted
        k *= 2
        if new_sorted[-1] == n - 1:
            break
    return sa.astype(np.int64)


def cmp_pattern(sa: np.ndarray, corpus: np.ndarray, mid: np.ndarray,
                pattern: np.ndarray, plen: np.ndarray) -> np.ndarray:
    """sa_search.py:25-63: -1 suffix < pattern, 0 starts with it, +1 >."""
    n = sa.shape[0]
    m = pattern.shape[1]
    pos = sa[mid].astype(np.int64)
    offs = np.arange(m, dtype=np.int64)
    idx = pos[:, None] + offs[None, :]
    tok = np.where(idx < n, corpus[np.clip(idx, 0, n - 1)], -1)
    pat_valid = offs[None, :] < plen[:, None]
    eq_ok = (tok == pattern) | ~pat_valid
    lcp_raw = np.cumprod(eq_ok.astype(np.int64), axis=1).sum(axis=1)
    lcp = np.minimum(lcp_raw, plen)
    full = lcp >= plen
    spos = np.clip(pos + lcp, 0, n - 1)
    schar = np.where(pos + lcp < n, corpus[spos], -1).astype(np.int64)
    pchar = np.take_along_axis(
        pattern, np.minimum(lcp, m - 1)[:, None], axis=1)[:, 0].astype(
            np.int64)
    c = np.where(schar < pchar, -1, np.where(schar > pchar, 1, 0))
    return np.where(full, 0, c)


def search_interval(sa: np.ndarray, corpus: np.ndarray, pattern: np.ndarray,
                    plen: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    n = sa.shape[0]
    iters = max(1, math.ceil(math.log2(n + 1)))
    b = pattern.shape[0]
    pat2 = np.concatenate([pattern, pattern], axis=0)
    plen2 = np.concatenate([plen, plen]).astype(np.int64)
    upper = np.zeros(2 * b, dtype=bool)
    upper[b:] = True
    lo = np.zeros(2 * b, dtype=np.int64)
    hi = np.full(2 * b, n, dtype=np.int64)
    for _ in range(iters):
        mid = np.minimum((lo + hi) // 2, n - 1)
        c = cmp_pattern(sa, corpus, mid, pat2, plen2)
        go = (c < 0) | (upper & (c == 0))
        lo = np.where(go, mid + 1, lo)
        hi = np.where(go, hi, mid)
    return lo[:b], lo[b:]


def suffix_match_backoff(sa, corpus, query, query_len, max_len, caps):
    """(len [B,C], start [B,C], end [B,C]); (0,0) where nothing matched."""
    b, q = query.shape
    m = max_len
    lengths = np.arange(1, m + 1, dtype=np.int64)
    offs = np.arange(m, dtype=np.int64)
    qlen = query_len.astype(np.int64)
    idx = qlen[:, None, None] - lengths[None, :, None] + offs[None, None, :]
    valid = (offs[None, None, :] < lengths[None, :, None]) & (idx >= 0)
    tok = np.take_along_axis(query, np.clip(idx, 0, q - 1).reshape(b, m * m),
                             axis=1).reshape(b, m, m)
    pat = np.where(valid, tok, 0).astype(np.int64)
    start, end = search_interval(sa, corpus, pat.reshape(b * m, m),
                                 np.tile(lengths, b))
    start = start.reshape(b, m)
    end = end.reshape(b, m)
    found = (end > start) & (lengths[None, :] <= qlen[:, None])
    found_len = found.astype(np.int64) * lengths[None, :]
    within = lengths[None, None, :] <= np.asarray(caps).reshape(1, -1, 1)
    best = (found_len[:, None, :] * within).max(axis=2)
    pick = np.maximum(best - 1, 0)
    s = np.take_along_axis(start, pick, axis=1)
    e = np.take_along_axis(end, pick, axis=1)
    return best, np.where(best > 0, s, 0), np.where(best > 0, e, 0)


def longest_suffix_match(sa, corpus, query, query_len, max_len):
    caps = np.array([max_len], dtype=np.int64)
    best, s, e = suffix_match_backoff(sa, corpus, query, query_len, max_len,
                                      caps)
    return best[:, 0], s[:, 0], e[:, 0]
