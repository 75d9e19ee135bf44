"""Brute-force definitions on plain Python lists (tiny inputs only).

Textbook definitions of the quantities the drafter computes, written from
the mathematics rather than from the reference's vectorised code:

* suffix array: positions sorted by suffix, a proper prefix sorting first
  (mirrors suffix_gpu/reference.py:16-19);
* interval search: the half-open range of SA ranks whose suffix starts with
  the pattern, a read past the end comparing smaller (reference.py:22-62);
* occurrences and longest suffix match (reference.py:65-79);
* the local multi-length backoff drafter (reference.py:82-157) and the
  global chain of tests/test_global_index.py:17-42.
"""

from __future__ import annotations

from collections import Counter
from collections.abc import Sequence


def suffix_array(tokens: Sequence[int]) -> list[int]:
    n = len(tokens)
    return sorted(range(n), key=lambda i: tuple(tokens[i:]))


def suffix_cmp(tokens: Sequence[int], pos: int,
               pattern: Sequence[int]) -> int:
    """-1 / 0 / +1: suffix < pattern, suffix starts with pattern, suffix >."""
    n = len(tokens)
    for j, t in enumerate(pattern):
        if pos + j >= n:
            return -1
        if tokens[pos + j] != t:
            return -1 if tokens[pos + j] < t else 1
    return 0


def search_interval(sa: Sequence[int], tokens: Sequence[int],
                    pattern: Sequence[int]) -> tuple[int, int]:
    """Linear scan: first rank with cmp >= 0 and first rank with cmp > 0."""
    cmps = [suffix_cmp(tokens, p, pattern) for p in sa]
    lo = next((i for i, c in enumerate(cmps) if c >= 0), len(sa))
    hi = next((i for i, c in enumerate(cmps) if c > 0), len(sa))
    return lo, max(lo, hi)


def occurrences(tokens: Sequence[int], pattern: Sequence[int]) -> list[int]:
    m = len(pattern)
    return [i for i in range(len(tokens) - m + 1)
            if list(tokens[i:i + m]) == list(pattern)]


def longest_suffix_match(tokens: Sequence[int], query: Sequence[int],
                         max_len: int) -> int:
    best = 0
    for ln in range(1, min(max_len, len(query)) + 1):
        if occurrences(tokens, query[len(query) - ln:]):
            best = ln
    return best


def local_match(tokens: Sequence[int], k: int, max_pattern_len: int,
                min_match_len: int = 1, max_occurrences: int = 32,
                min_token_prob: float = 0.0,
                max_spec_factor: float | None = None,
                max_spec_offset: float = 0.0,
                support_thresholds: Sequence[int] = (1, 2, 4, 8),
                ) -> tuple[list[int], int]:
    """Multi-length backoff drafter over one committed history.

    Candidate for support t: the longest suffix length L <= P whose
    occurrences ending before the history end (end index i in [L, q)) number
    at least t.  Each candidate drafts by depth-wise majority vote (ties to
    the smallest token) over its first ``max_occurrences`` occurrences, stops
    when the running vote-fraction product drops below ``min_token_prob``,
    is truncated to floor(f*L + off) and scored by the sum of the products
    it emits.  Highest score wins; equal scores prefer the longer match.
    """
    q = len(tokens)
    occ: dict[int, list[int]] = {}
    for ln in range(1, min(max_pattern_len, q - 1) + 1 if q > 1 else 0):
        pat = list(tokens[q - ln:])
        ends = [i for i in range(ln, q) if list(tokens[i - ln:i]) == pat]
        if ends:
            occ[ln] = ends
    cands = []
    for t in support_thresholds:
        best = max([ln for ln, e in occ.items() if len(e) >= t], default=0)
        if best >= max(1, min_match_len):
            cands.append(best)
    best_chain: list[int] = []
    best_len, best_score = 0, -1.0
    for lc in cands:
        active = occ[lc][:max_occurrences]
        chain: list[int] = []
        cums: list[float] = []
        cum = 1.0
        for d in range(k):
            live = [i for i in active if i + d < q]
            if not live:
                break
            cnt = Counter(tokens[i + d] for i in live)
            top = max(cnt.items(), key=lambda kv: (kv[1], -kv[0]))[0]
            nxt = cum * cnt[top] / len(live)
            if min_token_prob > 0 and nxt < min_token_prob:
                break
            cum = nxt
            chain.append(top)
            cums.append(cum)
            active = [i for i in live if tokens[i + d] == top]
        cap = k if max_spec_factor is None else max(
            0, int(max_spec_factor * lc + max_spec_offset + 1e-9))
        emit = min(len(chain), cap)
        score = sum(cums[:emit])
        if score > best_score or (score == best_score and lc > best_len):
            best_chain, best_len, best_score = chain[:emit], lc, score
    if best_len == 0:
        return [], 0
    return best_chain, best_len


def global_chain(docs: Sequence[Sequence[int]], query: Sequence[int], k: int,
                 max_len: int, max_occurrences: int) -> tuple[list[int], int]:
    """Longest-suffix match over SEP(-2)-joined docs, then majority chain."""
    corpus: list[int] = []
    for d in docs:
        corpus.extend(d)
        corpus.append(-2)
    ln = longest_suffix_match(corpus, query, max_len)
    if ln == 0:
        return [], 0
    active = occurrences(corpus, query[len(query) - ln:])[:max_occurrences]
    chain: list[int] = []
    for _ in range(k):
        pos = ln + len(chain)
        toks = [corpus[s + pos] for s in active
                if s + pos < len(corpus) and corpus[s + pos] >= 0]
        if not toks:
            break
        cnt = Counter(toks)
        top = max(cnt.items(), key=lambda kv: (kv[1], -kv[0]))[0]
        chain.append(top)
        active = [s for s in active
                  if s + pos < len(corpus) and corpus[s + pos] == top]
    return chain, ln
