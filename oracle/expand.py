"""Depth-wise majority-vote chain expansion (numpy restatement).

Follows suffix_gpu/expand.py:16-147 (the torch fallback) and the GPU kernel
semantics of suffix_gpu/triton_kernels.py:139-215 (identical for unweighted
votes): per depth the active occurrences vote, the winner is the most voted
token with ties to the smallest id, the chain probability is multiplied by
``votes / (max(active, 1) + alpha)`` in fp32 (IEEE divide, then multiply),
a depth is valid while votes > 0 and the probability is >= fl32(min_prob),
and the score sums the probability over valid depths below the cap.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def majority_token(values: np.ndarray, active: np.ndarray, sentinel: int,
                   weights: np.ndarray | None = None
                   ) -> tuple[np.ndarray, np.ndarray]:
    """Per-row majority token among active entries (expand.py:16-56).

    Returns (token [B] in values' dtype, count [B]); rows without an active
    entry get (sentinel, 0).  Count is int64 for unit votes, fp32 weight mass
    otherwise.
    """
    eq = values[:, :, None] == values[:, None, :]
    if weights is None:
        votes = (eq & active[:, None, :]).sum(axis=2)
        votes = np.where(active, votes, 0)
    else:
        w = np.where(active, weights.astype(F32), F32(0))
        votes = (eq.astype(F32) * w[:, None, :]).sum(axis=2, dtype=F32)
        votes = np.where(active, votes, F32(0))
    mx = votes.max(axis=1)
    win = active & (votes == mx[:, None]) & (mx[:, None] > 0)
    big = np.iinfo(np.int64).max
    tok = np.where(win, values.astype(np.int64), big).min(axis=1)
    any_act = active.any(axis=1)
    token = np.where(any_act, tok, sentinel).astype(values.dtype)
    count = np.where(any_act, mx, np.zeros_like(mx))
    return token, count


def expand_chain(cont: np.ndarray, num_occ: np.ndarray, k: int,
                 sentinel: int = -1, min_token_prob: float = 0.0,
                 cap: np.ndarray | None = None,
                 weights: np.ndarray | None = None, alpha: float = 0.0
                 ) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """expand.py:59-147.  Returns (chain [B,k], num_valid, num_emit, score).

    ``cont`` is [B, R, k]; rows r >= num_occ are ignored.  ``cap`` defaults
    to k.  fp32 arithmetic is done with numpy float32 scalars and arrays, so
    every operation rounds to fp32 exactly as torch's CPU kernels do.
    """
    b, r, _ = cont.shape
    if cap is None:
        cap = np.full(b, k, dtype=np.int64)
    cap = cap.astype(np.int64)
    offs = np.arange(r)
    prefix_ok = offs[None, :] < num_occ.astype(np.int64)[:, None]
    chain = np.full((b, k), sentinel, dtype=cont.dtype)
    cum = np.ones(b, dtype=F32)
    score = np.zeros(b, dtype=F32)
    minp = F32(min_token_prob)
    alpha32 = F32(alpha)
    for d in range(k):
        col = cont[:, :, d]
        act = prefix_ok & (col != sentinel)
        tok, cnt = majority_token(col, act, sentinel, weights)
        if weights is None:
            denom = np.maximum(act.sum(axis=1), 1).astype(F32)
        else:
            denom = np.where(act, weights.astype(F32), F32(0)).sum(
                axis=1, dtype=F32)
        with np.errstate(invalid="ignore", divide="ignore"):
            cum = (cum * (cnt.astype(F32) / (denom + alpha32))).astype(F32)
        valid = (tok != sentinel) & (cnt > 0) & (cum >= minp)
        chain[:, d] = np.where(valid, tok, chain[:, d])
        score = (score + np.where(valid & (cap > d), cum, F32(0))).astype(F32)
        prefix_ok = prefix_ok & (col == tok[:, None]) & valid[:, None]
    filled = (chain != sentinel).astype(np.int64)
    num_valid = np.cumprod(filled, axis=1).sum(axis=1)
    num_emit = np.minimum(num_valid, np.maximum(cap, 0))
    return chain, num_valid, num_emit, score


def expand_chain_pairwise(cont, num_occ, k, min_token_prob, cap):
    """Pairwise-vote formulation (triton_kernels.py:96-133), row by row.

    Kept as an independent restatement: for unit votes it must equal
    ``expand_chain`` bit for bit (the reference's v2 == pairwise property,
    tests/test_expand_v2.py:28-43).
    """
    b, r, _ = cont.shape
    chain = np.full((b, k), -1, dtype=np.int32)
    nv = np.zeros(b, dtype=np.int64)
    emit = np.zeros(b, dtype=np.int64)
    score = np.zeros(b, dtype=F32)
    minp = F32(min_token_prob)
    for row in range(b):
        ok = np.arange(r) < int(num_occ[row])
        prob = F32(1.0)
        sc = F32(0.0)
        n = 0
        for d in range(k):
            c = cont[row, :, d]
            act = ok & (c != -1)
            votes = np.array([int(np.sum(act & (c == c[i]))) if act[i] else 0
                              for i in range(r)])
            mx = int(votes.max()) if r else 0
            if mx > 0:
                tok = int(c[(votes == mx) & act].min())
            else:
                tok = 2147483647
            nact = max(int(act.sum()), 1)
            prob = F32(prob * (F32(mx) / F32(nact)))
            valid = mx > 0 and prob >= minp
            chain[row, d] = tok if valid else -1
            if valid and d < int(cap[row]):
                sc = F32(sc + prob)
            n += int(valid)
            ok = ok & (c == tok) & valid
        nv[row] = n
        emit[row] = min(n, max(int(cap[row]), 0))
        score[row] = sc
    return chain, nv, emit, score
