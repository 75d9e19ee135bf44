"""Operator-level entry points (the reference's kernel boundary).

Mirrors suffix_gpu/triton_kernels.py:33-402 -- ``available``,
``match_back``, ``sa_search``, ``expand_chain``, ``first_occurrences`` and
``scatter_append`` -- on the hand-written gfx950 kernels of
libsuffixgpu_amd.so.  Unlike the reference there is no torch fallback:
``available`` only reports whether the HIP path can run, and every call
raises when it cannot.
"""

from __future__ import annotations

import torch

from suffixgpu_amd import _lib
from suffixgpu_amd._lib import check, lib, ptr, require_gpu, stream_of


def available(*tensors: torch.Tensor) -> bool:
    """True when the library loads and every tensor is on a ROCm GPU."""
    if not all(t.device.type == "cuda" for t in tensors):
        return False
    try:
        lib()
    except Exception:
        return False
    return True


def match_back(src: torch.Tensor, pat: torch.Tensor,
               n_out: int) -> torch.Tensor:
    """[B, n_out] int32: longest L with src[.., i-L:i] == newest-first pat.

    ``src`` is [B, S] (row per pattern) or [N] (shared, e.g. the delta).
    """
    require_gpu(src, pat)
    b, p = pat.shape
    src = src.to(torch.int32).contiguous()
    pat = pat.to(torch.int32).contiguous()
    if src.dim() == 2 and src.shape[0] != b:
        raise ValueError("match_back: src rows != pattern rows")
    out = torch.empty(b, n_out, dtype=torch.int32, device=src.device)
    stride = src.stride(0) if src.dim() == 2 else 0
    if src.dim() == 2 and src.shape[1] < n_out:
        raise ValueError("match_back: n_out exceeds the row length")
    if src.dim() == 1 and src.shape[0] + 1 < n_out:
        raise ValueError("match_back: n_out exceeds the buffer length + 1")
    check(lib().sfx_match_back(src.data_ptr(), stride, pat.data_ptr(), b, p,
                               n_out, out.data_ptr(),
                               stream_of(src.device)), "match_back")
    return out


def first_occurrences(mb: torch.Tensor, thr: torch.Tensor, c: int,
                      r: int) -> tuple[torch.Tensor, torch.Tensor]:
    """First r ascending columns with mb >= thr per (row, candidate).

    Returns (positions [B*C, r] i64 zero padded, count [B*C] i64).
    """
    require_gpu(mb, thr)
    mb = mb.to(torch.int32).contiguous()
    thr = thr.to(torch.int64).contiguous()
    bc = thr.shape[0]
    if bc != mb.shape[0] * c:
        raise ValueError("first_occurrences: thr must hold B*C entries")
    pos = torch.empty(bc, r, dtype=torch.int64, device=mb.device)
    cnt = torch.empty(bc, dtype=torch.int64, device=mb.device)
    check(lib().sfx_first_occurrences(mb.data_ptr(), mb.shape[1],
                                      thr.data_ptr(), bc, c, r,
                                      pos.data_ptr(), cnt.data_ptr(),
                                      stream_of(mb.device)),
          "first_occurrences")
    return pos, cnt


def sa_search(sa: torch.Tensor, corpus: torch.Tensor, pattern: torch.Tensor,
              pattern_len: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Exact [lower, upper) SA bounds of each row of ``pattern``."""
    require_gpu(sa, corpus, pattern, pattern_len)
    n = sa.shape[0]
    if corpus.shape[0] != n:
        raise ValueError("sa_search: corpus and sa lengths differ")
    sa = sa.to(torch.int32).contiguous()
    corpus = corpus.to(torch.int32).contiguous()
    b, m = pattern.shape
    pattern = pattern.to(torch.int32).contiguous()
    plen = pattern_len.to(torch.int64).contiguous()
    lo = torch.empty(b, dtype=torch.int64, device=sa.device)
    hi = torch.empty(b, dtype=torch.int64, device=sa.device)
    if n == 0:
        return lo.zero_(), hi.zero_()
    check(lib().sfx_sa_search(sa.data_ptr(), corpus.data_ptr(), n,
                              pattern.data_ptr(), b, m, plen.data_ptr(),
                              lo.data_ptr(), hi.data_ptr(),
                              stream_of(sa.device)), "sa_search")
    return lo, hi


def expand_chain(cont: torch.Tensor, num_occ: torch.Tensor, k: int,
                 min_token_prob: float, cap: torch.Tensor,
                 weights: torch.Tensor | None = None,
                 alpha: float = 0.0):
    """(chain [B,k] int32, num_valid i64, num_emit i64, score f32)."""
    require_gpu(cont, num_occ, cap, weights)
    b, r, kk = cont.shape
    if kk != k:
        raise ValueError("expand_chain: cont depth must equal k")
    cont = cont.to(torch.int32).contiguous()
    nocc = num_occ.to(torch.int64).contiguous()
    capc = cap.to(torch.int64).contiguous()
    w = None
    if weights is not None:
        w = weights.to(torch.float32).contiguous()
        if tuple(w.shape) != (b, r):
            raise ValueError("expand_chain: weights must be [B, R]")
    dev = cont.device
    chain = torch.empty(b, k, dtype=torch.int32, device=dev)
    nv = torch.empty(b, dtype=torch.int64, device=dev)
    ne = torch.empty(b, dtype=torch.int64, device=dev)
    score = torch.empty(b, dtype=torch.float32, device=dev)
    if b == 0:
        return chain, nv, ne, score
    check(lib().sfx_expand_chain(cont.data_ptr(), b, r, k, nocc.data_ptr(),
                                 capc.data_ptr(), ptr(w),
                                 float(min_token_prob), float(alpha),
                                 chain.data_ptr(), nv.data_ptr(),
                                 ne.data_ptr(), score.data_ptr(),
                                 stream_of(dev)), "expand_chain")
    return chain, nv, ne, score


def scatter_append(token_ids_gpu: torch.Tensor, base: torch.Tensor,
                   cnt: torch.Tensor, sampled: torch.Tensor) -> None:
    """Writes row b's first cnt[b] sampled ids (skipping -1) at
    positions base[b], base[b] + 1, ... of its token row, below S."""
    bt, keep = _lib.make_batch(token_ids_gpu, base, sampled=sampled,
                               valid_count=cnt)
    check(lib().sfx_scatter_append(bt, None,
                                   stream_of(token_ids_gpu.device)),
          "scatter_append")
    del keep
