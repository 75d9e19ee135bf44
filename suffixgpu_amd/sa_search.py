"""Suffix-array interval search (public API).

Mirrors suffix_gpu/sa_search.py:66-185.  ``search_interval`` returns the
exact lower/upper bounds; the bounds come from an 8-lane k-ary search per
pattern (csrc/sa_search.h) instead of the reference's fixed-iteration
binary search, which leaves every result unchanged since only the exact
bounds are returned.  ``suffix_match_backoff`` runs the global-match kernel
with an empty delta.
"""

from __future__ import annotations

import torch

from suffixgpu_amd import _lib, kernels
from suffixgpu_amd._lib import check, lib, require_gpu, stream_of


def search_interval(sa: torch.Tensor, corpus: torch.Tensor,
                    pattern: torch.Tensor, pattern_len: torch.Tensor
                    ) -> tuple[torch.Tensor, torch.Tensor]:
    """Per pattern, the ranks [start, end) of the suffixes that begin
    with its first pattern_len tokens (start == end: none)."""
    return kernels.sa_search(sa, corpus, pattern, pattern_len)


def suffix_match_backoff(sa: torch.Tensor, corpus: torch.Tensor,
                         query: torch.Tensor, query_len: torch.Tensor,
                         max_len: int, caps: torch.Tensor):
    """Longest suffix match per capped length (sa_search.py:110-163).

    Returns (match_len [B, C] i64, start [B, C] i64, end [B, C] i64);
    (0, 0) where nothing matched.
    """
    require_gpu(sa, corpus, query, query_len, caps)
    dev = sa.device
    b = query.shape[0]
    cnum = caps.shape[0]
    caps_l = [int(x) for x in caps.tolist()]
    p = _lib.make_params(1, max_len, 1, 1, (1,), caps_l, None, 0.0, 0.0, 0.0)
    delta = torch.zeros(1, dtype=torch.int32, device=dev)
    dlen = torch.zeros((), dtype=torch.int64, device=dev)
    sa32 = sa.to(torch.int32).contiguous()
    corpus32 = corpus.to(torch.int32).contiguous()
    ix = _lib.SfxIndex(corpus32.data_ptr(), sa32.data_ptr(), sa.shape[0],
                       delta.data_ptr(), 1, dlen.data_ptr())
    q = query.to(torch.int32).contiguous()
    ql = query_len.to(torch.int64).contiguous()
    out_len = torch.empty(b, cnum, dtype=torch.int64, device=dev)
    out_s = torch.empty_like(out_len)
    out_e = torch.empty_like(out_len)
    out = _lib.SfxGlobalOut()
    out.sa_len = out_len.data_ptr()
    out.sa_start = out_s.data_ptr()
    out.sa_end = out_e.data_ptr()
    nbytes = lib().sfx_global_query_workspace_size(p, b, 1)
    ws = torch.zeros(max(1, nbytes), dtype=torch.uint8, device=dev)
    if b:
        check(lib().sfx_global_query(p, ix, q.data_ptr(), b, q.shape[1],
                                     ql.data_ptr(), out, ws.data_ptr(),
                                     nbytes, stream_of(dev)),
              "suffix_match_backoff")
    return out_len, out_s, out_e


def longest_suffix_match(sa: torch.Tensor, corpus: torch.Tensor,
                         query: torch.Tensor, query_len: torch.Tensor,
                         max_len: int):
    """Single-cap special case (sa_search.py:166-185)."""
    caps = torch.full((1,), max_len, dtype=torch.int64, device=sa.device)
    best, start, end = suffix_match_backoff(sa, corpus, query, query_len,
                                            max_len, caps)
    return best[:, 0], start[:, 0], end[:, 0]
