"""Per-request multi-length suffix matcher (public API).

Mirrors suffix_gpu/local_matcher.py:49-263.  ``LocalMatchKernel`` keeps the
reference's constructor, ``gather_candidates`` and ``forward``; both run as
one workgroup per request row on gfx950 (csrc/local.hip): the row is
staged in LDS, match_back / candidate lengths / earliest occurrences /
continuations / majority-vote expansion / best-candidate selection all run
from there.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
import torch.nn as nn

from suffixgpu_amd import _lib
from suffixgpu_amd._lib import check, lib, require_gpu, stream_of


class LocalMatchKernel(nn.Module):
    """Matches each row's newest tokens against the row itself at
    several support thresholds and drafts from the best-scored match."""

    def __init__(self, k: int, max_pattern_len: int = 32,
                 min_match_len: int = 1, max_occurrences: int = 32,
                 min_token_prob: float = 0.0,
                 max_spec_factor: float | None = None,
                 max_spec_offset: float = 0.0,
                 support_thresholds: Sequence[int] = (1, 2, 4, 8),
                 vote_smoothing_alpha: float = 0.0):
        super().__init__()
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
        self.register_buffer(
            "_thresholds",
            torch.tensor(self.support_thresholds, dtype=torch.int64),
            persistent=False)
        self.params = _lib.make_params(
            k, max_pattern_len, max_occurrences, self.min_match_len,
            self.support_thresholds, (), max_spec_factor, max_spec_offset,
            min_token_prob, vote_smoothing_alpha)

    def gather_candidates(self, num_tokens_no_spec: torch.Tensor,
                          token_ids: torch.Tensor,
                          combined_mask: torch.Tensor):
        """(cand [B, C] i64, cont [B, C, R, K] int32, occ_count [B, C] i64)."""
        require_gpu(token_ids)
        b = token_ids.shape[0]
        c = len(self.support_thresholds)
        r, k = self.max_occurrences, self.k
        dev = token_ids.device
        bt, keep = _lib.make_batch(token_ids, num_tokens_no_spec,
                                   mask=combined_mask)
        cand = torch.empty(b, c, dtype=torch.int64, device=dev)
        cont = torch.empty(b, c, r, k, dtype=torch.int32, device=dev)
        occ = torch.empty(b, c, dtype=torch.int64, device=dev)
        if b:
            check(lib().sfx_local_gather(self.params, bt, cand.data_ptr(),
                                         cont.data_ptr(), occ.data_ptr(),
                                         stream_of(dev)),
                  "LocalMatchKernel.gather_candidates")
        del keep
        return cand, cont, occ

    def forward(self, num_tokens_no_spec: torch.Tensor,
                token_ids: torch.Tensor, combined_mask: torch.Tensor):
        """(draft [B,K] int32, num_valid [B] int32, match_len [B] i64,
        occ_count [B] i64, score [B] f32)."""
        require_gpu(token_ids)
        b = token_ids.shape[0]
        k = self.k
        dev = token_ids.device
        bt, keep = _lib.make_batch(token_ids, num_tokens_no_spec,
                                   mask=combined_mask)
        draft = torch.empty(b, k, dtype=torch.int32, device=dev)
        nv = torch.empty(b, dtype=torch.int32, device=dev)
        mlen = torch.empty(b, dtype=torch.int64, device=dev)
        occ = torch.empty(b, dtype=torch.int64, device=dev)
        score = torch.empty(b, dtype=torch.float32, device=dev)
        if b:
            check(lib().sfx_local_forward(
                self.params, bt, draft.data_ptr(), nv.data_ptr(),
                mlen.data_ptr(), occ.data_ptr(), score.data_ptr(),
                stream_of(dev)), "LocalMatchKernel.forward")
        del keep
        return draft, nv, mlen, occ, score

