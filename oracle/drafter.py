"""SuffixGPUDrafter -- numpy restatement of the public drafter API.

Follows suffix_gpu/proposer.py:33-393: backoff thresholds and global caps
(:71-85), update_state (:135-184), propose_with_update (:186-214), propose
with the local/global merge and hierarchical selection (:216-327), and the
host-side harvest / ingest entry points (:329-390).
"""

from __future__ import annotations

import numpy as np

from oracle.expand import expand_chain
from oracle.global_index import GlobalIndexOracle
from oracle.local import LocalMatcher, gather_tails, select_local_best


def backoff_thresholds(num_backoff: int) -> tuple[int, ...]:
    """proposer.py:73-74: support thresholds 2^0 .. 2^(C-1)."""
    return tuple(2 ** i for i in range(max(1, int(num_backoff))))


def global_caps(max_pattern_len: int, num_backoff: int) -> list[int]:
    """proposer.py:78-83: caps max(2, P>>i) for i < C-1, plus 2, desc."""
    nb = max(1, int(num_backoff))
    if nb == 1:
        caps = [max_pattern_len]
    else:
        caps = [max(2, max_pattern_len >> i) for i in range(nb - 1)] + [2]
    return sorted(set(caps), reverse=True)


class DrafterOracle:
    def __init__(self, k: int, max_pattern_len: int = 32,
                 min_match_len: int = 1, max_occurrences: int = 128,
                 enable_global: bool = False, global_capacity: int = 1 << 22,
                 delta_capacity: int = 1 << 16,
                 rebuild_threshold: int | None = None,
                 max_spec_factor: float | None = None,
                 max_spec_offset: float = 0.0, min_token_prob: float = 0.0,
                 num_backoff: int = 8, vote_smoothing_alpha: float = 0.0,
                 async_rebuild: bool = False,
                 finish_at_user_poll: bool = False):
        self.k = k
        self.max_pattern_len = max_pattern_len
        self.min_token_prob = min_token_prob
        self.vote_smoothing_alpha = float(vote_smoothing_alpha)
        self.num_backoff = max(1, int(num_backoff))
        self._global_caps = np.array(
            global_caps(max_pattern_len, self.num_backoff), dtype=np.int64)
        self.local_kernel = LocalMatcher(
            k=k, max_pattern_len=max_pattern_len,
            min_match_len=min_match_len, max_occurrences=max_occurrences,
            min_token_prob=min_token_prob, max_spec_factor=max_spec_factor,
            max_spec_offset=max_spec_offset,
            support_thresholds=backoff_thresholds(self.num_backoff),
            vote_smoothing_alpha=self.vote_smoothing_alpha)
        self.global_index = None
        self._ingested: dict = {}
        if enable_global:
            self.global_index = GlobalIndexOracle(
                capacity=global_capacity, delta_capacity=delta_capacity, k=k,
                max_occurrences=max_occurrences,
                rebuild_threshold=rebuild_threshold,
                async_rebuild=async_rebuild,
                finish_at_user_poll=finish_at_user_poll)

    def poll(self) -> None:
        if self.global_index is not None:
            self.global_index.poll_rebuild()

    def update_state(self, num_tokens, tok, sampled, valid_cnt=None):
        """proposer.py:162-184 (tok updated in place)."""
        b, s = tok.shape
        t = sampled.shape[1]
        base = num_tokens.astype(np.int64)
        if valid_cnt is None:
            valid_cnt = (sampled != -1).sum(axis=1)
        cnt = np.asarray(valid_cnt).astype(np.int64)
        for j in range(t):
            ok = (j < cnt) & (sampled[:, j] != -1) & (base + j < s)
            rows = np.flatnonzero(ok)
            tok[rows, base[rows] + j] = sampled[rows, j]
        return (base + cnt).astype(np.int32)

    def propose_with_update(self, num_tokens, tok, sampled, valid_cnt=None,
                            max_model_len=None):
        """proposer.py:186-214."""
        if valid_cnt is None:
            valid_cnt = (sampled != -1).sum(axis=1)
        new = self.update_state(num_tokens, tok, sampled, valid_cnt)
        mask = np.asarray(valid_cnt).astype(np.int64) > 0
        s = tok.shape[1]
        limit = s if max_model_len is None else min(max_model_len, s)
        mask &= new.astype(np.int64) < limit
        draft, nv = self.propose(new, tok, mask)
        return draft, nv, new

    def propose(self, num_tokens, tok, mask=None):
        """proposer.py:216-327."""
        b = num_tokens.shape[0]
        k = self.k
        if mask is None:
            mask = np.ones(b, dtype=bool)
        mask = mask.astype(bool)
        lk = self.local_kernel
        if self.global_index is None:
            draft, nv, _, _, _ = lk.forward(num_tokens, tok, mask)
        else:
            r = lk.max_occurrences
            tails, tail_len = gather_tails(num_tokens, tok,
                                           self.max_pattern_len)
            g_len, g_cont, g_occ = self.global_index._query_backoff(
                tails.astype(np.int32), tail_len, self.max_pattern_len,
                self._global_caps)
            cand_l, cont_l, occ_l = lk.gather_candidates(num_tokens, tok, mask)
            cl = cand_l.shape[1]
            cg = g_len.shape[1]
            len_all = np.concatenate([cand_l, g_len], axis=1)
            cont_all = np.concatenate([cont_l, g_cont], axis=1)
            occ_all = np.concatenate([occ_l, g_occ], axis=1)
            cap_all = lk.spec_cap(len_all.reshape(-1))
            chain, _, emit, score = expand_chain(
                cont_all.reshape(b * (cl + cg), r, k), occ_all.reshape(-1),
                k, min_token_prob=self.min_token_prob, cap=cap_all,
                alpha=self.vote_smoothing_alpha)
            chain = chain.reshape(b, cl + cg, k)
            emit = emit.reshape(b, cl + cg)
            score = score.reshape(b, cl + cg)
            l_chain, l_emit, _, _, l_score = select_local_best(
                cand_l, chain[:, :cl], emit[:, :cl], occ_all[:, :cl],
                score[:, :cl])
            gs = score[:, cl:]
            best_g = gs.argmax(axis=1)
            i = np.arange(b)
            g_chain = chain[:, cl:][i, best_g]
            g_emit = emit[:, cl:][i, best_g]
            g_score = gs[i, best_g]
            pick = (g_score > l_score) & mask
            draft = np.where(pick[:, None], g_chain, l_chain)
            nv = np.where(pick, g_emit, l_emit.astype(np.int64))
        nv = np.where(mask, nv.astype(np.int64), 0)
        slot = np.arange(k)[None, :]
        draft = np.where(slot < nv[:, None], draft, -1)
        return draft.astype(np.int32), nv.astype(np.int32)

    def harvest_finished(self, row_indices, lengths, tok) -> None:
        """proposer.py:329-343."""
        self.harvest_rows([tok[r] for r in row_indices], lengths)

    def harvest_rows(self, rows, lengths) -> None:
        """proposer.py:345-352."""
        if self.global_index is None or not rows:
            return
        docs = [row[:ln] for row, ln in zip(rows, lengths) if ln > 0]
        if docs:
            self.global_index.append_documents(docs)

    def ingest_active(self, keys, rows, lengths, final=False, chunk=64):
        """proposer.py:354-390."""
        if self.global_index is None:
            return
        overlap = self.max_pattern_len + self.k
        docs = []
        for key, row, ln in zip(keys, rows, lengths):
            done = self._ingested.get(key, 0)
            if ln - done >= chunk or (final and ln > done):
                start = max(0, done - overlap)
                docs.append(row[start:ln])
                self._ingested[key] = ln
            if final:
                self._ingested.pop(key, None)
        if docs:
            self.global_index.append_documents(docs)
