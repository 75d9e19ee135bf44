"""Cross-request global index -- numpy restatement of GlobalIndex.

Follows suffix_gpu/global_index.py:34-553: the PAD-filled corpus ring with
its suffix array, the append-only delta with SEP separators, the rebuild
state machine (evict whole oldest docs, whole-doc delta snapshot, compact the
delta at launch, build over the real prefix plus one sentinel column, swap in
place), and the capped-length SA + delta query path.
"""

from __future__ import annotations

from collections import deque

import numpy as np

from oracle.expand import expand_chain
from oracle.local import newest_first_pattern, match_back, first_occurrences
from oracle.local import spec_cap
from oracle.sa import build_suffix_array, suffix_match_backoff

PAD_TOKEN = np.iinfo(np.int32).max   # global_index.py:34
SEP_TOKEN = -2                       # global_index.py:38


class _DoneAtPoll:
    """Stands in for a rebuild event: complete at the next poll."""

    def query(self) -> bool:
        return True


class GlobalIndexOracle:
    """global_index.py:41-553 on host arrays.

    With ``async_rebuild=False`` (the reference's CPU behaviour,
    global_index.py:213-215) a rebuild builds and swaps immediately.  With
    ``async_rebuild=True`` it behaves like a rebuild on a side stream that has
    finished by the next ``poll_rebuild`` -- the deterministic schedule the
    GPU implementation uses in its blocking-poll mode.  Adding
    ``finish_at_user_poll=True``, a rebuild is still running when
    append_documents polls (global_index.py:111,140 find its event not yet
    complete) and finishes at the caller's next poll_rebuild: the schedule
    of the GPU's device-side ingest, whose builds start at that poll.
    """

    def __init__(self, capacity: int, delta_capacity: int, k: int,
                 max_occurrences: int = 32,
                 rebuild_threshold: int | None = None,
                 async_rebuild: bool = False,
                 finish_at_user_poll: bool = False):
        self.capacity = capacity
        self.delta_capacity = delta_capacity
        self.k = k
        self.max_occurrences = max_occurrences
        self.rebuild_threshold = rebuild_threshold or max(
            1, delta_capacity // 2)
        self.async_rebuild = async_rebuild
        self.finish_at_user_poll = finish_at_user_poll
        self.corpus = np.full(capacity, PAD_TOKEN, dtype=np.int32)
        self.staging_corpus = self.corpus.copy()
        self.sa = np.arange(capacity, dtype=np.int32)
        self.staging_sa = self.sa.copy()
        self.delta = np.zeros(delta_capacity, dtype=np.int32)
        self.active_len = 0
        self.delta_len = 0
        self.active_doc_lens: deque[int] = deque()
        self.delta_doc_lens: list[int] = []
        self._rebuild_event = None
        self._pending = None
        # what an async rebuild's event is: by default complete at the next
        # poll_rebuild; tests replace it with one that completes at the
        # poll where another index (the GPU's) swapped
        self.rebuild_event_factory = _DoneAtPoll

    # ---------------------------------------------------------------- writes
    def append_documents(self, docs) -> None:
        """global_index.py:86-108."""
        for doc in docs:
            doc = np.asarray(doc).astype(np.int32).reshape(-1)
            n = doc.shape[0]
            if n == 0:
                continue
            if n + 1 > self.delta_capacity:
                doc = doc[-(self.delta_capacity - 1):]
                n = doc.shape[0]
            if self.delta_len + n + 1 > self.delta_capacity:
                self._make_room(n + 1)
            self.delta[self.delta_len:self.delta_len + n] = doc
            self.delta[self.delta_len + n] = SEP_TOKEN
            self.delta_len += n + 1
            self.delta_doc_lens.append(n + 1)
        self.maybe_rebuild()

    def _poll_internal(self) -> None:
        """The polls inside append_documents (global_index.py:111,140)."""
        if not self.finish_at_user_poll:
            self.poll_rebuild()

    def _make_room(self, needed: int) -> None:
        """global_index.py:110-118."""
        self._poll_internal()
        if self._rebuild_event is None:
            self._launch_rebuild()
        if self.delta_len + needed <= self.delta_capacity:
            return
        self._drop_oldest_docs(self.delta_len + needed - self.delta_capacity)

    def _drop_oldest_docs(self, drop: int) -> None:
        """global_index.py:120-133."""
        acc = 0
        dropped = 0
        for ln in self.delta_doc_lens:
            if acc >= drop:
                break
            acc += ln
            dropped += 1
        remaining = self.delta_len - acc
        if remaining > 0:
            self.delta[:remaining] = self.delta[acc:self.delta_len].copy()
        self.delta_len = remaining
        self.delta_doc_lens = self.delta_doc_lens[dropped:]

    def maybe_rebuild(self) -> None:
        """global_index.py:138-145."""
        self._poll_internal()
        if self._rebuild_event is not None or self.delta_len == 0:
            return
        if self.delta_len < self.rebuild_threshold:
            return
        self._launch_rebuild()

    def plan_rebuild(self):
        """Eviction / snapshot arithmetic of global_index.py:150-169.

        Returns (keep_start, n_active_keep, snap, n_new).
        """
        keep_start = 0
        for ln in self.active_doc_lens:
            if self.active_len - keep_start + self.delta_len <= self.capacity:
                break
            keep_start += ln
        n_keep = self.active_len - keep_start
        snap = min(self.delta_len, self.capacity - n_keep)
        acc = 0
        for ln in self.delta_doc_lens:
            if acc + ln <= snap:
                acc += ln
            else:
                break
        snap = acc
        return keep_start, n_keep, snap, n_keep + snap

    def _launch_rebuild(self) -> None:
        """global_index.py:147-215."""
        if self._rebuild_event is not None:
            return
        keep_start, n_keep, snap, n_new = self.plan_rebuild()
        if n_new == 0:
            return
        dst = self.staging_corpus
        dst[:] = PAD_TOKEN
        if n_keep > 0:
            dst[:n_keep] = self.corpus[keep_start:self.active_len]
        if snap > 0:
            dst[n_keep:n_new] = self.delta[:snap]
        new_lens: deque[int] = deque()
        acc = 0
        for ln in self.active_doc_lens:
            acc += ln
            if acc > keep_start:
                new_lens.append(ln)
        acc = 0
        for ln in self.delta_doc_lens:
            acc += ln
            if acc <= snap:
                new_lens.append(ln)
        absorbed = self._count_docs_within(snap)
        remaining = self.delta_len - snap
        if remaining > 0:
            self.delta[:remaining] = self.delta[snap:self.delta_len].copy()
        self.delta_len = remaining
        self.delta_doc_lens = self.delta_doc_lens[absorbed:]
        m = min(n_new + 1, self.capacity)
        self._build_staging_sa(dst, m)
        if self.async_rebuild:
            self._pending = (n_new, new_lens)
            self._rebuild_event = self.rebuild_event_factory()
        else:
            self._finish_swap(n_new, new_lens)

    def _build_staging_sa(self, dst: np.ndarray, m: int) -> None:
        """global_index.py:217-223."""
        self.staging_sa[:m] = build_suffix_array(dst[:m]).astype(np.int32)
        if m < self.capacity:
            self.staging_sa[m:] = np.arange(m, self.capacity, dtype=np.int32)

    def _count_docs_within(self, tokens: int) -> int:
        """global_index.py:225-233."""
        acc = 0
        count = 0
        for ln in self.delta_doc_lens:
            acc += ln
            if acc > tokens:
                break
            count += 1
        return count

    def _finish_swap(self, n_new: int, new_lens) -> None:
        """global_index.py:235-244."""
        self.corpus[:] = self.staging_corpus
        self.sa[:] = self.staging_sa
        self.active_len = n_new
        self.active_doc_lens = new_lens
        self._rebuild_event = None
        self._pending = None

    def poll_rebuild(self) -> None:
        """global_index.py:246-252."""
        if self._rebuild_event is None:
            return
        if self._rebuild_event.query():
            n_new, new_lens = self._pending
            self._finish_swap(n_new, new_lens)

    def load_documents(self, docs) -> None:
        """State after one rebuild whose active set is exactly ``docs``.

        Equivalent to _launch_rebuild with an empty active corpus and the
        docs (each + SEP) as the snapshot: corpus = packed docs then PAD,
        SA over the first min(n+1, N) positions, identity beyond.
        """
        lens = [int(len(d)) + 1 for d in docs]
        n = sum(lens)
        assert n <= self.capacity
        dst = self.staging_corpus
        dst[:] = PAD_TOKEN
        off = 0
        for d in docs:
            dst[off:off + len(d)] = d
            dst[off + len(d)] = SEP_TOKEN
            off += len(d) + 1
        self._build_staging_sa(dst, min(n + 1, self.capacity))
        self._finish_swap(n, deque(lens))

    # --------------------------------------------------------------- queries
    def query(self, query, query_len, max_len):
        """global_index.py:257-284."""
        caps = np.array([max_len], dtype=np.int64)
        ml, cont, occ = self._query_backoff(query, query_len, max_len, caps)
        return ml[:, 0], cont[:, 0], occ[:, 0]

    def _query_backoff(self, query, query_len, max_len, caps):
        """global_index.py:286-370."""
        b = query.shape[0]
        cnum = caps.shape[0]
        r = self.max_occurrences
        sa_len, sa_start, sa_end = suffix_match_backoff(
            self.sa, self.corpus, query, query_len, max_len, caps)
        d_len, d_pos, d_cnt = self._delta_match_backoff(
            query, query_len, max_len, caps)
        use_sa = (sa_len >= d_len) & (sa_len > 0)
        use_delta = (d_len > sa_len) & (d_len > 0)
        match_len = np.where(use_sa, sa_len, np.where(use_delta, d_len, 0))
        if cnum > 1:
            src = use_sa.astype(np.int8) + 2 * use_delta.astype(np.int8)
            dup = np.zeros_like(use_sa)
            dup[:, 1:] = ((match_len[:, 1:] == match_len[:, :-1])
                          & (src[:, 1:] == src[:, :-1])
                          & (match_len[:, 1:] > 0))
            use_sa = use_sa & ~dup
            use_delta = use_delta & ~dup
            match_len = np.where(dup, 0, match_len)
        offs = np.arange(r, dtype=np.int64)
        ilen = sa_end - sa_start
        strided = sa_start[:, :, None] + (offs[None, None, :]
                                          * ilen[:, :, None]) // r
        seq = sa_start[:, :, None] + offs[None, None, :]
        sa_idx = np.clip(np.where((ilen > r)[:, :, None], strided, seq), 0,
                         self.capacity - 1)
        sa_cnt = np.minimum(ilen, r)
        take = offs[None, None, :] < sa_cnt[:, :, None]
        pos = self.sa[sa_idx.reshape(-1)].reshape(b, cnum, r).astype(np.int64)
        sa_occ = np.where(take, pos, 0)
        flat_len = match_len.reshape(-1)
        sa_cont = self._gather_cont(self.corpus, self.capacity,
                                    sa_occ.reshape(b * cnum, r),
                                    sa_cnt.reshape(-1), flat_len,
                                    use_sa.reshape(-1))
        d_cont = self._gather_cont(self.delta, self.delta_len,
                                   d_pos.reshape(b * cnum, r),
                                   d_cnt.reshape(-1), flat_len,
                                   use_delta.reshape(-1))
        cont = np.full((b * cnum, r, self.k), -1, dtype=np.int32)
        cont = np.where(use_sa.reshape(-1, 1, 1), sa_cont, cont)
        cont = np.where(use_delta.reshape(-1, 1, 1), d_cont, cont)
        occ_count = np.where(use_sa, sa_cnt, np.where(use_delta, d_cnt, 0))
        return match_len, cont.reshape(b, cnum, r, self.k), occ_count

    def _gather_cont(self, src, src_len, occ_pos, occ_cnt, match_len, sel):
        """global_index.py:443-463."""
        b, r = occ_pos.shape
        n = src.shape[0]
        row = np.arange(r)[None, :]
        row_active = (row < occ_cnt[:, None]) & sel[:, None]
        idx = (occ_pos[:, :, None] + match_len[:, None, None]
               + np.arange(self.k)[None, None, :])
        valid = row_active[:, :, None] & (idx < src_len) & (idx >= 0)
        vals = src[np.clip(idx, 0, n - 1)]
        ok = valid & (vals != PAD_TOKEN) & (vals >= 0)
        return np.where(ok, vals, -1).astype(np.int32)

    def _delta_match_backoff(self, query, query_len, max_len, caps):
        """global_index.py:465-546: (len [B,C], starts [B,C,R], cnt [B,C])."""
        n_i = self.delta_capacity + 1
        pat = newest_first_pattern(query, query_len, max_len, -3)
        mb = match_back(self.delta, pat, n_i)
        valid = np.arange(n_i)[None, :] <= self.delta_len
        mb = np.where(valid, mb, 0)
        lo_full = mb.max(axis=1).astype(np.int64)
        lo = np.minimum(lo_full[:, None], np.asarray(caps)[None, :])
        occ_end, cnt = first_occurrences(mb, lo, self.max_occurrences)
        occ = np.maximum(occ_end - lo[:, :, None], 0)
        return lo, occ, cnt

    def draft(self, query, query_len, max_len, k, min_token_prob=0.0,
              max_spec_factor=None, max_spec_offset=0.0, caps=None,
              alpha=0.0):
        """global_index.py:372-441."""
        b = query.shape[0]
        if caps is None:
            caps = np.array(sorted({max_len, max(2, max_len // 2),
                                    max(2, max_len // 4), 2}, reverse=True),
                            dtype=np.int64)
        cnum = caps.shape[0]
        ml, cont, occ = self._query_backoff(query, query_len, max_len, caps)
        flat = ml.reshape(-1)
        cap_emit = spec_cap(flat, k, max_spec_factor, max_spec_offset)
        chain, _, emit, score = expand_chain(
            cont.reshape(b * cnum, self.max_occurrences, k), occ.reshape(-1),
            k, min_token_prob=min_token_prob, cap=cap_emit, alpha=alpha)
        score = score.reshape(b, cnum)
        best = score.argmax(axis=1)
        i = np.arange(b)
        ch = chain.reshape(b, cnum, k)[i, best]
        em = emit.reshape(b, cnum)[i, best]
        ch = np.where(np.arange(k)[None, :] < em[:, None], ch, -1)
        return ch, em, ml[i, best], occ[i, best], score[i, best]

    def expand(self, cont, occ_count, min_token_prob=0.0):
        """global_index.py:548-553."""
        chain, nv, _, _ = expand_chain(cont, occ_count, self.k,
                                       min_token_prob=min_token_prob)
        return chain, nv
