"""The drafter's memory of earlier responses, held on the GPU.

Follows suffix_gpu/global_index.py:34-553.  Finished responses live in two
places: a ring of ``capacity`` int32 tokens (whole documents, PAD after
the last one) indexed by a suffix array that only a rebuild changes, and a
small append-only ``delta`` of the most recent documents (each closed by
SEP) that queries scan directly.  A rebuild assembles the next ring in
staging buffers -- the oldest whole documents dropped until the kept ones
plus the delta's whole documents fit -- removes the absorbed documents
from the delta at once, sorts the staging suffixes on the rebuild stream
(csrc/sa_build.hip, no host synchronisation) and writes the staging key
rows.  ``poll_rebuild`` then copies ring and suffix array into the live
tensors in place, so captured graphs keep their pointers, and flips a
device selector word to the freshly written key rows (no key-row copy).

Host bookkeeping (document lengths, eviction and snapshot arithmetic) is
plain Python exactly as in the reference; every device operation is a
stream-ordered copy/fill or a libsuffixgpu_amd kernel.  Appends are
batched: the documents between two room-making steps go to the delta in
one launch (copies, separators and the device length), and delta
compactions are one in-place launch.  Queries run the fused SA-search +
delta-scan + merge kernel (csrc/global.hip).
"""

from __future__ import annotations

from collections import deque
from ctypes import c_int64 as ctypes_i64

import torch

from suffixgpu_amd import _lib
from suffixgpu_amd._lib import check, lib, require_gpu, stream_of
from suffixgpu_amd.expand import expand_chain
from suffixgpu_amd.suffix_array import (DEFAULT_RADIX_MASK, STATE_WORDS,
                                        BuildState, enqueue_rounds,
                                        sa_workspace_bytes, state_view)

PAD_TOKEN = torch.iinfo(torch.int32).max
# Tokens of every suffix kept next to the suffix array (one 128-byte row
# per rank) so an interval-search probe is a single row load.
KEY_WIDTH = 32
# Slots of the n-gram range table per corpus position (in buckets of 16,
# 24 bytes a slot): a corpus of real text holds about 1.6 distinct runs of
# 1-4 tokens per position, so the buckets stay about half full and rarely
# overflow into the next one.
GRAM_SLOTS_PER_TOKEN = 3


def gram_slots_for(capacity: int) -> int:
    n = max(1024, GRAM_SLOTS_PER_TOKEN * capacity)
    return (n + 15) // 16 * 16
# Delta token index buckets: about four delta positions per bucket, a
# power of two from 2^10 to 2^17; deltas above 2^30 positions are scanned.
DELTA_INDEX_MAX = 1 << 30


def delta_buckets_for(delta_capacity: int) -> int:
    b = 1 << max(0, (max(1, delta_capacity // 4) - 1).bit_length())
    return min(max(b, 1 << 10), 1 << 17)


# Written between documents; negative, so no query token (>= 0) can match
# it and neither matches nor continuations cross document boundaries.
SEP_TOKEN = -2


class GlobalIndex:
    """Suffix-array memory of finished responses on one GPU: a sorted
    ring rebuilt in the background plus a directly scanned delta."""

    def __init__(self, capacity: int, delta_capacity: int, k: int,
                 max_occurrences: int = 32,
                 rebuild_threshold: int | None = None,
                 device: torch.device | str = "cuda",
                 rebuild_stream: torch.cuda.Stream | None = None,
                 gram_slots: int | None = None,
                 search_tables: bool = True,
                 delta_index: bool = True):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise _lib.SuffixGPUError(
                "GlobalIndex needs a ROCm GPU device; there is no CPU path")
        if not 1 <= capacity <= 2 ** 31 - 1:
            raise ValueError("capacity must be in [1, 2^31)")
        if not 1 <= delta_capacity <= 2 ** 31 - 1:
            raise ValueError("delta_capacity must be in [1, 2^31)")
        self.capacity = capacity
        self.delta_capacity = delta_capacity
        self.k = k
        self.max_occurrences = max_occurrences
        self.rebuild_threshold = rebuild_threshold or max(
            1, delta_capacity // 2)
        self.rebuild_stream = rebuild_stream
        # True: poll_rebuild waits for an in-flight build (deterministic
        # swap points); False (default, as the reference): event.query().
        self.blocking_poll = False

        dev = self.device
        self.corpus = torch.full((capacity,), PAD_TOKEN, dtype=torch.int32,
                                 device=dev)
        self.staging_corpus = self.corpus.clone()
        self.sa = torch.arange(capacity, dtype=torch.int32, device=dev)
        self.staging_sa = self.sa.clone()
        self.delta = torch.zeros(delta_capacity, dtype=torch.int32,
                                 device=dev)
        self.delta_len_t = torch.zeros((), dtype=torch.int64, device=dev)
        # Delta token index (sfx_delta_index_build): the delta positions by
        # token bucket, rebuilt after every write to the delta, so that a
        # decode row visits only the positions of its newest token's
        # bucket.  delta_index=False: every row scans the whole delta.
        self.delta_buckets = 0
        self._dix_ent = self._dix_start = self._dix_ws = None
        if delta_index and delta_capacity <= DELTA_INDEX_MAX:
            self.delta_buckets = delta_buckets_for(delta_capacity)
            # {q, x(q), x(q - 1), x(q - 2)} per entry
            self._dix_ent = torch.empty((delta_capacity, 4),
                                        dtype=torch.int32, device=dev)
            self._dix_start = torch.zeros(self.delta_buckets + 1,
                                          dtype=torch.int32, device=dev)
            self._dix_ws = torch.empty(
                int(lib().sfx_delta_index_bytes(delta_capacity)),
                dtype=torch.uint8, device=dev)
            self._index_delta()
        # One key-row buffer and one n-gram range table, of the live
        # suffix array.  A swap brings in a new array with the device word
        # key_select set (the steps then search through the suffix array
        # and the corpus, exact but slower: the selector names no second
        # buffer) and the rebuild stream writes the new rows and table; the
        # next poll clears the word once they are done.  search_tables=
        # False keeps neither (about 130 bytes per corpus position less)
        # and releases the build workspace between builds.
        self.search_tables = bool(search_tables)
        self._keys = None
        self._gram = None
        self.gram_slots = 0
        self.key_select = None
        if self.search_tables:
            self._keys = torch.empty(capacity * KEY_WIDTH, dtype=torch.int32,
                                     device=dev)
            # gram_slots (a multiple of 16) overrides the table size; a
            # table too small for the corpus keeps the run lengths that
            # fit (possibly none).
            self.gram_slots = gram_slots or gram_slots_for(capacity)
            self._gram = torch.zeros(
                int(lib().sfx_gram_table_bytes(self.gram_slots)),
                dtype=torch.uint8, device=dev)
            self.key_select = torch.zeros(1, dtype=torch.int32, device=dev)
        # Ranks from this one on hold padding-suffix rows (the suffix array
        # is the identity there and the corpus PAD), so the next key build
        # rewrites only the rows below max(m, this).
        self._key_rows = capacity
        # the background build of the live array's key rows and table:
        # its event on the rebuild stream until a poll has cleared the
        # selector
        self._tables_event = None
        self._sa_ws: torch.Tensor | None = None
        self._build_tables(0)
        self._query_ws: dict = {}

        self.active_len = 0
        self.delta_len = 0
        self.active_doc_lens: deque[int] = deque()
        self.delta_doc_lens: list[int] = []
        self._rebuild_event = None
        self._pending = None
        # swaps of a rebuild into the live buffers so far
        self.swap_count = 0
        # Device-side ingest (harvest_device): the bookkeeping lives in
        # device memory while _ing_live; poll reads a pinned copy of its
        # header, and the host lists above are refreshed only by
        # sync_host_state (or any host-side write, which calls it).
        self._ing: torch.Tensor | None = None
        self._ing_layout: list[int] | None = None
        self._ing_live = False
        self._ing_mirror = torch.zeros(16, dtype=torch.int64,
                                       pin_memory=True)
        self._ing_event = None
        # swap_count when the pinned header copy was issued: a header
        # copied before a swap holds the corpus length from before it
        self._ing_mirror_swaps = 0
        self._ing_seen_seq = 0
        # device-side ingest totals: documents appended, dropped to make
        # room (and their tokens), rows outside the token buffer
        self.ingest_counters: dict = {}
        # Background rebuilds run their doubling rounds in chunks: the
        # first sized from the rounds the previous build needed (plus a
        # margin), with the radix path enqueued for the rounds that took it
        # then; the rest only if the device reports the array is not final
        # yet, or is stalled at a round that needs the radix path (a pinned
        # copy of the build's state block).  The rounds past those the
        # previous build needed (sa_final_hint on; 0: no build yet) are
        # enqueued as expected to find the array final.
        self.sa_round_hint = 12
        self.sa_radix_hint = DEFAULT_RADIX_MASK
        self.sa_final_hint = 0
        # (m, next_round) while rounds may remain; (m, None) once the suffix
        # array is final and its n-gram table is being built
        self._build_state = None
        self._flag_host = torch.zeros(STATE_WORDS, dtype=torch.int32,
                                      pin_memory=True)

    # ------------------------------------------------------------------
    # device views
    # ------------------------------------------------------------------
    @property
    def sa_key(self) -> torch.Tensor | None:
        """Key rows of the live suffix array ([capacity * 32] int32); being
        rewritten while tables_pending."""
        return self._keys

    @property
    def tables_pending(self) -> bool:
        """The live array's key rows and table are still being built (the
        steps search without them)."""
        return self._tables_event is not None

    def index_struct(self) -> _lib.SfxIndex:
        if self._dix_ent is not None:
            dix = (self._dix_ent.data_ptr(), self._dix_start.data_ptr(),
                   self.delta_buckets)
        else:
            dix = (None, None, 0)
        if not self.search_tables:
            return _lib.SfxIndex(self.corpus.data_ptr(), self.sa.data_ptr(),
                                 self.capacity, self.delta.data_ptr(),
                                 self.delta_capacity,
                                 self.delta_len_t.data_ptr(), None, 0, None,
                                 None, None, None, 0, *dix)
        return _lib.SfxIndex(self.corpus.data_ptr(), self.sa.data_ptr(),
                             self.capacity, self.delta.data_ptr(),
                             self.delta_capacity,
                             self.delta_len_t.data_ptr(),
                             self._keys.data_ptr(), KEY_WIDTH, None,
                             self.key_select.data_ptr(),
                             self._gram.data_ptr(), None, self.gram_slots,
                             *dix)

    def device_bytes(self) -> dict:
        """Device memory held by the index, by role (bytes)."""
        ws = self._sa_ws.numel() if self._sa_ws is not None else 0
        qws = sum(t.numel() for t in self._query_ws.values())
        return {
            "corpus_sa": 4 * 4 * self.capacity,  # live + staging, int32
            "key_rows": 4 * self._keys.numel() if self.search_tables else 0,
            "gram_tables": self._gram.numel() if self.search_tables else 0,
            "delta": 4 * self.delta_capacity + 8,
            "delta_index": sum(t.numel() * t.element_size() for t in (
                self._dix_ent, self._dix_start, self._dix_ws)
                if t is not None),
            "sa_build_workspace": ws,
            "query_workspace": qws,
        }

    def _build_tables(self, m: int) -> None:
        """Key rows and n-gram range table of the live suffix array (m
        ranks hold real suffixes) on the current stream.  Ranks from m on
        are the padding suffixes: their rows are rewritten only where the
        previous build had real ones, and they hold no run of real tokens
        for the table.  The key-row launch also writes each rank's first
        four tokens compactly into the build workspace (dead between
        builds), from which the table is built."""
        if not self.search_tables:
            return
        st = stream_of(self.device)
        rows = max(m, self._key_rows)
        ws = self._sa_workspace() if m > 0 else None
        first4 = ws.data_ptr() if m > 0 else None
        check(lib().sfx_sa_keys(self.corpus.data_ptr(), self.sa.data_ptr(),
                                self.capacity, rows, KEY_WIDTH,
                                self._keys.data_ptr(), first4, st),
              "SA key rows")
        self._key_rows = m
        src = first4 if m > 0 else self._keys.data_ptr()
        check(lib().sfx_gram_build(src, 4 if m > 0 else KEY_WIDTH, m,
                                   self._gram.data_ptr(), self.gram_slots,
                                   st), "n-gram table")

    def _swap_tables(self, m: int, sync: bool) -> None:
        """After a swap (selector set): build the new array's key rows and
        table, on the rebuild stream (cleared by a later poll) or, with
        `sync` or no rebuild stream, on the current one (cleared now)."""
        if not self.search_tables:
            return
        if sync or self.rebuild_stream is None:
            self._build_tables(m)
            self._clear_selector()
            return
        self.rebuild_stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.rebuild_stream):
            self._build_tables(m)
        ev = torch.cuda.Event()
        ev.record(self.rebuild_stream)
        self._tables_event = ev

    def _clear_selector(self) -> None:
        check(lib().sfx_index_swap(None, None, None, None, 0,
                                   self.key_select.data_ptr(), 0,
                                   stream_of(self.device)), "tables live")

    def poll_tables(self, wait: bool = False) -> None:
        """Clear the selector once the key rows and table of the live
        array are built (the current stream waits for their event first),
        so later steps use them again."""
        ev = self._tables_event
        if ev is None:
            return
        if wait:
            ev.synchronize()
        elif not ev.query():
            return
        torch.cuda.current_stream(self.device).wait_event(ev)
        self._clear_selector()
        self._tables_event = None

    def _index_delta(self) -> None:
        """Rebuild the delta token index on the current stream (after
        every write to the delta or its device length)."""
        if self._dix_ent is None:
            return
        check(lib().sfx_delta_index_build(
            self.delta.data_ptr(), self.delta_len_t.data_ptr(),
            self.delta_capacity, self._dix_ent.data_ptr(),
            self._dix_start.data_ptr(), self.delta_buckets,
            self._dix_ws.data_ptr(), self._dix_ws.numel(),
            stream_of(self.device)), "delta index")

    # ------------------------------------------------------------------
    # writes (global_index.py:86-133)
    # ------------------------------------------------------------------
    def append_documents(self, docs: list[torch.Tensor]) -> None:
        """Append token tensors to the delta, each followed by SEP_TOKEN.

        Recorded doc lengths include the separator.  The host takes every
        per-document decision of the reference (truncation to the last
        delta_capacity - 1 tokens, making room); the documents between two
        room-making steps are written by one sfx_delta_append launch.
        """
        self.sync_host_state()
        pending: list[tuple[torch.Tensor, int, int]] = []
        for doc in docs:
            doc = doc.to(self.device).to(torch.int32).reshape(-1)
            n = doc.shape[0]
            if n == 0:
                continue
            if n + 1 > self.delta_capacity:
                doc = doc[-(self.delta_capacity - 1):]
                n = doc.shape[0]
            if self.delta_len + n + 1 > self.delta_capacity:
                self._flush_appends(pending)
                self._make_room(n + 1)
            pending.append((doc.contiguous(), n, self.delta_len))
            self.delta_len += n + 1
            self.delta_doc_lens.append(n + 1)
        self._flush_appends(pending)
        self.maybe_rebuild()

    def _flush_appends(self, pending: list) -> None:
        """Write the pending (doc, n, dst) appends and the delta length."""
        if not pending:
            return
        arr = (_lib.SfxAppendDoc * len(pending))(
            *[_lib.SfxAppendDoc(d.data_ptr(), n, dst)
              for d, n, dst in pending])
        check(lib().sfx_delta_append(arr, len(pending), self.delta.data_ptr(),
                                     self.delta_capacity,
                                     self.delta_len_t.data_ptr(),
                                     self.delta_len, stream_of(self.device)),
              "delta append")
        pending.clear()
        self._index_delta()

    def _shift_delta(self, start: int) -> None:
        """Drop delta[:start]: the rest moves to the front in place and the
        device length follows (one launch)."""
        remaining = self.delta_len - start
        check(lib().sfx_delta_shift(self.delta.data_ptr(),
                                    self.delta_capacity, start, remaining,
                                    self.delta_len_t.data_ptr(),
                                    stream_of(self.device)), "delta shift")
        self.delta_len = remaining
        self._index_delta()

    def _make_room(self, needed: int) -> None:
        self.poll_rebuild()
        if self._rebuild_event is None:
            self._launch_rebuild()
        if self.delta_len + needed <= self.delta_capacity:
            return
        # The staging buffers still belong to the running rebuild, so the
        # delta can only make room by forgetting its earliest documents.
        self._drop_oldest_docs(
            self.delta_len + needed - self.delta_capacity)

    def _drop_oldest_docs(self, drop: int) -> None:
        acc = 0
        dropped = 0
        for ln in self.delta_doc_lens:
            if acc >= drop:
                break
            acc += ln
            dropped += 1
        self._shift_delta(acc)
        self.delta_doc_lens = self.delta_doc_lens[dropped:]

    # ------------------------------------------------------------------
    # rebuild (global_index.py:138-252)
    # ------------------------------------------------------------------
    def maybe_rebuild(self) -> None:
        """Start a background rebuild once the delta holds at least
        rebuild_threshold tokens and none is running."""
        self.sync_host_state()
        self.poll_rebuild()
        if self._rebuild_event is not None or self.delta_len == 0:
            return
        if self.delta_len < self.rebuild_threshold:
            return
        self._launch_rebuild()

    def _plan_rebuild(self) -> tuple[int, int, int, int]:
        """(keep_start, n_active_keep, snap, n_new): evict oldest whole
        docs until the snapshot fits, round the delta snapshot down to
        whole docs (global_index.py:150-167)."""
        keep_start = 0
        for ln in self.active_doc_lens:
            if self.active_len - keep_start + self.delta_len \
                    <= self.capacity:
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
        return keep_start, n_keep, acc, n_keep + acc

    def _launch_rebuild(self) -> None:
        if self._rebuild_event is not None:
            return
        keep_start, n_keep, snap, n_new = self._plan_rebuild()
        if n_new == 0:
            return
        dst = self.staging_corpus
        dst.fill_(PAD_TOKEN)
        if n_keep > 0:
            dst[:n_keep].copy_(self.corpus[keep_start:self.active_len])
        if snap > 0:
            dst[n_keep:n_new].copy_(self.delta[:snap])

        new_doc_lens: deque[int] = deque()
        acc = 0
        for ln in self.active_doc_lens:
            acc += ln
            if acc > keep_start:
                new_doc_lens.append(ln)
        acc = 0
        for ln in self.delta_doc_lens:
            acc += ln
            if acc <= snap:
                new_doc_lens.append(ln)

        # Staging owns a copy of the snapshot: compact it out of the delta
        # now so appends always see the full capacity.
        absorbed = self._count_docs_within(snap)
        self._shift_delta(snap)
        self.delta_doc_lens = self.delta_doc_lens[absorbed:]

        # Real prefix plus one PAD sentinel column, so build-time suffix
        # order equals query-time comparison order.
        m = min(n_new + 1, self.capacity)
        if self.rebuild_stream is not None:
            self.rebuild_stream.wait_stream(
                torch.cuda.current_stream(self.device))
            with torch.cuda.stream(self.rebuild_stream):
                self._staged_build_begin(dst, m)
            event = torch.cuda.Event()
            event.record(self.rebuild_stream)
            self._pending = (n_new, new_doc_lens)
            self._rebuild_event = event
        else:
            self._build_staging_sa(dst, m)
            self._finish_swap(n_new, new_doc_lens)

    def _sa_workspace(self) -> torch.Tensor:
        """The suffix-array build workspace (also where the table build
        finds each rank's first four tokens).  Work enqueued on another
        stream than a pending table build's waits for it first."""
        need = max(sa_workspace_bytes(self.capacity), 16 * self.capacity)
        if self._sa_ws is None or self._sa_ws.numel() < need:
            self._sa_ws = torch.empty(max(need, 1), dtype=torch.uint8,
                                      device=self.device)
        if self._tables_event is not None:
            torch.cuda.current_stream(self.device).wait_event(
                self._tables_event)
        return self._sa_ws

    def _build_staging_sa(self, dst: torch.Tensor, m: int) -> None:
        """staging_sa[:m] = SA(dst[:m]); staging_sa[m:] = m .. N-1."""
        ws = self._sa_workspace()
        check(lib().sfx_sa_build(dst.data_ptr(), m, self.capacity,
                                 self.staging_sa.data_ptr(), 0,
                                 ws.data_ptr(), ws.numel(),
                                 stream_of(self.device)), "SA rebuild")

    # Background builds, enqueued on the current (rebuild) stream.
    def _staged_build_begin(self, dst: torch.Tensor, m: int) -> None:
        """Token round + the hinted doubling rounds, a pinned copy of the
        build state, then (speculatively) the output and key rows."""
        L = lib()
        ws = self._sa_workspace()
        st = stream_of(self.device)
        total = int(L.sfx_sa_build_rounds_total(m))
        first = min(self.sa_round_hint, total)
        check(L.sfx_sa_build_begin(dst.data_ptr(), m, ws.data_ptr(),
                                   ws.numel(), st), "SA rebuild")
        enqueue_rounds(m, 1, first, self.sa_radix_hint, ws.data_ptr(),
                       ws.numel(), st, self.sa_final_hint)
        self._copy_build_state(m)
        self._staged_build_finish(dst, m)
        # Kept even when every round was enqueued: the state copy then
        # still tells how many rounds this text needed (the next hint).
        self._build_state = (m, first + 1)

    def _copy_build_state(self, m: int) -> None:
        if m <= 1:
            self._flag_host.zero_()
            self._flag_host[0] = 1
            return
        self._flag_host.copy_(state_view(self._sa_ws, m), non_blocking=True)

    def _staged_build_finish(self, dst: torch.Tensor, m: int) -> None:
        """The output, speculatively (the host has not seen whether the
        array is final yet)."""
        ws = self._sa_ws
        check(lib().sfx_sa_build_finish(m, self.capacity,
                                        self.staging_sa.data_ptr(), 0,
                                        ws.data_ptr(), ws.numel(),
                                        stream_of(self.device)),
              "SA rebuild")

    def _staged_build_check(self) -> bool:
        """After the build's event: True when the staged output is final;
        otherwise the remaining rounds (from the stalled round, with its
        radix path, when the build stalled), the output and the key rows
        are enqueued again under a new event.  Every state copy of a final
        build sets the round hint to the rounds this text needed plus 2 and
        the radix hint to the rounds that took the radix path, so a
        long-repeat text raises them only until a shorter one follows."""
        if self._build_state is None:
            return True
        m, nxt = self._build_state
        self._build_state = None
        if m <= 1:
            return True  # nothing to sort
        state = BuildState.of(self._flag_host.tolist())
        L = lib()
        total = int(L.sfx_sa_build_rounds_total(m))
        if state.done:
            self.sa_round_hint = state.needed + 2
            self.sa_radix_hint = state.radix_mask & ~1
            self.sa_final_hint = state.needed + 1
            return True
        if state.stalled:
            nxt, radix = state.stalled, 1 << state.stalled
        elif nxt > total:
            # Every round ran; only the round after the last one could
            # have raised the flag, so the array is final as it stands.
            self.sa_round_hint = total
            self.sa_radix_hint = state.radix_mask & ~1
            self.sa_final_hint = 0
            return True
        else:
            radix = 0
        self.rebuild_stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.rebuild_stream):
            ws = self._sa_ws
            enqueue_rounds(m, nxt, total - nxt + 1, radix, ws.data_ptr(),
                           ws.numel(), stream_of(self.device))
            self._copy_build_state(m)
            self._staged_build_finish(self.staging_corpus, m)
        self._build_state = (m, total + 1)
        event = torch.cuda.Event()
        event.record(self.rebuild_stream)
        self._rebuild_event = event
        return False

    def _count_docs_within(self, tokens: int) -> int:
        acc = 0
        count = 0
        for ln in self.delta_doc_lens:
            acc += ln
            if acc > tokens:
                break
            count += 1
        return count

    def _finish_swap(self, n_new: int, new_doc_lens: deque[int],
                     sync_tables: bool = False) -> None:
        # Ring and suffix array are copied into the live tensors (captured
        # graphs hold their pointers) and the selector set in the same
        # launch: the steps search without key rows and table until the
        # new array's are built.  A table build still pending reads the
        # live arrays: the swap waits for it.
        if self._tables_event is not None:
            torch.cuda.current_stream(self.device).wait_event(
                self._tables_event)
            self._tables_event = None
        check(lib().sfx_index_swap(
            self.corpus.data_ptr(), self.sa.data_ptr(),
            self.staging_corpus.data_ptr(), self.staging_sa.data_ptr(),
            self.capacity,
            self.key_select.data_ptr() if self.search_tables else None,
            1, stream_of(self.device)), "swap")
        self._swap_tables(min(n_new + 1, self.capacity), sync_tables)
        self.swap_count += 1
        self.active_len = n_new
        if new_doc_lens is not None:  # None: the device keeps them
            self.active_doc_lens = new_doc_lens
        if self._ing_live:
            check(lib().sfx_ingest_swapped(self._ing.data_ptr(),
                                           stream_of(self.device)),
                  "ingest swap")
        self._rebuild_event = None
        self._pending = None
        if not self.search_tables:
            # the smallest footprint: the build workspace is held only
            # while a build runs (the next one allocates it again)
            self._sa_ws = None

    def poll_rebuild(self) -> None:
        """Swap in a finished background rebuild.  After device-side
        ingest, first read a pinned copy of the device bookkeeping's header
        (issued by an earlier poll and landed by now; with blocking_poll
        issued now and waited for) and start the build of a snapshot the
        device staged."""
        if self._ing_live:
            # the copy is issued here, never by harvest_device
            if self._ing_event is None or self.blocking_poll:
                self._ing_mirror.copy_(self._ing[:128].view(torch.int64),
                                       non_blocking=True)
                self._ing_mirror_swaps = self.swap_count
                self._ing_event = torch.cuda.Event()
                self._ing_event.record(torch.cuda.current_stream(
                    self.device))
            if self.blocking_poll:
                self._ing_event.synchronize()
            if self._ing_event.query():
                self._ing_event = None
                self._read_ingest_mirror()
        self.poll_tables(wait=self.blocking_poll)
        ev = self._rebuild_event
        if ev is None:
            return
        if self.blocking_poll and hasattr(ev, "synchronize"):
            ev.synchronize()
            done = True
        else:
            done = ev.query()
        if done and self._staged_build_check():
            n_new, new_doc_lens = self._pending
            self._finish_swap(n_new, new_doc_lens)
        elif done and self.blocking_poll:
            self.poll_rebuild()  # the remaining rounds, waited for too

    # ------------------------------------------------------------------
    # device-side ingest (proposer.py:329-343 with device lengths)
    # ------------------------------------------------------------------
    def _device_docs_args(self, what: str, idx: torch.Tensor,
                          lengths: torch.Tensor, tokens: torch.Tensor):
        """Checked (idx, lengths, tokens, n) of a device-side ingest call:
        zip() semantics (the shorter of idx and lengths), int32 tokens."""
        for t in (idx, lengths, tokens):
            if not isinstance(t, torch.Tensor) or t.device != self.device:
                raise ValueError(f"{what}: tensors must be on {self.device}")
        if idx.dtype not in (torch.int32, torch.int64) or \
                lengths.dtype not in (torch.int32, torch.int64):
            raise TypeError(f"{what}: int32 or int64 indices and lengths")
        if tokens.dim() != 2:
            raise TypeError(f"{what}: tokens must be a [rows, seq] tensor")
        if tokens.is_floating_point() or tokens.is_complex():
            raise TypeError(f"{what}: integer token ids")
        idx = idx.reshape(-1)
        lengths = lengths.reshape(-1)
        n = min(idx.numel(), lengths.numel())
        if n > _lib.INGEST_MAX_DOCS:
            raise ValueError(f"{what}: at most {_lib.INGEST_MAX_DOCS} "
                             "documents per call")
        tokens = tokens.to(torch.int32).contiguous()
        return idx[:n].contiguous(), lengths[:n].contiguous(), tokens, n

    def harvest_device(self, row_idx: torch.Tensor, lengths: torch.Tensor,
                       tokens: torch.Tensor) -> None:
        """append_documents of tokens[r, :n] for (r, n) in
        zip(row_idx, lengths), with row_idx and lengths in device memory
        (int32 or int64): every decision of append_documents -- truncation,
        making room, dropping the oldest delta documents and the rebuild
        snapshot -- is taken on the device and nothing is read back.  A
        snapshot's build starts from the next poll_rebuild (until it is
        swapped in, the rebuild counts as running), which also refreshes
        delta_len and active_len; the host doc-length lists follow only
        through sync_host_state.  At most 4096 rows per call.  Row indices
        are Python indices (negative ones count from the end); rows outside
        [-rows, rows), where the reference raises IndexError, are skipped
        and counted in ingest_counters["bad_rows"]."""
        row_idx, lengths, tokens, n = self._device_docs_args(
            "harvest_device", row_idx, lengths, tokens)
        if n == 0:
            return
        self._ingest_to_device()
        check(lib().sfx_ingest_docs(
            self._ing.data_ptr(), self.corpus.data_ptr(), self.capacity,
            self.delta.data_ptr(), self.delta_capacity,
            self.delta_len_t.data_ptr(), self.staging_corpus.data_ptr(),
            tokens.data_ptr(), tokens.shape[0], tokens.shape[1],
            row_idx.data_ptr(), int(row_idx.dtype == torch.int64),
            lengths.data_ptr(), int(lengths.dtype == torch.int64), n,
            self.rebuild_threshold, stream_of(self.device)), "ingest")
        self._index_delta()

    def ingest_active_device(self, keys: torch.Tensor, rows: torch.Tensor,
                             lengths: torch.Tensor, ingested: torch.Tensor,
                             final: bool, chunk: int, overlap: int) -> None:
        """ingest_active's chunking (proposer.py:354-390) on the device:
        keys are slots of the int64 progress table `ingested`, row i of
        `rows` belongs to keys[i]; the documents it emits go through the
        same device-side append_documents as harvest_device.  Keys outside
        the table are skipped and counted in ingest_counters["bad_rows"]."""
        keys, lengths, rows, n = self._device_docs_args(
            "ingest_active", keys, lengths, rows)
        n = min(n, rows.shape[0])
        if n == 0:
            return
        if ingested.dtype != torch.int64 or ingested.device != self.device \
                or not ingested.is_contiguous():
            raise TypeError("ingest_active: the progress table must be a "
                            f"contiguous int64 tensor on {self.device}")
        self._ingest_to_device()
        check(lib().sfx_ingest_active(
            self._ing.data_ptr(), self.corpus.data_ptr(), self.capacity,
            self.delta.data_ptr(), self.delta_capacity,
            self.delta_len_t.data_ptr(), self.staging_corpus.data_ptr(),
            rows.data_ptr(), rows.shape[0], rows.shape[1],
            keys.data_ptr(), int(keys.dtype == torch.int64),
            lengths.data_ptr(), int(lengths.dtype == torch.int64), n,
            ingested.data_ptr(), ingested.numel(), int(bool(final)),
            int(chunk), int(overlap), self.rebuild_threshold,
            stream_of(self.device)), "ingest_active")
        self._index_delta()

    def _ingest_header(self, words) -> dict:
        return dict(zip(_lib.INGEST_HEADER_FIELDS, (int(x) for x in words)))

    def _ingest_to_device(self) -> None:
        """Make the device bookkeeping authoritative (host lists uploaded;
        a rebuild the host started counts as running there)."""
        if self._ing_live:
            return
        if self._ing is None:
            lay = (ctypes_i64 * 8)()
            check(lib().sfx_ingest_layout(self.capacity, self.delta_capacity,
                                          lay), "ingest layout")
            self._ing_layout = [int(x) for x in lay]
            self._ing = torch.zeros(self._ing_layout[0], dtype=torch.uint8,
                                    device=self.device)
        total, acap, dcap, aoff, doff = self._ing_layout[:5]
        running = self._rebuild_event is not None
        if running:
            n_new, new_lens = self._pending
            plan_len, plan_lens = n_new, list(new_lens)
        else:
            plan_len, plan_lens = self.active_len, list(self.active_doc_lens)
        head = [0] * 16
        head[0] = plan_len
        head[1] = self.active_len
        head[2] = self.delta_len
        head[4] = len(plan_lens)
        head[6] = len(self.delta_doc_lens)
        head[7] = int(running)
        for i, name in enumerate(("docs_in", "docs_dropped",
                                  "tokens_dropped", "bad_rows")):
            head[11 + i] = self.ingest_counters.get(name, 0)
        self._ing[:128].view(torch.int64).copy_(
            torch.tensor(head, dtype=torch.int64))
        if plan_lens:
            self._ing[aoff:aoff + 4 * len(plan_lens)].view(torch.int32) \
                .copy_(torch.tensor(plan_lens, dtype=torch.int32))
        if self.delta_doc_lens:
            self._ing[doff:doff + 4 * len(self.delta_doc_lens)] \
                .view(torch.int32).copy_(
                    torch.tensor(self.delta_doc_lens, dtype=torch.int32))
        self._ing_seen_seq = 0
        self._ing_live = True

    def _read_ingest_mirror(self) -> None:
        h = self._ingest_header(self._ing_mirror.tolist())
        self.delta_len = h["delta_len"]
        if self._ing_mirror_swaps == self.swap_count:
            # (a copy issued before a swap since then holds the corpus
            # length from before it; _finish_swap has set the new one)
            self.active_len = h["live_active_len"]
        self.ingest_counters = {k: h[k] for k in (
            "docs_in", "docs_dropped", "tokens_dropped", "bad_rows")}
        if h["snap_seq"] > self._ing_seen_seq:
            self._ing_seen_seq = h["snap_seq"]
            self._start_staged_build(h["snap_n_new"], h["snap_m"], None)

    def _start_staged_build(self, n_new: int, m: int, new_doc_lens) -> None:
        """Build staging_corpus[:m] (already written) and swap it in: in
        the background on rebuild_stream, else now."""
        dst = self.staging_corpus
        if self.rebuild_stream is not None:
            self.rebuild_stream.wait_stream(
                torch.cuda.current_stream(self.device))
            with torch.cuda.stream(self.rebuild_stream):
                self._staged_build_begin(dst, m)
            event = torch.cuda.Event()
            event.record(self.rebuild_stream)
            self._pending = (n_new, new_doc_lens)
            self._rebuild_event = event
        else:
            self._build_staging_sa(dst, m)
            self._finish_swap(n_new, new_doc_lens)

    def _read_device_state(self) -> dict:
        """Header fields and both doc-length rings of the device
        bookkeeping (one device read; waits for the current stream)."""
        raw = self._ing.cpu()
        h = self._ingest_header(raw[:128].view(torch.int64).tolist())
        total, acap, dcap, aoff, doff = self._ing_layout[:5]

        def ring(off, cap, head, cnt):
            r = raw[off:off + 4 * cap].view(torch.int32)
            idx = [(head + i) % cap for i in range(cnt)]
            return r[idx].tolist() if cnt else []

        h["corpus_doc_lens"] = ring(aoff, acap, h["active_head"],
                                    h["active_docs"])
        h["delta_doc_lens"] = ring(doff, dcap, h["delta_head"],
                                   h["delta_docs"])
        h["_raw_header"] = raw[:128].view(torch.int64)
        return h

    def sync_host_state(self) -> None:
        """Bring the device bookkeeping of harvest_device back into the
        host fields and lists (reads device memory; waits for the stream).
        A staged snapshot whose build has not started is started first.
        Host-side writes call this themselves."""
        if not self._ing_live:
            return
        self._ing_event = None
        h = self._read_device_state()
        self._ing_mirror.copy_(h["_raw_header"])
        self._ing_mirror_swaps = self.swap_count
        self._read_ingest_mirror()
        self.delta_doc_lens = h["delta_doc_lens"]
        self.delta_len = h["delta_len"]
        if self._rebuild_event is not None:
            # running: the device lists already describe the corpus after
            # the swap
            n_new, _ = self._pending
            self._pending = (n_new, deque(h["corpus_doc_lens"]))
        else:
            self.active_len = h["active_len"]
            self.active_doc_lens = deque(h["corpus_doc_lens"])
        self._ing_live = False

    def device_state(self) -> dict:
        """The bookkeeping of device-side ingest as the device holds it,
        read without handing it back to the host (so later harvests stay
        device-resident): the header fields, and the two doc-length lists
        -- "corpus_doc_lens" describes the corpus once a staged or running
        rebuild is swapped in, "delta_doc_lens" the delta.  Waits for the
        current stream.  Before any device-side ingest: the host's."""
        if not self._ing_live:
            running = self._rebuild_event is not None
            return {"active_len": (self._pending[0] if running
                                   else self.active_len),
                    "live_active_len": self.active_len,
                    "delta_len": self.delta_len, "in_flight": int(running),
                    "corpus_doc_lens": list(self._pending[1] if running
                                            else self.active_doc_lens),
                    "delta_doc_lens": list(self.delta_doc_lens)}
        h = self._read_device_state()
        del h["_raw_header"]
        return h

    # ------------------------------------------------------------------
    # persistence (this library's own format; suffixgpu_amd.persist)
    # ------------------------------------------------------------------
    def save(self, path) -> None:
        """Write the index to ``path``.  An in-flight rebuild is completed
        (and swapped in) first, so the file holds one consistent state."""
        self.sync_host_state()
        from suffixgpu_amd.persist import write_index_file
        if self._rebuild_event is not None:
            blocking = self.blocking_poll
            self.blocking_poll = True
            try:
                self.poll_rebuild()
            finally:
                self.blocking_poll = blocking
        m = min(self.active_len + 1, self.capacity) if self.active_len else 0
        arrays = {
            "corpus": self.corpus[:m].cpu().numpy(),
            "sa": self.sa[:m].cpu().numpy(),
            "delta": self.delta[:self.delta_len].cpu().numpy(),
        }
        meta = {
            "capacity": self.capacity,
            "delta_capacity": self.delta_capacity,
            "k": self.k,
            "max_occurrences": self.max_occurrences,
            "rebuild_threshold": self.rebuild_threshold,
            "active_len": self.active_len,
            "delta_len": self.delta_len,
            "active_doc_lens": list(self.active_doc_lens),
            "delta_doc_lens": list(self.delta_doc_lens),
            "sa_prefix": m,
            "pad_token": PAD_TOKEN,
            "sep_token": SEP_TOKEN,
        }
        write_index_file(path, meta, arrays)

    def restore(self, path) -> None:
        """Load a saved index into this one, in place (tensor identities
        are kept, so captured graphs stay valid).  Capacities must match;
        any in-flight rebuild is dropped."""
        self.sync_host_state()
        from suffixgpu_amd.persist import IndexFormatError, read_index_file
        meta, arrays = read_index_file(path)
        if (meta["capacity"] != self.capacity
                or meta["delta_capacity"] != self.delta_capacity):
            raise IndexFormatError(
                f"{path}: capacity {meta['capacity']}/"
                f"{meta['delta_capacity']} does not match this index "
                f"({self.capacity}/{self.delta_capacity})")
        if (meta["pad_token"] != PAD_TOKEN
                or meta["sep_token"] != SEP_TOKEN):
            raise IndexFormatError(f"{path}: different sentinel tokens")
        m = int(meta["sa_prefix"])
        n_act, n_del = int(meta["active_len"]), int(meta["delta_len"])
        if (arrays["corpus"].shape != (m,) or arrays["sa"].shape != (m,)
                or arrays["delta"].shape != (n_del,) or m > self.capacity
                or n_act > self.capacity or n_del > self.delta_capacity
                or sum(meta["active_doc_lens"]) != n_act
                or sum(meta["delta_doc_lens"]) != n_del):
            raise IndexFormatError(f"{path}: inconsistent index state")
        if self._rebuild_event is not None:
            self._rebuild_event.synchronize()
        self._rebuild_event = None
        self._pending = None
        self._build_state = None
        dev = self.device
        self.corpus.fill_(PAD_TOKEN)
        self.corpus[:m].copy_(torch.from_numpy(arrays["corpus"]).to(dev))
        self.sa.copy_(torch.arange(self.capacity, dtype=torch.int32,
                                   device=dev))
        self.sa[:m].copy_(torch.from_numpy(arrays["sa"]).to(dev))
        self.delta.zero_()
        self.delta[:n_del].copy_(torch.from_numpy(arrays["delta"]).to(dev))
        self.delta_len = n_del
        self.delta_len_t.fill_(n_del)
        self._index_delta()
        self.active_len = n_act
        self.active_doc_lens = deque(int(x) for x in meta["active_doc_lens"])
        self.delta_doc_lens = [int(x) for x in meta["delta_doc_lens"]]
        if self._tables_event is not None:
            self._tables_event.synchronize()
            self._tables_event = None
        self._build_tables(m)
        if self.search_tables:
            self._clear_selector()

    @classmethod
    def from_file(cls, path, device="cuda",
                  rebuild_stream: torch.cuda.Stream | None = None
                  ) -> "GlobalIndex":
        """A new index with the geometry and state saved in ``path``."""
        from suffixgpu_amd.persist import read_index_file
        meta, _ = read_index_file(path)
        gi = cls(meta["capacity"], meta["delta_capacity"], meta["k"],
                 max_occurrences=meta["max_occurrences"],
                 rebuild_threshold=meta["rebuild_threshold"], device=device,
                 rebuild_stream=rebuild_stream)
        gi.restore(path)
        return gi

    def load_documents(self, docs: list[torch.Tensor]) -> None:
        """Make ``docs`` (oldest first) the active corpus in one rebuild.

        The state equals what a rebuild whose active set is exactly these
        documents leaves behind: corpus = docs each + SEP, then PAD; SA
        over the first min(n + 1, capacity) positions.  The delta is left
        untouched.  Synchronous on the current stream.
        """
        self.sync_host_state()
        if self._rebuild_event is not None:
            raise RuntimeError("load_documents: a rebuild is in flight")
        lens = [int(d.numel()) + 1 for d in docs]
        n = sum(lens)
        if n > self.capacity:
            raise ValueError("load_documents: documents exceed capacity")
        dst = self.staging_corpus
        dst.fill_(PAD_TOKEN)
        off = 0
        for d in docs:
            d = d.to(self.device).to(torch.int32).reshape(-1)
            dst[off:off + d.shape[0]].copy_(d)
            dst[off + d.shape[0]] = SEP_TOKEN
            off += d.shape[0] + 1
        self._build_staging_sa(dst, min(n + 1, self.capacity))
        self._finish_swap(n, deque(lens), sync_tables=True)

    # ------------------------------------------------------------------
    # queries (global_index.py:257-553)
    # ------------------------------------------------------------------
    def _run_query(self, query, query_len, max_len, caps, *, want,
                   k=None, min_token_prob=0.0, max_spec_factor=None,
                   max_spec_offset=0.0, alpha=0.0):
        require_gpu(query, query_len)
        b = query.shape[0]
        dev = self.device
        caps_l = ([int(x) for x in caps.tolist()]
                  if isinstance(caps, torch.Tensor) else list(caps))
        cnum = len(caps_l)
        r = self.max_occurrences
        kk = self.k if k is None else k
        p = _lib.make_params(kk, max_len, r, 1, (1,), caps_l,
                             max_spec_factor, max_spec_offset,
                             min_token_prob, alpha)
        q = query.to(torch.int32).contiguous()
        ql = query_len.to(torch.int64).contiguous()
        out = _lib.SfxGlobalOut()
        res = {}

        def alloc(name, shape, dtype):
            t = torch.empty(*shape, dtype=dtype, device=dev)
            setattr(out, name, t.data_ptr())
            res[name] = t

        shapes = {
            "sa_len": ((b, cnum), torch.int64),
            "sa_start": ((b, cnum), torch.int64),
            "sa_end": ((b, cnum), torch.int64),
            "d_len": ((b, cnum), torch.int64),
            "d_pos": ((b, cnum, r), torch.int64),
            "d_cnt": ((b, cnum), torch.int64),
            "len": ((b, cnum), torch.int64),
            "cont": ((b, cnum, r, kk), torch.int32),
            "occ": ((b, cnum), torch.int64),
            "draft": ((b, kk), torch.int32),
            "emit": ((b,), torch.int64),
            "draft_len": ((b,), torch.int64),
            "draft_occ": ((b,), torch.int64),
            "draft_score": ((b,), torch.float32),
        }
        for name in want:
            alloc(name, *shapes[name])
        nbytes = int(lib().sfx_global_query_workspace_size(
            p, b, self.delta_capacity))
        ws = self._query_ws.get((b, cnum, kk))
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(max(1, nbytes), dtype=torch.uint8, device=dev)
            self._query_ws[(b, cnum, kk)] = ws
        if b:
            check(lib().sfx_global_query(p, self.index_struct(),
                                         q.data_ptr(), b, q.shape[1],
                                         ql.data_ptr(), out, ws.data_ptr(),
                                         ws.numel(), stream_of(dev)),
                  "GlobalIndex query")
        return res

    def query(self, query: torch.Tensor, query_len: torch.Tensor,
              max_len: int):
        """(match_len [B] i64, cont [B, R, k] int32, occ_count [B] i64)."""
        res = self._run_query(query, query_len, max_len, [max_len],
                              want=("len", "cont", "occ"))
        return res["len"][:, 0], res["cont"][:, 0], res["occ"][:, 0]

    def _query_backoff(self, query: torch.Tensor, query_len: torch.Tensor,
                       max_len: int, caps):
        """(match_len [B, C] i64, cont [B, C, R, k] int32, occ [B, C] i64)."""
        res = self._run_query(query, query_len, max_len, caps,
                              want=("len", "cont", "occ"))
        return res["len"], res["cont"], res["occ"]

    def _delta_match_backoff(self, query: torch.Tensor,
                             query_len: torch.Tensor, max_len: int, caps):
        """(match_len [B, C], starts [B, C, R], count [B, C]) in the delta."""
        res = self._run_query(query, query_len, max_len, caps,
                              want=("d_len", "d_pos", "d_cnt"))
        return res["d_len"], res["d_pos"], res["d_cnt"]

    def draft(self, query: torch.Tensor, query_len: torch.Tensor,
              max_len: int, k: int, min_token_prob: float = 0.0,
              max_spec_factor: float | None = None,
              max_spec_offset: float = 0.0, caps=None, alpha: float = 0.0):
        """(chain [B, k] int32, num_valid [B] i64, match_len [B] i64,
        occ_count [B] i64, score [B] f32) of the best-scored cap."""
        if caps is None:
            caps = sorted({max_len, max(2, max_len // 2),
                           max(2, max_len // 4), 2}, reverse=True)
        res = self._run_query(
            query, query_len, max_len, caps,
            want=("draft", "emit", "draft_len", "draft_occ", "draft_score"),
            k=k, min_token_prob=min_token_prob,
            max_spec_factor=max_spec_factor,
            max_spec_offset=max_spec_offset, alpha=alpha)
        return (res["draft"], res["emit"], res["draft_len"],
                res["draft_occ"], res["draft_score"])

    def expand(self, cont: torch.Tensor, occ_count: torch.Tensor,
               min_token_prob: float = 0.0):
        chain, num_valid, _, _ = expand_chain(
            cont, occ_count, self.k, min_token_prob=min_token_prob)
        return chain, num_valid
