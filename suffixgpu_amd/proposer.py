"""SuffixGPUDrafter: the drop-in drafter API on gfx950.

Mirrors suffix_gpu/proposer.py:26-393 (constructor, update_state,
propose_with_update, propose, poll, harvest_finished, harvest_rows,
ingest_active, load_model).  Device tensors in and out, no host
synchronisation on the step, static shapes: a step is one kernel launch on
the current stream (local, SA-search and delta-scan workgroups per row), so
``torch.cuda.graph`` captures it as a single node.

Local candidates use support thresholds 2^0..2^(C-1); global candidates use
length caps max(2, P >> i) for i < C-1 plus 2, deduplicated, descending
(proposer.py:71-85).  Local and global winners compete by score; global
wins only on a strictly greater score (proposer.py:290-320).
"""

from __future__ import annotations

import torch

from suffixgpu_amd import _lib
from suffixgpu_amd._lib import check, lib, stream_of
from suffixgpu_amd.global_index import GlobalIndex
from suffixgpu_amd.local_matcher import LocalMatchKernel

# Slots of the device table behind ingest_active with device keys: one
# int64 of progress per in-flight request slot.
INGEST_SLOTS = 1 << 16


def backoff_thresholds(num_backoff: int) -> tuple[int, ...]:
    return tuple(2 ** i for i in range(max(1, int(num_backoff))))


def global_caps(max_pattern_len: int, num_backoff: int) -> list[int]:
    nb = max(1, int(num_backoff))
    if nb == 1:
        caps = [max_pattern_len]
    else:
        caps = [max(2, max_pattern_len >> i) for i in range(nb - 1)] + [2]
    return sorted(set(caps), reverse=True)


class SuffixGPUDrafter:
    """Device-resident suffix-decoding drafter (vLLM NgramProposerGPU
    contract: device tensors in, device tensors out, no host sync)."""

    def __init__(
        self,
        k: int,
        device: torch.device | str = "cuda",
        max_pattern_len: int = 32,
        min_match_len: int = 1,
        max_occurrences: int = 128,
        enable_global: bool = False,
        global_capacity: int = 1 << 22,
        delta_capacity: int = 1 << 16,
        rebuild_threshold: int | None = None,
        rebuild_stream: torch.cuda.Stream | None = None,
        max_spec_factor: float | None = None,
        max_spec_offset: float = 0.0,
        min_token_prob: float = 0.0,
        num_backoff: int = 8,
        vote_smoothing_alpha: float = 0.0,
        parallel_paths: bool = True,
        global_search_tables: bool = True,
        global_gram_slots: int | None = None,
        global_delta_index: bool = True,
    ):
        self.k = k
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise _lib.SuffixGPUError(
                "SuffixGPUDrafter needs a ROCm GPU device; there is no CPU "
                "path")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.max_pattern_len = max_pattern_len
        self.max_spec_factor = max_spec_factor
        self.max_spec_offset = max_spec_offset
        self.min_token_prob = min_token_prob
        self.num_backoff = max(1, int(num_backoff))
        self.vote_smoothing_alpha = float(vote_smoothing_alpha)
        # The local and global paths always run concurrently: they are
        # workgroups of the same launch.  Kept for API compatibility.
        self.parallel_paths = bool(parallel_paths)
        support_thresholds = backoff_thresholds(self.num_backoff)
        caps = global_caps(max_pattern_len, self.num_backoff)
        self._global_caps = torch.tensor(caps, dtype=torch.int64,
                                         device=self.device)
        self.local_kernel = LocalMatchKernel(
            k=k, max_pattern_len=max_pattern_len,
            min_match_len=min_match_len, max_occurrences=max_occurrences,
            min_token_prob=min_token_prob, max_spec_factor=max_spec_factor,
            max_spec_offset=max_spec_offset,
            support_thresholds=support_thresholds,
            vote_smoothing_alpha=self.vote_smoothing_alpha,
        ).to(self.device)
        self._params = _lib.make_params(
            k, max_pattern_len, max_occurrences, min_match_len,
            support_thresholds, caps if enable_global else (),
            max_spec_factor, max_spec_offset, min_token_prob,
            self.vote_smoothing_alpha)
        self.global_index: GlobalIndex | None = None
        self._ingested: dict = {}
        # per-slot progress of ingest_active with device keys
        self._ingested_dev: torch.Tensor | None = None
        self._ws: dict[tuple, torch.Tensor] = {}
        if enable_global:
            self.global_index = GlobalIndex(
                capacity=global_capacity, delta_capacity=delta_capacity,
                k=k, max_occurrences=max_occurrences,
                rebuild_threshold=rebuild_threshold, device=self.device,
                rebuild_stream=rebuild_stream,
                search_tables=global_search_tables,
                gram_slots=global_gram_slots,
                delta_index=global_delta_index)

    # ------------------------------------------------------------------
    def poll(self) -> None:
        """Called by the host between steps: a background rebuild whose
        event has completed becomes the live index."""
        if self.global_index is not None:
            self.global_index.poll_rebuild()

    def update_state(self, num_tokens_no_spec: torch.Tensor,
                     token_ids_gpu: torch.Tensor,
                     sampled_token_ids: torch.Tensor,
                     valid_sampled_tokens_count: torch.Tensor | None = None,
                     ) -> torch.Tensor:
        """Scatter last step's sampled ids into the resident rows and return
        the updated counts [B] int32 (proposer.py:135-184)."""
        bt, keep = _lib.make_batch(token_ids_gpu, num_tokens_no_spec,
                                   sampled=sampled_token_ids,
                                   valid_count=valid_sampled_tokens_count)
        new = torch.empty(token_ids_gpu.shape[0], dtype=torch.int32,
                          device=token_ids_gpu.device)
        if new.numel():
            check(lib().sfx_scatter_append(bt, new.data_ptr(),
                                           stream_of(token_ids_gpu.device)),
                  "update_state")
        del keep
        return new

    def propose_with_update(self, num_tokens_no_spec: torch.Tensor,
                            token_ids_gpu: torch.Tensor,
                            sampled_token_ids: torch.Tensor,
                            valid_sampled_tokens_count: torch.Tensor | None
                            = None,
                            max_model_len: int | None = None):
        """update_state + eligibility mask + propose, in one fused step.

        Rows draft only when they accepted at least one token and stay
        below min(max_model_len, S).  Returns (draft [B, k] int32,
        num_valid [B] int32, new_num_tokens [B] int32).
        """
        s = token_ids_gpu.shape[1]
        limit = s if max_model_len is None else min(max_model_len, s)
        return self._step(num_tokens_no_spec, token_ids_gpu,
                          sampled_token_ids, valid_sampled_tokens_count,
                          None, limit)

    def propose(self, num_tokens_no_spec: torch.Tensor,
                token_ids_gpu: torch.Tensor,
                combined_mask: torch.Tensor | None = None):
        """Draft from local history and the global index.

        Returns (draft_tokens [B, k] int32, num_valid [B] int32).
        """
        draft, nv, _ = self._step(num_tokens_no_spec, token_ids_gpu, None,
                                  None, combined_mask, 0)
        return draft, nv

    def _workspace(self, b: int, stream: int) -> torch.Tensor:
        """The fused step's workspace for `b` rows.

        Its handover counters must be zero when a call starts, and every
        call leaves them zero, so two calls that share a workspace must
        not run at the same time.  Eager calls therefore get one per
        (batch size, stream): two streams driving one drafter never share.
        Calls recorded into a HIP graph get one per batch size of their
        own ("graph"), so a replay never shares with an eager call on any
        stream.  It is made (and zeroed) outside the capture at the first
        eager call of that batch size -- a capture records no fill -- or,
        when a capture comes first, inside it (the replay then re-zeroes
        it, which is harmless).  Replays of graphs captured for one batch
        size share that workspace and must not overlap each other."""
        capturing = torch.cuda.is_current_stream_capturing()
        key = (b, "graph") if capturing else (b, stream)
        ws = self._ws.get(key)
        if ws is None:
            ws = self._new_workspace(b)
            self._ws[key] = ws
        if not capturing and (b, "graph") not in self._ws:
            self._ws[(b, "graph")] = self._new_workspace(b)
        return ws

    def _new_workspace(self, b: int) -> torch.Tensor:
        dcap = (self.global_index.delta_capacity
                if self.global_index is not None else 0)
        nbytes = int(lib().sfx_step_workspace_size(self._params, b, dcap))
        return torch.zeros(max(1, nbytes), dtype=torch.uint8,
                           device=self.device)

    def _step(self, num_tokens, tokens, sampled, valid_cnt, mask, limit):
        bt, keep = _lib.make_batch(tokens, num_tokens, sampled=sampled,
                                   valid_count=valid_cnt, mask=mask,
                                   limit=limit)
        b = tokens.shape[0]
        dev = tokens.device
        draft = torch.empty(b, self.k, dtype=torch.int32, device=dev)
        num_valid = torch.empty(b, dtype=torch.int32, device=dev)
        new = (torch.empty(b, dtype=torch.int32, device=dev)
               if sampled is not None else None)
        if b == 0:
            return draft, num_valid, new
        L = lib()
        cur = torch.cuda.current_stream(dev).cuda_stream
        if self.global_index is None:
            check(L.sfx_propose_step(self._params, None, bt,
                                     draft.data_ptr(), num_valid.data_ptr(),
                                     _lib.ptr(new), None, 0, cur),
                  "propose")
            del keep
            return draft, num_valid, new
        ws = self._workspace(b, cur)
        rc = L.sfx_propose_step(self._params,
                                self.global_index.index_struct(), bt,
                                draft.data_ptr(), num_valid.data_ptr(),
                                _lib.ptr(new), ws.data_ptr(), ws.numel(),
                                cur)
        if rc != 0:
            ws.zero_()  # never leave handover counters half set
        check(rc, "propose")
        del keep
        return draft, num_valid, new

    # ------------------------------------------------------------------
    # host-side ingestion (proposer.py:329-393)
    # ------------------------------------------------------------------
    def harvest_finished(self, row_indices: list[int], lengths: list[int],
                         token_ids_gpu: torch.Tensor) -> None:
        """Append rows[:length] of finished requests to the global memory
        (proposer.py:329-343).  With row_indices and lengths as tensors on
        the drafter's device the appends and every decision about them run
        on the device (GlobalIndex.harvest_device): nothing is read back,
        and a rebuild they trigger starts at the next poll().  Host lists
        (or host tensors) take the host path."""
        if self.global_index is None:
            return
        if (isinstance(row_indices, torch.Tensor)
                and isinstance(lengths, torch.Tensor)
                and row_indices.device == self.device
                and lengths.device == self.device):
            self.global_index.harvest_device(row_indices.reshape(-1),
                                             lengths.reshape(-1),
                                             token_ids_gpu)
            return
        if isinstance(row_indices, torch.Tensor):
            row_indices = row_indices.tolist()
        if isinstance(lengths, torch.Tensor):
            lengths = lengths.tolist()
        rows = [token_ids_gpu[r] for r in row_indices]
        self.harvest_rows(rows, lengths)

    def harvest_rows(self, rows: list[torch.Tensor],
                     lengths: list[int]) -> None:
        if self.global_index is None or not rows:
            return
        docs = [row[:ln] for row, ln in zip(rows, lengths) if ln > 0]
        if docs:
            self.global_index.append_documents(docs)

    def ingest_active(self, keys: list, rows: list[torch.Tensor],
                      lengths: list[int], final: bool = False,
                      chunk: int = 64) -> None:
        """Feed in-flight responses in chunks overlapping by P + k tokens
        (proposer.py:354-390).

        With keys and lengths as integer tensors on the drafter's device
        and rows a [n, seq] device tensor (row i for keys[i]), everything
        runs on the device: the keys are slots in [0, INGEST_SLOTS) of a
        device table of per-slot progress, the chunk / overlap / final
        rules and every append_documents decision are taken there, and
        nothing is read back (GlobalIndex.ingest_active_device).  Slot
        keys outside the table are skipped and counted in the index's
        ingest_counters["bad_rows"].  Host keys keep the reference's
        dict (``_ingested``); the two tables are separate."""
        if self.global_index is None:
            return
        overlap = self.max_pattern_len + self.k
        if (isinstance(keys, torch.Tensor) and isinstance(rows, torch.Tensor)
                and isinstance(lengths, torch.Tensor)
                and keys.device == self.device
                and lengths.device == self.device
                and rows.device == self.device and rows.dim() == 2):
            if self._ingested_dev is None:
                self._ingested_dev = torch.zeros(
                    INGEST_SLOTS, dtype=torch.int64, device=self.device)
            self.global_index.ingest_active_device(
                keys, rows, lengths, self._ingested_dev, final, chunk,
                overlap)
            return
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

    def save_global_index(self, path) -> None:
        """Persist the global memory (see GlobalIndex.save)."""
        if self.global_index is None:
            raise RuntimeError("save_global_index: global memory is off")
        self.global_index.save(path)

    def load_global_index(self, path) -> None:
        """Restore saved global memory into this drafter, in place."""
        if self.global_index is None:
            raise RuntimeError("load_global_index: global memory is off")
        self.global_index.restore(path)

    def load_model(self, *args, **kwargs) -> None:
        pass
