"""Engine adapter: the scatter / propose wiring an inference engine needs
around SuffixGPUDrafter.

The reference leaves this wiring to the engine: its tests name the vLLM
adapter ``SuffixProposerGPU`` and mimic its propose, which scatters the
verifier's sampled tokens into the resident token buffer and then drafts
with the updated lengths (suffix_gpu tests/test_verification.py:8-11,
39-49).  This module is that adapter, built on the fused step:

* it owns the resident state of a persistent batch -- token rows
  ``[max_num_seqs, max_model_len]`` and committed counts ``[max_num_seqs]``,
  both int32 on the device -- and a host map from request id to slot, with
  the live requests condensed into slots ``0 .. num_active - 1`` in batch
  order (a finished request's slot is refilled by the last live one);
* ``propose`` hands the verifier's sampled ids (device, ``[num_active, T]``,
  -1 padded) to one ``propose_with_update`` launch and copies the new counts
  back into the resident counts on the device.  No step reads device memory
  on the host, so an engine may queue the next step before this step's
  tokens are known (asynchronous scheduling), and a captured graph of
  ``propose`` holds two nodes;
* ``finish_requests`` harvests the finished rows into the global memory at
  the lengths the engine reports (it streams the tokens, so it knows them on
  the host), then condenses the batch;
* ``add_request`` stages a prompt through pinned memory without blocking.
"""

from __future__ import annotations

import numpy as np
import torch

from suffixgpu_amd.proposer import SuffixGPUDrafter


class SlotTable:
    """Request id <-> slot map of a condensed persistent batch (host only).

    ``add`` appends at the first free slot; ``remove`` frees slots and
    returns the moves ``(src, dst)`` that refill each hole, lowest hole
    first, with the highest live slot -- the order in which the device rows
    must be copied.
    """

    def __init__(self, capacity: int):
        self.capacity = int(capacity)
        self.req_at: list = []          # slot -> request id
        self.slot_of: dict = {}         # request id -> slot

    def __len__(self) -> int:
        return len(self.req_at)

    def add(self, req_id) -> int:
        if req_id in self.slot_of:
            raise KeyError(f"request {req_id!r} is already active")
        if len(self.req_at) >= self.capacity:
            raise RuntimeError("no free slot: max_num_seqs requests active")
        slot = len(self.req_at)
        self.req_at.append(req_id)
        self.slot_of[req_id] = slot
        return slot

    def remove(self, req_ids) -> list[tuple[int, int]]:
        holes = sorted(self.slot_of[r] for r in req_ids)
        if len(set(holes)) != len(holes):
            raise KeyError("a request id is given twice")
        for r in req_ids:
            del self.slot_of[r]
        dead = set(holes)
        moves = []
        last = len(self.req_at) - 1
        for hole in holes:
            while last > hole and last in dead:
                last -= 1
            if last <= hole:
                break
            rid = self.req_at[last]
            self.req_at[hole] = rid
            self.slot_of[rid] = hole
            moves.append((last, hole))
            dead.add(last)
            last -= 1
        del self.req_at[len(self.req_at) - len(holes):]
        return moves


class SuffixProposerGPU:
    """Persistent-batch drafter for an inference engine (see module doc).

    ``drafter_kwargs`` are SuffixGPUDrafter's (enable_global,
    max_spec_factor, min_token_prob, rebuild_stream, ...); an existing
    ``drafter`` (with its global memory) may be passed instead.
    """

    def __init__(self, k: int, max_num_seqs: int, max_model_len: int,
                 device: torch.device | str = "cuda",
                 drafter: SuffixGPUDrafter | None = None, **drafter_kwargs):
        if drafter is None:
            drafter = SuffixGPUDrafter(k=k, device=device, **drafter_kwargs)
        elif drafter_kwargs or drafter.k != k:
            raise ValueError("pass either a drafter or drafter arguments")
        self.drafter = drafter
        self.k = k
        self.device = self.drafter.device
        self.max_num_seqs = int(max_num_seqs)
        self.max_model_len = int(max_model_len)
        self.tokens = torch.zeros(self.max_num_seqs, self.max_model_len,
                                  dtype=torch.int32, device=self.device)
        self.num_tokens = torch.zeros(self.max_num_seqs, dtype=torch.int32,
                                      device=self.device)
        self.slots = SlotTable(self.max_num_seqs)
        # pinned prompt buffers and the events after their copies
        self._staged: list[tuple[torch.cuda.Event, torch.Tensor]] = []

    @property
    def num_active(self) -> int:
        return len(self.slots)

    def load_model(self, *args, **kwargs) -> None:
        pass

    def add_request(self, req_id, prompt_token_ids) -> int:
        """Place a new request's prompt in the next free slot."""
        prompt = np.asarray(prompt_token_ids, dtype=np.int32).reshape(-1)
        n = prompt.shape[0]
        if n > self.max_model_len:
            raise ValueError(f"prompt of {n} tokens exceeds max_model_len "
                             f"{self.max_model_len}")
        slot = self.slots.add(req_id)
        host = torch.from_numpy(np.concatenate(
            [prompt, np.array([n], dtype=np.int32)])).pin_memory()
        cur = torch.cuda.current_stream(self.device)
        if n:
            self.tokens[slot, :n].copy_(host[:n], non_blocking=True)
        self.num_tokens[slot:slot + 1].copy_(host[n:], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(cur)
        self._staged.append((ev, host))
        return slot

    def propose(self, sampled_token_ids: torch.Tensor,
                valid_sampled_tokens_count: torch.Tensor | None = None):
        """Scatter the last step's sampled ids of the live requests (rows in
        slot order) into their rows and draft.  Returns (draft
        [num_active, k] int32, num_valid [num_active] int32), device."""
        n = self.num_active
        if sampled_token_ids.shape[0] != n:
            raise ValueError(f"sampled_token_ids has "
                             f"{sampled_token_ids.shape[0]} rows for {n} "
                             "active requests")
        counts = self.num_tokens[:n]
        vc = (valid_sampled_tokens_count[:n]
              if valid_sampled_tokens_count is not None else None)
        draft, num_valid, new = self.drafter.propose_with_update(
            counts, self.tokens[:n], sampled_token_ids, vc,
            max_model_len=self.max_model_len)
        counts.copy_(new)
        return draft, num_valid

    def finish_requests(self, req_ids, lengths=None,
                        harvest: bool = True) -> None:
        """Retire requests: harvest ``tokens[slot, :length]`` into the
        global memory (lengths from the engine, host ints), then refill
        their slots with the last live requests."""
        req_ids = list(req_ids)
        if not req_ids:
            return
        slots = [self.slots.slot_of[r] for r in req_ids]
        if harvest and self.drafter.global_index is not None:
            if lengths is None:
                raise ValueError("harvest needs the finished lengths")
            self.drafter.harvest_finished(slots, list(lengths), self.tokens)
        for src, dst in self.slots.remove(req_ids):
            self.tokens[dst].copy_(self.tokens[src])
            self.num_tokens[dst:dst + 1].copy_(self.num_tokens[src:src + 1])

    def poll(self) -> None:
        """Host side, once per step outside any captured region: swap in a
        finished rebuild and release staged prompt buffers."""
        self.drafter.poll()
        self._staged = [(e, t) for e, t in self._staged if not e.query()]
