"""Suffix-array construction (public API).

Mirrors suffix_gpu/suffix_array.py:15-63.  The GPU build (csrc/sa_build.hip)
is prefix doubling that stops on the device once all ranks are distinct:
a round whose unsorted groups fit a workgroup sorts them there in one
launch, a round with a larger group takes LSD radix sorts.  The suffix
array is unique, so it equals the reference's.
"""

from __future__ import annotations

import torch

from suffixgpu_amd._lib import (SA_ROUNDS_EXPECT_FINAL, SA_ROUNDS_RADIX,
                                check, lib, require_gpu, stream_of)


def sa_workspace_bytes(n: int) -> int:
    return int(lib().sfx_sa_build_workspace_size(int(n)))


# Doubling rounds enqueued between two reads of the build's done flag in
# the adaptive build.
SA_CHECK_ROUNDS = 3

# int32 words of the build's state block a host copy reads, and the
# default rounds that enqueue the radix path (round 1: on natural text its
# two-token groups exceed a workgroup)
STATE_WORDS = 16
DEFAULT_RADIX_MASK = 1 << 1


def _workspace_ok(workspace: torch.Tensor | None, text: torch.Tensor,
                  need: int) -> torch.Tensor:
    """The caller's byte workspace, or a new one when it is None or short.
    A workspace must be a contiguous uint8 tensor on the text's device:
    its numel() is the byte count and the state block is sliced by byte
    offset."""
    if workspace is not None:
        if (workspace.dtype != torch.uint8 or not workspace.is_contiguous()
                or workspace.device != text.device):
            raise ValueError("workspace must be a contiguous uint8 tensor on "
                             f"{text.device}")
        if workspace.numel() >= need:
            return workspace
    return torch.empty(max(need, 1), dtype=torch.uint8, device=text.device)


def build_suffix_array_into(text: torch.Tensor, m: int, out: torch.Tensor,
                            workspace: torch.Tensor | None = None,
                            adaptive: bool = False) -> None:
    """out[:m] = SA(text[:m]); out[m:] = m .. len(out)-1 (int32 or int64).

    adaptive=False (the default) enqueues the fixed launch sequence for
    every doubling round the length allows, with no host read: launches
    after the finishing round return at their first instruction, and the
    call can be captured in a graph or run in the background.
    adaptive=True enqueues the rounds SA_CHECK_ROUNDS at a time and reads
    the device's done flag (one synchronisation of the current stream)
    before enqueuing more, so the build stops within a few launches of the
    round that finished it (the reference's build synchronises too, on
    torch.unique in suffix_gpu/suffix_array.py)."""
    require_gpu(text, out)
    if text.dtype != torch.int32 or not text.is_contiguous():
        raise ValueError("text must be a contiguous int32 tensor")
    if out.dtype not in (torch.int32, torch.int64) or not out.is_contiguous():
        raise ValueError("out must be a contiguous int32/int64 tensor")
    if m > text.shape[0] or m > out.shape[0]:
        raise ValueError("m exceeds the text or output length")
    workspace = _workspace_ok(workspace, text, sa_workspace_bytes(m))
    if adaptive and m > 1:
        _build_adaptive(text, m, out, workspace)
        return
    check(lib().sfx_sa_build(text.data_ptr(), m, out.shape[0],
                             out.data_ptr(), int(out.dtype == torch.int64),
                             workspace.data_ptr(), workspace.numel(),
                             stream_of(text.device)), "build_suffix_array")


def _build_adaptive(text: torch.Tensor, m: int, out: torch.Tensor,
                    workspace: torch.Tensor) -> None:
    L = lib()
    st = stream_of(text.device)
    ws, nbytes = workspace.data_ptr(), workspace.numel()
    total = int(L.sfx_sa_build_rounds_total(m))
    state = state_view(workspace, m)
    flag = torch.empty(STATE_WORDS, dtype=torch.int32, pin_memory=True)
    check(L.sfx_sa_build_begin(text.data_ptr(), m, ws, nbytes, st),
          "build_suffix_array")
    first = 1
    radix_first = True  # round 1 and a resumed round enqueue the radix path
    while first <= total:
        n = min(SA_CHECK_ROUNDS, total - first + 1)
        enqueue_rounds(m, first, n, 1 << first if radix_first else 0, ws,
                       nbytes, st)
        flag.copy_(state, non_blocking=True)
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(text.device))
        done.synchronize()
        s = BuildState.of(flag.tolist())
        if s.done:
            break
        if s.stalled:
            first, radix_first = s.stalled, True
            continue
        first += n
        radix_first = False
    check(L.sfx_sa_build_finish(m, out.shape[0], out.data_ptr(),
                                int(out.dtype == torch.int64), ws, nbytes,
                                st), "build_suffix_array")


def build_suffix_array(tokens: torch.Tensor) -> torch.Tensor:
    """Suffix array (int64) of a 1-D token sequence; negatives allowed."""
    require_gpu(tokens)
    tokens = tokens.reshape(-1).to(torch.int32).contiguous()
    n = tokens.shape[0]
    out = torch.empty(n, dtype=torch.int64, device=tokens.device)
    if n == 0:
        return out
    build_suffix_array_into(tokens, n, out, adaptive=True)
    return out


def build_suffix_array_rounds(text: torch.Tensor, m: int, out: torch.Tensor,
                              workspace: torch.Tensor, rounds: int,
                              radix_mask: int = DEFAULT_RADIX_MASK,
                              final_from: int = 0) -> None:
    """The build with only its first ``rounds`` doubling rounds enqueued
    (then the output copy): the background rebuild's first chunk.  Rounds
    whose bit is set in ``radix_mask`` enqueue the radix path too; rounds
    from ``final_from`` on (0: none) are enqueued as expected to find the
    array final (see :func:`enqueue_rounds`).  The result is final iff
    :func:`build_state` says so afterwards."""
    require_gpu(text, out, workspace)
    workspace = _workspace_ok(workspace, text, sa_workspace_bytes(m))
    L = lib()
    st = stream_of(text.device)
    ws, nbytes = workspace.data_ptr(), workspace.numel()
    check(L.sfx_sa_build_begin(text.data_ptr(), m, ws, nbytes, st),
          "SA build")
    enqueue_rounds(m, 1, max(0, rounds), radix_mask, ws, nbytes, st,
                   final_from)
    check(L.sfx_sa_build_finish(m, out.shape[0], out.data_ptr(),
                                int(out.dtype == torch.int64), ws, nbytes,
                                st), "SA build")


def enqueue_rounds(m: int, first: int, count: int, radix_mask: int,
                   ws: int, nbytes: int, stream, final_from: int = 0) -> None:
    """Doubling rounds first .. first+count-1 on ``stream``: a round r with
    bit r of ``radix_mask`` set enqueues the radix path too, the others
    only the local launch (a round that needs the radix path then stalls
    the build, see :class:`BuildState`).  Rounds r >= ``final_from`` (when
    it is positive) are flagged as expected to find the array final, as a
    rebuild's margin rounds are: their launches check the build state
    before reading their tiles.  The flag changes no result."""
    L = lib()

    def flags(r: int) -> int:
        f = SA_ROUNDS_RADIX if (radix_mask >> r) & 1 else 0
        if 0 < final_from <= r:
            f |= SA_ROUNDS_EXPECT_FINAL
        return f

    r, end = first, first + count
    while r < end:
        f = flags(r)
        r2 = r + 1
        while r2 < end and flags(r2) == f:
            r2 += 1
        check(L.sfx_sa_build_rounds(m, r, r2 - r, f, ws, nbytes, stream),
              "SA build")
        r = r2


def state_view(workspace: torch.Tensor, m: int) -> torch.Tensor:
    """The device words of a build's state block (a view of the byte
    workspace)."""
    off = int(lib().sfx_sa_build_flag_offset(m))
    return workspace[off:off + 4 * STATE_WORDS].view(torch.int32)


class BuildState:
    """A build's state words: done (the array is final), found_none (the
    round that found no unsorted group), stalled (the round that needs the
    radix path it was not given, 0 for none) and radix_mask (bit r for each
    round that took the radix path; bit 0 is the token round)."""

    def __init__(self, done: bool, found_none: int, stalled: int,
                 radix_mask: int):
        self.done = done
        self.found_none = found_none
        self.stalled = stalled
        self.radix_mask = radix_mask

    @classmethod
    def of(cls, words: list[int]) -> "BuildState":
        return cls(bool(words[0]), int(words[2]), int(words[7]),
                   int(words[8]) & 0xffffffff)

    @property
    def needed(self) -> int:
        """Doubling rounds the array needed (-1 while not final)."""
        return max(self.found_none - 1, 0) if self.done else -1


def read_build_state(workspace: torch.Tensor, m: int) -> BuildState:
    """The state of a build (synchronises the current stream)."""
    if m <= 1:
        return BuildState(True, 1, 0, 0)
    return BuildState.of(state_view(workspace, m).cpu().tolist())


def build_state(workspace: torch.Tensor, m: int) -> tuple[bool, int]:
    """(final, rounds the array needed) from a build's workspace; reads the
    device (synchronises the current stream)."""
    s = read_build_state(workspace, m)
    return s.done, (s.needed if m > 1 else 0)
