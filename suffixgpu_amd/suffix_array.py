"""Suffix-array construction (public API).

Mirrors suffix_gpu/suffix_array.py:15-63.  The GPU build (csrc/sa_build.hip)
is prefix doubling over LSD radix sorts that stops on the device once all
ranks are distinct; the suffix array is unique, so it equals the
reference's.
"""

from __future__ import annotations

import torch

from suffixgpu_amd._lib import check, lib, require_gpu, stream_of


def sa_workspace_bytes(n: int) -> int:
    return int(lib().sfx_sa_build_workspace_size(int(n)))


# Doubling rounds enqueued between two reads of the build's done flag in
# the adaptive build.
SA_CHECK_ROUNDS = 3


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
    off = int(L.sfx_sa_build_flag_offset(m))
    state = workspace[off:off + 16].view(torch.int32)
    flag = torch.empty(4, dtype=torch.int32, pin_memory=True)
    check(L.sfx_sa_build_begin(text.data_ptr(), m, ws, nbytes, st),
          "build_suffix_array")
    first = 1
    while first <= total:
        n = min(SA_CHECK_ROUNDS, total - first + 1)
        check(L.sfx_sa_build_rounds(m, first, n, ws, nbytes, st),
              "build_suffix_array")
        first += n
        flag.copy_(state, non_blocking=True)
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(text.device))
        done.synchronize()
        if int(flag[0]):
            break
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
                              workspace: torch.Tensor, rounds: int) -> None:
    """The build with only its first ``rounds`` doubling rounds enqueued
    (then the output copy): the background rebuild's first chunk.  The
    result is final iff :func:`build_is_final` says so afterwards."""
    require_gpu(text, out, workspace)
    workspace = _workspace_ok(workspace, text, sa_workspace_bytes(m))
    L = lib()
    st = stream_of(text.device)
    check(L.sfx_sa_build_begin(text.data_ptr(), m, workspace.data_ptr(),
                               workspace.numel(), st), "SA build")
    check(L.sfx_sa_build_rounds(m, 1, max(0, rounds), workspace.data_ptr(),
                                workspace.numel(), st), "SA build")
    check(L.sfx_sa_build_finish(m, out.shape[0], out.data_ptr(),
                                int(out.dtype == torch.int64),
                                workspace.data_ptr(), workspace.numel(), st),
          "SA build")


def build_state(workspace: torch.Tensor, m: int) -> tuple[bool, int]:
    """(final, rounds the array needed) from a build's workspace; reads the
    device (synchronises the current stream)."""
    if m <= 1:
        return True, 0
    off = int(lib().sfx_sa_build_flag_offset(m))
    st = workspace[off:off + 16].view(torch.int32).cpu().tolist()
    # st[2]: the doubling round that found no unsorted group left
    return bool(st[0]), (max(int(st[2]) - 1, 0) if st[0] else -1)
