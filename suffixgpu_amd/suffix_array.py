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


def build_suffix_array_into(text: torch.Tensor, m: int, out: torch.Tensor,
                            workspace: torch.Tensor | None = None) -> None:
    """out[:m] = SA(text[:m]); out[m:] = m .. len(out)-1 (int32 or int64)."""
    require_gpu(text, out)
    if text.dtype != torch.int32 or not text.is_contiguous():
        raise ValueError("text must be a contiguous int32 tensor")
    if out.dtype not in (torch.int32, torch.int64) or not out.is_contiguous():
        raise ValueError("out must be a contiguous int32/int64 tensor")
    if m > text.shape[0] or m > out.shape[0]:
        raise ValueError("m exceeds the text or output length")
    need = sa_workspace_bytes(m)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8,
                                device=text.device)
    check(lib().sfx_sa_build(text.data_ptr(), m, out.shape[0],
                             out.data_ptr(), int(out.dtype == torch.int64),
                             workspace.data_ptr(), workspace.numel(),
                             stream_of(text.device)), "build_suffix_array")


def build_suffix_array(tokens: torch.Tensor) -> torch.Tensor:
    """Suffix array (int64) of a 1-D token sequence; negatives allowed."""
    require_gpu(tokens)
    tokens = tokens.reshape(-1).to(torch.int32).contiguous()
    n = tokens.shape[0]
    out = torch.empty(n, dtype=torch.int64, device=tokens.device)
    if n == 0:
        return out
    build_suffix_array_into(tokens, n, out)
    return out
