"""Frequency-ranked chain expansion (public helper API).

Mirrors suffix_gpu/expand.py:16-147.  Both functions run the wave-level
majority-vote kernel of libsuffixgpu_amd.so: per depth the most voted
continuation token wins (ties to the smallest id), the chain probability is
multiplied by votes / (active + alpha) in fp32, and the chain stops once it
falls below ``min_token_prob``.
"""

from __future__ import annotations

import torch

from suffixgpu_amd import kernels
from suffixgpu_amd._lib import require_gpu


def _majority_token(values: torch.Tensor, active: torch.Tensor,
                    sentinel: int, weights: torch.Tensor | None = None,
                    ) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row majority token among active entries (expand.py:16-56).

    Returns (token [B], count [B]); rows without an active entry get
    (sentinel, 0).  Runs as a one-depth chain expansion.
    """
    require_gpu(values, active, weights)
    b, r = values.shape
    if (values[active] == -1).any().item() if values.numel() else False:
        raise ValueError("_majority_token: -1 is reserved for inactive slots")
    cont = torch.where(active, values.to(torch.int32),
                       torch.full_like(values, -1, dtype=torch.int32))
    occ = torch.full((b,), r, dtype=torch.int64, device=values.device)
    cap = torch.ones(b, dtype=torch.int64, device=values.device)
    chain, nv, _, score = kernels.expand_chain(
        cont.unsqueeze(2).contiguous(), occ, 1, 0.0, cap, weights=weights)
    act_n = active.sum(dim=1)
    if weights is None:
        count = torch.where(nv > 0,
                            torch.round(score * act_n.clamp(min=1)).to(
                                torch.int64),
                            torch.zeros_like(nv))
    else:
        w = torch.where(active, weights.to(torch.float32),
                        torch.zeros_like(weights, dtype=torch.float32))
        eq = cont == chain[:, :1]
        count = torch.where(nv > 0, (w * eq).sum(dim=1),
                            torch.zeros(b, device=values.device))
    token = torch.where(nv > 0, chain[:, 0].to(values.dtype),
                        torch.full_like(chain[:, 0], sentinel).to(
                            values.dtype))
    return token, count


def expand_chain(cont: torch.Tensor, num_occ: torch.Tensor, k: int,
                 sentinel: int = -1, min_token_prob: float = 0.0,
                 cap: torch.Tensor | None = None,
                 weights: torch.Tensor | None = None, alpha: float = 0.0,
                 ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                            torch.Tensor]:
    """Majority-vote chain expansion with fused scoring (expand.py:59-147).

    Returns (chain [B, k], num_valid [B] i64, num_emit [B] i64, score [B]
    f32); the chain is int32 for the drafter's sentinel -1 and of cont's
    dtype otherwise, as the reference's two paths return.

    The kernel marks inactive continuation slots with -1.  Another
    sentinel s (any int32 value; -1 may then be a real token) is moved
    onto -1 by an order-preserving bijection of the int32 values without
    s onto those without -1: for s < -1 the values in (s, -1] move down
    by one, for s > -1 those in [-1, s) move up by one, and s becomes -1.
    Votes compare tokens for equality and break ties by the smallest
    token, both of which the bijection keeps, so the chain maps back
    exactly (slots the kernel leaves at -1 become s).
    """
    require_gpu(cont, num_occ, cap, weights)
    b = cont.shape[0]
    if cap is None:
        cap = torch.full((b,), k, dtype=torch.int64, device=cont.device)
    if sentinel == -1:
        return kernels.expand_chain(cont, num_occ, k, min_token_prob, cap,
                                    weights=weights, alpha=alpha)
    s = int(sentinel)
    if not -2 ** 31 <= s < 2 ** 31:
        raise ValueError("expand_chain: the sentinel must be an int32 value")
    if cont.dtype not in (torch.int32, torch.int64):
        raise TypeError("expand_chain: integer continuation tokens")
    c = cont.to(torch.int64)
    if s < -1:
        mapped = torch.where((c > s) & (c <= -1), c - 1, c)
    else:
        mapped = torch.where((c >= -1) & (c < s), c + 1, c)
    mapped = torch.where(c == s, torch.full_like(c, -1), mapped)
    chain, nv, ne, score = kernels.expand_chain(
        mapped.to(torch.int32).contiguous(), num_occ, k, min_token_prob,
        cap, weights=weights, alpha=alpha)
    ch = chain.to(torch.int64)
    if s < -1:
        back = torch.where((ch >= s) & (ch <= -2), ch + 1, ch)
    else:
        back = torch.where((ch >= 0) & (ch <= s), ch - 1, ch)
    back = torch.where(ch == -1, torch.full_like(ch, s), back)
    return back.to(cont.dtype), nv, ne, score
