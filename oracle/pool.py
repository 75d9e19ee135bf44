"""The oracle's drafter step spread over worker processes, row by row.

Test infrastructure, like the rest of oracle/: only the benchmark's CPU
baseline uses it, to time the reference's CPU semantics with every host
core instead of one thread.  Each row of a step is independent in the
reference (suffix_gpu/proposer.py:216-327: the local match, the global
query, the expansion and the selection all work per row, and update_state
writes only its own row), so splitting the batch into contiguous row
slices and concatenating the slices' outputs gives exactly the
single-process result; ``test_oracle_kats.py`` checks that.

Workers are started with the "spawn" method: each is a fresh interpreter
that imports numpy and oracle/ only and never touches a GPU.  The global
index state (corpus, suffix array, delta) is sent once to every worker at
start-up.
"""

from __future__ import annotations

import multiprocessing as mp
import os

import numpy as np

_W = None  # the worker's DrafterOracle


def _init(kw: dict, index: dict | None) -> None:
    global _W
    from oracle.drafter import DrafterOracle
    _W = DrafterOracle(**kw)
    if index is not None:
        g = _W.global_index
        g.corpus[:] = index["corpus"]
        g.sa[:] = index["sa"]
        g.delta[:index["delta"].shape[0]] = index["delta"]
        g.active_len = int(index["active_len"])
        g.delta_len = int(index["delta_len"])


def _step(args):
    kind, nt, tok, extra = args
    if kind == "update":
        draft, nv, new = _W.propose_with_update(nt, tok, extra)
        return draft, nv, new, tok
    draft, nv = _W.propose(nt, tok, extra)
    return draft, nv, None, tok


def default_workers() -> int:
    """The host cores this process may run on, at most 16 (the CPU share
    of one GPU on the measurement hosts)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


class RowPool:
    """DrafterOracle(**kw) evaluated over row slices in `workers`
    processes.  ``index`` (optional) is the global index state to load into
    every worker: corpus, sa, delta arrays and active_len / delta_len."""

    def __init__(self, kw: dict, index: dict | None = None,
                 workers: int | None = None):
        self.workers = workers or default_workers()
        ctx = mp.get_context("spawn")
        self._pool = ctx.Pool(self.workers, initializer=_init,
                              initargs=(kw, index))

    def _run(self, kind, num_tokens, tok, extra):
        b = tok.shape[0]
        cuts = np.linspace(0, b, min(self.workers, b) + 1).astype(int)
        parts = [(kind, num_tokens[a:z], tok[a:z].copy(),
                  None if extra is None else extra[a:z])
                 for a, z in zip(cuts[:-1], cuts[1:]) if z > a]
        res = self._pool.map(_step, parts)
        for (a, z), r in zip([(a, z) for a, z in zip(cuts[:-1], cuts[1:])
                              if z > a], res):
            tok[a:z] = r[3]
        draft = np.concatenate([r[0] for r in res])
        nv = np.concatenate([r[1] for r in res])
        new = (np.concatenate([r[2] for r in res]) if kind == "update"
               else None)
        return draft, nv, new

    def propose_with_update(self, num_tokens, tok, sampled):
        """As DrafterOracle.propose_with_update (tok updated in place)."""
        return self._run("update", num_tokens, tok, sampled)

    def propose(self, num_tokens, tok, mask=None):
        draft, nv, _ = self._run("propose", num_tokens, tok, mask)
        return draft, nv

    def close(self) -> None:
        self._pool.close()
        self._pool.join()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
