"""Write golden input/output vectors from the reference implementation.

Run in the build container only (it imports zip95297/SuffixGPU from
/root/reference, which never travels to a GPU host):

    python tests/golden/make_golden.py

Only functions that no known-answer test, brute-force definition or closed
form pins are recorded here:

* whole-drafter compositions (propose / propose_with_update, local-only and
  local+global) -- they depend on torch.topk tie order, torch's fp32 scalar
  casts in _spec_cap / select_local_best and the hierarchical selection;
* the GlobalIndex host state machine over scripted append / rebuild /
  eviction / in-flight sequences, and harvest_finished / ingest_active
  under rebuilds that finish only at the script's own polls (the schedule
  of device-side ingest);
* expand_chain with vote smoothing (alpha) and with per-occurrence weights.

The reference runs on CPU tensors, i.e. its pure-torch path (the Triton
kernels are gated on CUDA tensors).  Each fixture is an .npz of inputs and
outputs; the inputs come from suffixgpu_amd.synth seeds and are stored too.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))
sys.path.insert(0, "/root/reference")

from suffix_gpu.expand import expand_chain  # noqa: E402
from suffix_gpu.proposer import SuffixGPUDrafter  # noqa: E402

from suffixgpu_amd import synth  # noqa: E402

torch.set_num_threads(min(8, os.cpu_count() or 1))


def t32(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.int32)


def np_(t):
    return t.detach().cpu().numpy().copy()


def save(name: str, **arrays) -> None:
    path = HERE / f"{name}.npz"
    np.savez_compressed(path, **arrays)
    print(f"wrote {path.name}: " + ", ".join(
        f"{k}{tuple(v.shape)}" for k, v in arrays.items()))


def drafter_kwargs(**kw):
    base = dict(k=16, device="cpu", max_pattern_len=32, max_occurrences=128)
    base.update(kw)
    return base


def local_cases() -> None:
    # Uniform vocab, one backoff level, propose only.
    w = synth.local_uniform(seed=1)
    kw = drafter_kwargs(num_backoff=1)
    d = SuffixGPUDrafter(**kw)
    draft, nv = d.propose(t32(w.num_tokens), t32(w.tokens))
    cand, cont, occ = d.local_kernel.gather_candidates(
        t32(w.num_tokens), t32(w.tokens), torch.ones(8, dtype=torch.bool))
    save("local_uniform", tokens=w.tokens, num_tokens=w.num_tokens,
         draft=np_(draft), num_valid=np_(nv), cand=np_(cand), cont=np_(cont),
         occ=np_(occ))

    # Zipf rows, full backoff, adaptive cap and min prob, update + propose.
    w = synth.local_zipf(seed=2, b=12, s=4096, lo=1024)
    kw = drafter_kwargs(num_backoff=8, max_spec_factor=2.0,
                        min_token_prob=0.1)
    d = SuffixGPUDrafter(**kw)
    tok = t32(w.tokens)
    draft, nv, new = d.propose_with_update(t32(w.num_tokens), tok,
                                           t32(w.sampled))
    mask = torch.ones(12, dtype=torch.bool)
    fw = d.local_kernel(new, tok, mask)
    save("local_zipf_update", tokens=w.tokens, num_tokens=w.num_tokens,
         sampled=w.sampled, tokens_after=np_(tok), draft=np_(draft),
         num_valid=np_(nv), new_counts=np_(new), fw_draft=np_(fw[0]),
         fw_nv=np_(fw[1]), fw_len=np_(fw[2]), fw_occ=np_(fw[3]),
         fw_score=np_(fw[4]))

    # Tiny vocab: dense ties everywhere; non-fp32-exact factor/offset,
    # smoothing and a mask.
    rng = np.random.default_rng(11)
    b, s = 16, 384
    tok_np = rng.integers(0, 4, size=(b, s)).astype(np.int32)
    nt = rng.integers(2, s + 1, size=b).astype(np.int32)
    nt[0], nt[1] = 0, 1
    mask_np = rng.random(b) < 0.8
    kw = dict(k=8, device="cpu", max_pattern_len=12, max_occurrences=16,
              num_backoff=6, max_spec_factor=0.7, max_spec_offset=0.3,
              min_token_prob=0.05, vote_smoothing_alpha=0.5)
    d = SuffixGPUDrafter(**kw)
    draft, nv = d.propose(t32(nt), t32(tok_np), torch.from_numpy(mask_np))
    fw = d.local_kernel(t32(nt), t32(tok_np), torch.from_numpy(mask_np))
    save("local_ties", tokens=tok_np, num_tokens=nt, mask=mask_np,
         draft=np_(draft), num_valid=np_(nv), fw_len=np_(fw[2]),
         fw_occ=np_(fw[3]), fw_score=np_(fw[4]))


def index_state(gi) -> dict:
    return dict(active_len=np.array(gi.active_len),
                delta_len=np.array(gi.delta_len),
                active_doc_lens=np.array(list(gi.active_doc_lens), np.int64),
                delta_doc_lens=np.array(gi.delta_doc_lens, np.int64),
                corpus=np_(gi.corpus), sa=np_(gi.sa),
                delta=np_(gi.delta)[:gi.delta_len])


def global_cases() -> None:
    # Template corpus at small capacity: rebuilds, evictions and delta
    # queries through the public drafter API.
    tc = synth.TemplateCorpus(seed=3, n_templates=16)
    docs = [tc.sequence(lo=96, hi=400) for _ in range(48)]
    held = [tc.sequence(lo=160, hi=400) for _ in range(10)]
    kw = drafter_kwargs(num_backoff=8, max_spec_factor=2.0,
                        min_token_prob=0.1, enable_global=True,
                        global_capacity=1 << 13, delta_capacity=1 << 10,
                        rebuild_threshold=700)
    d = SuffixGPUDrafter(**kw)
    b, s, t = len(held), 512, 17
    rows = np.zeros((b, s), np.int32)
    nt = np.zeros(b, np.int32)
    sampled = np.full((b, t), -1, np.int32)
    rng = np.random.default_rng(5)
    for i, seq in enumerate(held):
        rows[i, :min(len(seq), s)] = seq[:s]
        n = int(rng.integers(32, min(len(seq), s) - t))
        nt[i] = n
        acc = int(rng.integers(0, 5)) + 1
        sampled[i, :acc] = seq[n:n + acc]
    sampled[3, :] = -1
    outs = {}
    lens = []
    for step, lo in enumerate(range(0, len(docs), 8)):
        chunk = docs[lo:lo + 8]
        lens.append(len(chunk))
        d.harvest_rows([torch.from_numpy(x) for x in chunk],
                       [len(x) for x in chunk])
        d.poll()
        tok = t32(rows)
        draft, nv, new = d.propose_with_update(t32(nt), tok, t32(sampled))
        outs[f"draft_{step}"] = np_(draft)
        outs[f"nv_{step}"] = np_(nv)
        for key, v in index_state(d.global_index).items():
            outs[f"{key}_{step}"] = v
    flat = np.concatenate(docs)
    offs = np.cumsum([0] + [len(x) for x in docs])
    save("global_drafter", doc_flat=flat, doc_offs=offs, rows=rows,
         num_tokens=nt, sampled=sampled, steps=np.array(len(lens)), **outs)

    # Tiny vocab global: ties in SA intervals, strided sampling (R small),
    # delta vs SA merge, and query()/draft() outputs.
    rng = np.random.default_rng(17)
    kw = dict(k=6, device="cpu", max_pattern_len=10, max_occurrences=8,
              num_backoff=5, enable_global=True, global_capacity=2048,
              delta_capacity=300, rebuild_threshold=200,
              min_token_prob=0.0, max_spec_factor=None)
    d = SuffixGPUDrafter(**kw)
    docs = [rng.integers(0, 5, size=int(rng.integers(5, 90))).astype(np.int32)
            for _ in range(30)]
    d.harvest_rows([torch.from_numpy(x) for x in docs[:20]],
                   [len(x) for x in docs[:20]])
    d.harvest_rows([torch.from_numpy(x) for x in docs[20:]],
                   [len(x) for x in docs[20:]])
    gi = d.global_index
    qb = 24
    q = rng.integers(0, 5, size=(qb, 10)).astype(np.int32)
    ql = rng.integers(0, 11, size=qb).astype(np.int64)
    caps = torch.tensor([10, 5, 3, 2], dtype=torch.int64)
    ml, cont, occ = gi._query_backoff(t32(q), torch.from_numpy(ql), 10, caps)
    dl, dp, dc = gi._delta_match_backoff(t32(q), torch.from_numpy(ql), 10,
                                         caps)
    dr = gi.draft(t32(q), torch.from_numpy(ql), 10, 6, min_token_prob=0.05,
                  max_spec_factor=1.5, max_spec_offset=1.0, caps=caps)
    rows = np.zeros((qb, 64), np.int32)
    rows[:, :10] = q
    draft, nv = d.propose(torch.from_numpy(ql.astype(np.int32)), t32(rows))
    flat = np.concatenate(docs)
    offs = np.cumsum([0] + [len(x) for x in docs])
    save("global_ties", doc_flat=flat, doc_offs=offs, query=q, query_len=ql,
         caps=np_(caps), q_len=np_(ml), q_cont=np_(cont), q_occ=np_(occ),
         d_len=np_(dl), d_pos=np_(dp), d_cnt=np_(dc), dr_chain=np_(dr[0]),
         dr_emit=np_(dr[1]), dr_len=np_(dr[2]), dr_occ=np_(dr[3]),
         dr_score=np_(dr[4]), rows=rows, draft=np_(draft), num_valid=np_(nv),
         **index_state(gi))


class _NeverDone:
    def query(self) -> bool:
        return False


def trace_cases() -> None:
    """Scripted GlobalIndex write-path trace (evict / drop / compact)."""
    from suffix_gpu.global_index import GlobalIndex
    rng = np.random.default_rng(23)
    gi = GlobalIndex(capacity=96, delta_capacity=40, k=4, max_occurrences=8,
                     rebuild_threshold=25, device="cpu")
    ops = []
    outs = {}
    docs_flat = []
    for step in range(40):
        kind = "append"
        if step in (12, 13, 14, 27):
            kind = "inflight_append"
        n_docs = int(rng.integers(1, 4))
        docs = [rng.integers(0, 7, size=int(rng.integers(1, 20))).astype(
            np.int32) for _ in range(n_docs)]
        if step == 20:
            docs.append(rng.integers(0, 7, size=55).astype(np.int32))
        if kind == "inflight_append" and gi._rebuild_event is None:
            gi._rebuild_event = _NeverDone()
            gi._pending = (gi.active_len, gi.active_doc_lens)
        gi.append_documents([torch.from_numpy(x) for x in docs])
        if step in (14, 27):
            gi._rebuild_event = None
            gi._pending = None
        ops.append([step, len(docs), int(kind == "inflight_append")])
        docs_flat.append(np.concatenate(
            [np.array([len(x)] + list(x), np.int32) for x in docs]))
        for key, v in index_state(gi).items():
            outs[f"{key}_{step}"] = v
    save("index_trace", ops=np.array(ops, np.int64),
         docs_blob=np.concatenate(docs_flat),
         docs_blob_offs=np.cumsum([0] + [len(x) for x in docs_flat]), **outs)


class _UserPollEvent:
    """A rebuild event that is complete only inside the script's own polls
    that it marks done: append_documents' polls (global_index.py:111,140)
    find the rebuild still running, as a device-side ingest does."""

    def __init__(self):
        self.in_user_poll = False
        self.done = False

    def query(self) -> bool:
        return self.in_user_poll and self.done


def _defer_swaps(gi, event: _UserPollEvent) -> None:
    """On a CPU index the reference builds and swaps inside _launch_rebuild
    (global_index.py:213-215); keep its build (the staging buffers are not
    written again before the swap) and defer the swap to the poll where
    `event` completes, as a rebuild on a side stream would."""
    launch, finish = gi._launch_rebuild, gi._finish_swap
    state = {"launching": False}

    def deferred_launch():
        state["launching"] = True
        try:
            launch()
        finally:
            state["launching"] = False

    def deferred_finish(n_new, lens):
        if state["launching"]:
            gi._pending = (n_new, lens)
            gi._rebuild_event = event
        else:
            finish(n_new, lens)

    gi._launch_rebuild = deferred_launch
    gi._finish_swap = deferred_finish


def ingest_cases() -> None:
    """harvest_finished (row indices as Python indices, lengths <= 0 and
    past the row, documents longer than the delta) and ingest_active
    (chunks, overlap, final) on a small index whose rebuilds finish only
    at the script's polls, some of which find them still running."""
    rng = np.random.default_rng(41)
    kw = dict(k=4, device="cpu", max_pattern_len=8, max_occurrences=8,
              num_backoff=3, enable_global=True, global_capacity=200,
              delta_capacity=64, rebuild_threshold=32)
    d = SuffixGPUDrafter(**kw)
    gi = d.global_index
    ev = _UserPollEvent()
    _defer_swaps(gi, ev)
    rows, seq_a = 6, 96
    resp = {}  # slot -> (response row, current length)
    outs = {}
    kinds = []
    for i in range(90):
        kind = 2 if i % 4 == 3 else int(rng.random() < 0.5)
        kinds.append(kind)
        if kind == 0:
            seq = int(rng.choice([24, 80]))
            tok = rng.integers(0, 6, size=(rows, seq)).astype(np.int32)
            n = int(rng.integers(1, 5))
            idx = rng.integers(-rows, rows, size=n).astype(np.int64)
            lens = rng.integers(-3, seq + 10, size=n).astype(np.int64)
            d.harvest_finished([int(x) for x in idx], [int(x) for x in lens],
                               torch.from_numpy(tok))
            outs.update({f"tok_{i}": tok, f"idx_{i}": idx, f"len_{i}": lens})
        elif kind == 1:
            n = int(rng.integers(1, 4))
            keys = rng.choice(5, size=n, replace=False).astype(np.int64)
            final = bool(rng.random() < 0.2)
            chunk = int(rng.choice([16, 32]))
            tok = np.zeros((n, seq_a), np.int32)
            lens = np.zeros(n, np.int64)
            for j, key in enumerate(keys):
                row, ln = resp.get(int(key), (None, 0))
                if row is None:
                    row = rng.integers(0, 6, size=seq_a).astype(np.int32)
                ln = min(seq_a + 4, ln + int(rng.integers(0, 40)))
                resp[int(key)] = (row, ln)
                tok[j], lens[j] = row, ln
            d.ingest_active([int(x) for x in keys],
                            [torch.from_numpy(r) for r in tok],
                            [int(x) for x in lens], final=final, chunk=chunk)
            if final:
                for key in keys:
                    resp.pop(int(key), None)
            outs.update({f"tok_{i}": tok, f"keys_{i}": keys,
                         f"len_{i}": lens, f"final_{i}": np.array(final),
                         f"chunk_{i}": np.array(chunk)})
        else:
            done = bool(rng.random() < 0.75)
            ev.done, ev.in_user_poll = done, True
            d.poll()
            ev.in_user_poll = False
            outs[f"done_{i}"] = np.array(done)
        running = gi._rebuild_event is not None
        for key, v in index_state(gi).items():
            outs[f"{key}_{i}"] = v
        outs[f"in_flight_{i}"] = np.array(running)
        outs[f"pend_n_new_{i}"] = np.array(gi._pending[0] if running else 0)
        outs[f"pend_lens_{i}"] = np.array(
            list(gi._pending[1]) if running else [], np.int64)
        outs[f"staging_{i}"] = np_(gi.staging_corpus)
        ing = sorted(d._ingested.items())
        outs[f"ing_keys_{i}"] = np.array([k for k, _ in ing], np.int64)
        outs[f"ing_vals_{i}"] = np.array([v for _, v in ing], np.int64)
    save("ingest_trace", kinds=np.array(kinds, np.int64), **outs)


def expand_cases() -> None:
    rng = torch.Generator().manual_seed(99)
    outs = {}
    for i, (alpha, r, k) in enumerate([(0.5, 32, 12), (1.0, 32, 12),
                                       (2.0, 64, 16), (0.25, 128, 16)]):
        b = 21
        cont = torch.randint(0, 9, (b, r, k), dtype=torch.int32, generator=rng)
        tail = torch.randint(0, k + 1, (b, r), generator=rng)
        cont = torch.where(torch.arange(k).view(1, 1, k) < tail.unsqueeze(2),
                           cont, -1)
        occ = torch.randint(0, r + 1, (b,), dtype=torch.int64, generator=rng)
        cap = torch.randint(-1, k + 1, (b,), dtype=torch.int64, generator=rng)
        ch, nv, ne, sc = expand_chain(cont, occ, k, min_token_prob=0.05,
                                      cap=cap, alpha=alpha)
        w = torch.rand(b, r, generator=rng) + 0.05
        chw, nvw, new, scw = expand_chain(cont, occ, k, min_token_prob=0.05,
                                          cap=cap, weights=w)
        outs.update({f"cont_{i}": np_(cont), f"occ_{i}": np_(occ),
                     f"cap_{i}": np_(cap), f"alpha_{i}": np.array(alpha),
                     f"chain_{i}": np_(ch), f"nv_{i}": np_(nv),
                     f"emit_{i}": np_(ne), f"score_{i}": np_(sc),
                     f"w_{i}": np_(w), f"wchain_{i}": np_(chw),
                     f"wnv_{i}": np_(nvw), f"wemit_{i}": np_(new),
                     f"wscore_{i}": np_(scw)})
    save("expand_alpha_weights", n=np.array(4), **outs)


if __name__ == "__main__":
    local_cases()
    global_cases()
    trace_cases()
    ingest_cases()
    expand_cases()
