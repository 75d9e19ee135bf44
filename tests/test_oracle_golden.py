"""The oracle reproduces vectors written by the reference implementation.

tests/golden/make_golden.py ran zip95297/SuffixGPU's own pure-torch path on
these inputs; every draft, count, occurrence list, suffix array and index
state must match bit for bit (weighted-vote scores within the reference's
own rtol=1e-4, since fp32 sum order of weights is not fixed by torch).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.drafter import DrafterOracle
from oracle.expand import expand_chain
from oracle.global_index import GlobalIndexOracle
from tests.conftest import golden


def test_local_uniform_propose_and_candidates():
    z = golden("local_uniform")
    d = DrafterOracle(k=16, max_pattern_len=32, max_occurrences=128,
                      num_backoff=1)
    draft, nv = d.propose(z["num_tokens"], z["tokens"].copy())
    np.testing.assert_array_equal(draft, z["draft"])
    np.testing.assert_array_equal(nv, z["num_valid"])
    cand, cont, occ = d.local_kernel.gather_candidates(
        z["num_tokens"], z["tokens"], np.ones(8, bool))
    np.testing.assert_array_equal(cand, z["cand"])
    np.testing.assert_array_equal(cont, z["cont"])
    np.testing.assert_array_equal(occ, z["occ"])


def test_local_zipf_update_and_forward():
    z = golden("local_zipf_update")
    d = DrafterOracle(k=16, max_pattern_len=32, max_occurrences=128,
                      num_backoff=8, max_spec_factor=2.0, min_token_prob=0.1)
    tok = z["tokens"].copy()
    draft, nv, new = d.propose_with_update(z["num_tokens"], tok, z["sampled"])
    np.testing.assert_array_equal(tok, z["tokens_after"])
    np.testing.assert_array_equal(new, z["new_counts"])
    np.testing.assert_array_equal(draft, z["draft"])
    np.testing.assert_array_equal(nv, z["num_valid"])
    fw = d.local_kernel.forward(new, tok, np.ones(tok.shape[0], bool))
    for got, key in zip(fw, ["fw_draft", "fw_nv", "fw_len", "fw_occ",
                             "fw_score"]):
        np.testing.assert_array_equal(got, z[key], err_msg=key)


def test_local_ties_mask_and_scalar_casts():
    z = golden("local_ties")
    d = DrafterOracle(k=8, max_pattern_len=12, max_occurrences=16,
                      num_backoff=6, max_spec_factor=0.7,
                      max_spec_offset=0.3, min_token_prob=0.05,
                      vote_smoothing_alpha=0.5)
    draft, nv = d.propose(z["num_tokens"], z["tokens"].copy(), z["mask"])
    np.testing.assert_array_equal(draft, z["draft"])
    np.testing.assert_array_equal(nv, z["num_valid"])
    fw = d.local_kernel.forward(z["num_tokens"], z["tokens"], z["mask"])
    np.testing.assert_array_equal(fw[2], z["fw_len"])
    np.testing.assert_array_equal(fw[3], z["fw_occ"])
    np.testing.assert_array_equal(fw[4], z["fw_score"])


def _docs(z):
    offs = z["doc_offs"]
    return [z["doc_flat"][a:b] for a, b in zip(offs[:-1], offs[1:])]


def _state_equal(gi, z, suffix=""):
    assert gi.active_len == int(z["active_len" + suffix])
    assert gi.delta_len == int(z["delta_len" + suffix])
    np.testing.assert_array_equal(
        np.array(list(gi.active_doc_lens), np.int64),
        z["active_doc_lens" + suffix])
    np.testing.assert_array_equal(np.array(gi.delta_doc_lens, np.int64),
                                  z["delta_doc_lens" + suffix])
    np.testing.assert_array_equal(gi.corpus, z["corpus" + suffix])
    np.testing.assert_array_equal(gi.sa, z["sa" + suffix])
    np.testing.assert_array_equal(gi.delta[:gi.delta_len],
                                  z["delta" + suffix])


def test_global_drafter_sequence():
    z = golden("global_drafter")
    docs = _docs(z)
    d = DrafterOracle(k=16, max_pattern_len=32, max_occurrences=128,
                      num_backoff=8, max_spec_factor=2.0, min_token_prob=0.1,
                      enable_global=True, global_capacity=1 << 13,
                      delta_capacity=1 << 10, rebuild_threshold=700)
    for step, lo in enumerate(range(0, len(docs), 8)):
        chunk = docs[lo:lo + 8]
        d.harvest_rows(chunk, [len(x) for x in chunk])
        d.poll()
        tok = z["rows"].copy()
        draft, nv, _ = d.propose_with_update(z["num_tokens"], tok,
                                             z["sampled"])
        np.testing.assert_array_equal(draft, z[f"draft_{step}"])
        np.testing.assert_array_equal(nv, z[f"nv_{step}"])
        _state_equal(d.global_index, z, f"_{step}")
    assert int(z["steps"]) == step + 1


def test_global_ties_query_delta_draft():
    z = golden("global_ties")
    docs = _docs(z)
    d = DrafterOracle(k=6, max_pattern_len=10, max_occurrences=8,
                      num_backoff=5, enable_global=True,
                      global_capacity=2048, delta_capacity=300,
                      rebuild_threshold=200)
    d.harvest_rows(docs[:20], [len(x) for x in docs[:20]])
    d.harvest_rows(docs[20:], [len(x) for x in docs[20:]])
    gi = d.global_index
    _state_equal(gi, z)
    q, ql, caps = z["query"], z["query_len"], z["caps"]
    ml, cont, occ = gi._query_backoff(q, ql, 10, caps)
    np.testing.assert_array_equal(ml, z["q_len"])
    np.testing.assert_array_equal(cont, z["q_cont"])
    np.testing.assert_array_equal(occ, z["q_occ"])
    dl, dp, dc = gi._delta_match_backoff(q, ql, 10, caps)
    np.testing.assert_array_equal(dl, z["d_len"])
    np.testing.assert_array_equal(dp, z["d_pos"])
    np.testing.assert_array_equal(dc, z["d_cnt"])
    dr = gi.draft(q, ql, 10, 6, min_token_prob=0.05, max_spec_factor=1.5,
                  max_spec_offset=1.0, caps=caps)
    for got, key in zip(dr, ["dr_chain", "dr_emit", "dr_len", "dr_occ",
                             "dr_score"]):
        np.testing.assert_array_equal(got, z[key], err_msg=key)
    draft, nv = d.propose(ql.astype(np.int32), z["rows"].copy())
    np.testing.assert_array_equal(draft, z["draft"])
    np.testing.assert_array_equal(nv, z["num_valid"])


class _NeverDone:
    def query(self) -> bool:
        return False


def trace_ops(z):
    """Yield (step, docs, inflight) of the scripted index trace."""
    blob, offs = z["docs_blob"], z["docs_blob_offs"]
    for step, (s, nd, infl) in enumerate(z["ops"]):
        b = blob[offs[step]:offs[step + 1]]
        docs, p = [], 0
        for _ in range(int(nd)):
            n = int(b[p])
            docs.append(b[p + 1:p + 1 + n])
            p += 1 + n
        yield step, docs, bool(infl)


def test_index_trace():
    z = golden("index_trace")
    gi = GlobalIndexOracle(capacity=96, delta_capacity=40, k=4,
                           max_occurrences=8, rebuild_threshold=25)
    for step, docs, infl in trace_ops(z):
        if infl and gi._rebuild_event is None:
            gi._rebuild_event = _NeverDone()
            gi._pending = (gi.active_len, gi.active_doc_lens)
        gi.append_documents(docs)
        if step in (14, 27):
            gi._rebuild_event = None
            gi._pending = None
        _state_equal(gi, z, f"_{step}")


# ingest trace: the reference's harvest_finished / ingest_active under
# rebuilds that finish only at the script's polls marked done
INGEST_KW = dict(k=4, max_pattern_len=8, max_occurrences=8, num_backoff=3,
                 enable_global=True, global_capacity=200, delta_capacity=64,
                 rebuild_threshold=32)
HARVEST, ACTIVE, POLL = 0, 1, 2


class ScriptedEvent:
    """A rebuild event whose completion the test sets before each poll."""

    def __init__(self):
        self.done = False

    def query(self) -> bool:
        return self.done


def ingest_ops(z):
    """Yield (i, kind, args) of the ingest trace: HARVEST (tok, idx, len),
    ACTIVE (tok, keys, len, final, chunk), POLL (done,)."""
    for i, kind in enumerate(z["kinds"]):
        if kind == HARVEST:
            yield i, HARVEST, (z[f"tok_{i}"], z[f"idx_{i}"], z[f"len_{i}"])
        elif kind == ACTIVE:
            yield i, ACTIVE, (z[f"tok_{i}"], z[f"keys_{i}"], z[f"len_{i}"],
                              bool(z[f"final_{i}"]), int(z[f"chunk_{i}"]))
        else:
            yield i, POLL, (bool(z[f"done_{i}"]),)


def ingest_state_equal(gi, ingested: dict, z, i) -> None:
    """Index state after op i (live buffers, lists, the running rebuild's
    staged corpus and doc lengths) and ingest_active's progress dict."""
    _state_equal(gi, z, f"_{i}")
    running = gi._rebuild_event is not None
    assert running == bool(z[f"in_flight_{i}"])
    if running:
        assert gi._pending[0] == int(z[f"pend_n_new_{i}"])
        np.testing.assert_array_equal(np.array(list(gi._pending[1]),
                                               np.int64), z[f"pend_lens_{i}"])
        np.testing.assert_array_equal(gi.staging_corpus, z[f"staging_{i}"])
    items = sorted(ingested.items())
    assert [k for k, _ in items] == z[f"ing_keys_{i}"].tolist()
    assert [v for _, v in items] == z[f"ing_vals_{i}"].tolist()


def test_ingest_trace_finish_at_user_poll():
    """The oracle's schedule behind device-side ingest (a rebuild is still
    running at append_documents' own polls and completes at a caller's
    poll) against the reference driven that way: Python row indices,
    lengths <= 0 and past the row, documents longer than the delta, drops
    while a snapshot is running, evictions, ingest_active's chunk /
    overlap / final rules, and polls that find the rebuild running."""
    z = golden("ingest_trace")
    o = DrafterOracle(async_rebuild=True, finish_at_user_poll=True,
                      **INGEST_KW)
    ev = ScriptedEvent()
    o.global_index.rebuild_event_factory = lambda: ev
    for i, kind, args in ingest_ops(z):
        if kind == HARVEST:
            tok, idx, lens = args
            o.harvest_finished([int(r) for r in idx], [int(x) for x in lens],
                               tok)
        elif kind == ACTIVE:
            tok, keys, lens, final, chunk = args
            o.ingest_active([int(k) for k in keys], list(tok),
                            [int(x) for x in lens], final=final, chunk=chunk)
        else:
            ev.done = args[0]
            o.poll()
            ev.done = False
        ingest_state_equal(o.global_index, o._ingested, z, i)


@pytest.mark.parametrize("i", range(4))
def test_expand_alpha_and_weights(i):
    z = golden("expand_alpha_weights")
    cont, occ, cap = z[f"cont_{i}"], z[f"occ_{i}"], z[f"cap_{i}"]
    k = cont.shape[2]
    ch, nv, ne, sc = expand_chain(cont, occ, k, min_token_prob=0.05, cap=cap,
                                  alpha=float(z[f"alpha_{i}"]))
    np.testing.assert_array_equal(ch, z[f"chain_{i}"])
    np.testing.assert_array_equal(nv, z[f"nv_{i}"])
    np.testing.assert_array_equal(ne, z[f"emit_{i}"])
    np.testing.assert_array_equal(sc, z[f"score_{i}"])
    ch, nv, ne, sc = expand_chain(cont, occ, k, min_token_prob=0.05, cap=cap,
                                  weights=z[f"w_{i}"])
    np.testing.assert_array_equal(ch, z[f"wchain_{i}"])
    np.testing.assert_array_equal(nv, z[f"wnv_{i}"])
    np.testing.assert_array_equal(ne, z[f"wemit_{i}"])
    np.testing.assert_allclose(sc, z[f"wscore_{i}"], rtol=1e-4, atol=1e-5)
