"""Engine adapter on gfx950: a simulated serving loop with arrivals,
speculative verification, finishes and harvests, checked step by step
against the oracle drafter driven with the same persistent-batch state."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.drafter import DrafterOracle
from suffixgpu_amd import synth
from suffixgpu_amd.adapter import SlotTable

pytestmark = pytest.mark.gpu

I32 = np.int32
KW = dict(k=4, max_pattern_len=8, max_occurrences=16, num_backoff=3,
          enable_global=True, global_capacity=1 << 14, delta_capacity=1 << 11,
          rebuild_threshold=1 << 10, max_spec_factor=1.0,
          min_token_prob=0.05)


def _verify(draft, nv, truth, pos, k):
    """Sampled ids of one request: the accepted draft prefix plus the
    target's next token (-1 padded to k + 1)."""
    a = 0
    while a < nv and pos + a < len(truth) and draft[a] == truth[pos + a]:
        a += 1
    out = list(truth[pos:pos + a + 1])
    return out + [-1] * (k + 1 - len(out))


@pytest.mark.parametrize("seed", [1, 2])
def test_serving_loop_vs_oracle(gpu, seed):
    from suffixgpu_amd.adapter import SuffixProposerGPU
    rng = np.random.default_rng(seed)
    tc = synth.TemplateCorpus(seed=seed, n_templates=6)
    k, nseq, mlen = KW["k"], 6, 720
    ad = SuffixProposerGPU(max_num_seqs=nseq, max_model_len=mlen,
                           device=gpu, **KW)
    o = DrafterOracle(**KW)
    ot = np.zeros((nseq, mlen), I32)
    on = np.zeros(nseq, I32)
    table = SlotTable(nseq)           # the oracle side's own slot table
    truth, pos, last = {}, {}, {}
    nxt = 0
    finished = 0
    for step in range(260):
        # arrivals
        if len(table) < nseq and (len(table) < 2 or rng.random() < 0.25):
            seq = tc.sequence(lo=200, hi=mlen - 2 * (k + 1))
            plen = int(rng.integers(20, 120))
            rid = f"r{nxt}"
            nxt += 1
            truth[rid] = seq.tolist()
            pos[rid] = plen
            last[rid] = ([], 0)
            assert ad.add_request(rid, seq[:plen]) == table.add(rid)
            s = table.slot_of[rid]
            ot[s, :plen] = seq[:plen]
            on[s] = plen
        # verification of last step's drafts -> sampled ids
        n = len(table)
        samp = np.full((n, k + 1), -1, I32)
        for s, rid in enumerate(table.req_at):
            d, v = last[rid]
            row = _verify(d, v, truth[rid], pos[rid], k)
            samp[s] = row
            pos[rid] += sum(1 for x in row if x != -1)
        draft, nv = ad.propose(torch.from_numpy(samp).to(gpu))
        ed, env, enew = o.propose_with_update(on[:n].copy(), ot[:n], samp)
        on[:n] = enew
        np.testing.assert_array_equal(draft.cpu().numpy(), ed,
                                      err_msg=f"step {step}")
        np.testing.assert_array_equal(nv.cpu().numpy(), env)
        for s, rid in enumerate(table.req_at):
            last[rid] = (ed[s].tolist(), int(env[s]))
        # finishes: requests whose next verification could run past truth
        done = [r for r in table.req_at
                if pos[r] + k + 1 >= len(truth[r]) or rng.random() < 0.01]
        if done:
            lens = [pos[r] for r in done]
            ad.finish_requests(done, lens)
            slots = [table.slot_of[r] for r in done]
            o.harvest_finished(slots, lens, ot)
            for src, dst in table.remove(done):
                ot[dst] = ot[src]
                on[dst] = on[src]
            finished += len(done)
        ad.poll()
        o.poll()
    assert finished >= 4
    # committed rows are the truth, and the global memory matches
    rows = ad.tokens.cpu().numpy()
    counts = ad.num_tokens.cpu().numpy()
    for s, rid in enumerate(table.req_at):
        assert counts[s] == pos[rid]
        assert rows[s, :pos[rid]].tolist() == truth[rid][:pos[rid]]
    gi, og = ad.drafter.global_index, o.global_index
    assert gi.active_len == og.active_len and gi.delta_len == og.delta_len
    np.testing.assert_array_equal(gi.corpus.cpu().numpy(), og.corpus)
    np.testing.assert_array_equal(gi.delta.cpu().numpy()[:gi.delta_len],
                                  og.delta[:og.delta_len])


def test_captured_propose_matches_eager(gpu):
    """The adapter's propose (step kernel + count copy) captured once and
    replayed over several steps gives the eager adapter's drafts."""
    from suffixgpu_amd.adapter import SuffixProposerGPU
    rng = np.random.default_rng(3)
    tc = synth.TemplateCorpus(seed=3, n_templates=4)
    k, n = KW["k"], 4
    kw = dict(KW, enable_global=False)
    eager = SuffixProposerGPU(max_num_seqs=n, max_model_len=600, device=gpu,
                              **kw)
    graph = SuffixProposerGPU(max_num_seqs=n, max_model_len=600, device=gpu,
                              **kw)
    seqs = [tc.sequence(lo=300, hi=500) for _ in range(n)]
    for i, sq in enumerate(seqs):
        eager.add_request(i, sq[:40])
        graph.add_request(i, sq[:40])
    samp = torch.full((n, k + 1), -1, dtype=torch.int32, device=gpu)
    samp[:, 0] = torch.tensor([int(sq[40]) for sq in seqs], device=gpu)
    graph.propose(samp)
    eager.propose(samp)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gd, gnv = graph.propose(samp)
    pos = [41] * n
    for step in range(12):
        batch = np.full((n, k + 1), -1, I32)
        for i, sq in enumerate(seqs):
            a = int(rng.integers(1, k + 2))
            batch[i, :a] = sq[pos[i]:pos[i] + a]
            pos[i] += a
        samp.copy_(torch.from_numpy(batch))
        ed, env = eager.propose(samp)
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(gd.cpu().numpy(), ed.cpu().numpy())
        np.testing.assert_array_equal(gnv.cpu().numpy(), env.cpu().numpy())
    np.testing.assert_array_equal(graph.num_tokens.cpu().numpy(), pos)
