"""Whole drafter on gfx950 vs the oracle: local+global decode steps on the
synthetic workloads, HIP-graph capture and replay, serial vs parallel
paths, and the reference's speculative-loop verification tests."""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle.drafter import DrafterOracle
from suffixgpu_amd import synth

pytestmark = pytest.mark.gpu

I32 = np.int32


def T(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def N(t):
    return t.cpu().numpy()


GLOBAL_KW = dict(k=16, max_pattern_len=32, max_occurrences=128,
                 num_backoff=8, max_spec_factor=2.0, min_token_prob=0.1,
                 enable_global=True, global_capacity=1 << 16,
                 delta_capacity=1 << 12, rebuild_threshold=1 << 30)


def _global_pair(gpu, seed=3, b=24, s=2048, **over):
    from suffixgpu_amd import SuffixGPUDrafter
    kw = dict(GLOBAL_KW)
    kw.update(over)
    w = synth.global_corpus(seed=seed, capacity=kw["global_capacity"],
                            delta_fill=kw["delta_capacity"] // 2, n_docs=40,
                            b=b, s=s, seq_hi=1500)
    d = SuffixGPUDrafter(device=gpu, **kw)
    o = DrafterOracle(**kw)
    d.global_index.load_documents([T(x, gpu) for x in w.active_docs])
    o.global_index.load_documents(w.active_docs)
    d.global_index.append_documents([T(x, gpu) for x in w.delta_docs])
    o.global_index.append_documents(w.delta_docs)
    return w, d, o


def test_global_step_split_delta_vs_oracle(gpu):
    """A 2^16 delta capacity splits every row's delta scan over several
    workgroups of the fused step (B=24 rows)."""
    w, d, o = _global_pair(gpu, seed=6, delta_capacity=1 << 16)
    assert d.global_index.delta_len > 20000
    bt = w.batch
    tg = T(bt.tokens, gpu)
    draft, nv, new = d.propose_with_update(T(bt.num_tokens, gpu), tg,
                                           T(bt.sampled, gpu))
    to = bt.tokens.copy()
    ed, env, enew = o.propose_with_update(bt.num_tokens, to, bt.sampled)
    np.testing.assert_array_equal(N(new), enew)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)


def test_global_step_vs_oracle(gpu):
    w, d, o = _global_pair(gpu)
    bt = w.batch
    tg = T(bt.tokens, gpu)
    draft, nv, new = d.propose_with_update(T(bt.num_tokens, gpu), tg,
                                           T(bt.sampled, gpu))
    to = bt.tokens.copy()
    ed, env, enew = o.propose_with_update(bt.num_tokens, to, bt.sampled)
    np.testing.assert_array_equal(N(tg), to)
    np.testing.assert_array_equal(N(new), enew)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)
    assert (env > 0).sum() > 0
    # plain propose with a mask, and max_model_len / valid counts
    mask = np.arange(bt.tokens.shape[0]) % 3 != 0
    draft, nv = d.propose(new, tg, T(mask, gpu))
    ed, env = o.propose(enew, to, mask)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)
    vc = np.minimum((bt.sampled != -1).sum(1), 2).astype(np.int64)
    draft, nv, new = d.propose_with_update(new, tg, T(bt.sampled, gpu),
                                           T(vc, gpu), max_model_len=1500)
    ed, env, enew = o.propose_with_update(enew, to, bt.sampled, vc,
                                          max_model_len=1500)
    np.testing.assert_array_equal(N(tg), to)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)
    np.testing.assert_array_equal(N(new), enew)


def test_global_step_patterns_past_key_rows_vs_oracle(gpu):
    """Patterns of up to 48 tokens against 32-token key rows: a search
    probe whose row ties with the pattern finishes the comparison in the
    corpus.  The template corpus has matches longer than the rows."""
    from oracle.sa import suffix_match_backoff
    p = 48
    w, d, o = _global_pair(gpu, seed=5, max_pattern_len=p, num_backoff=5)
    bt = w.batch
    gi = o.global_index
    # the SA match lengths of the rows' tails, as the step will see them
    # after the update: some pass the key rows' 32 tokens
    q = np.zeros((bt.tokens.shape[0], p), dtype=np.int32)
    ql = np.zeros(bt.tokens.shape[0], dtype=np.int64)
    for i in range(bt.tokens.shape[0]):
        acc = int((bt.sampled[i] != -1).sum())
        ctx = np.concatenate([bt.tokens[i, :bt.num_tokens[i]],
                              bt.sampled[i, :acc]])
        n = min(len(ctx), p)
        q[i, :n] = ctx[len(ctx) - n:]
        ql[i] = n
    sa_len, _, _ = suffix_match_backoff(gi.sa, gi.corpus, q, ql, p,
                                        np.array([p], dtype=np.int64))
    assert (sa_len[:, 0] > 32).sum() >= 4, sa_len[:, 0]
    tg = T(bt.tokens, gpu)
    draft, nv, new = d.propose_with_update(T(bt.num_tokens, gpu), tg,
                                           T(bt.sampled, gpu))
    to = bt.tokens.copy()
    ed, env, enew = o.propose_with_update(bt.num_tokens, to, bt.sampled)
    np.testing.assert_array_equal(N(new), enew)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)


def test_serial_equals_parallel_paths(gpu):
    w, d, o = _global_pair(gpu)
    d2, _, _ = None, None, None
    from suffixgpu_amd import SuffixGPUDrafter
    kw = dict(GLOBAL_KW)
    d2 = SuffixGPUDrafter(device=gpu, parallel_paths=False, **kw)
    d2.global_index.load_documents([T(x, gpu) for x in w.active_docs])
    d2.global_index.append_documents([T(x, gpu) for x in w.delta_docs])
    bt = w.batch
    outs = []
    for dr in (d, d2):
        tg = T(bt.tokens, gpu)
        outs.append([N(x) for x in dr.propose_with_update(
            T(bt.num_tokens, gpu), tg, T(bt.sampled, gpu))] + [N(tg)])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("enable_global", [False, True])
def test_graph_capture_replay(gpu, enable_global):
    """A captured propose_with_update step replays identically to eager,
    across replays with eager work and syncs in between."""
    kw = {} if enable_global else dict(enable_global=False)
    w, d, o = _global_pair(gpu, **kw) if enable_global else (None, None, None)
    if not enable_global:
        from suffixgpu_amd import SuffixGPUDrafter
        wl = synth.local_zipf(seed=2, b=16, s=4096)
        kwl = dict(GLOBAL_KW)
        kwl["enable_global"] = False
        d = SuffixGPUDrafter(device=gpu, **kwl)
        tokens, nt, sampled = wl.tokens, wl.num_tokens, wl.sampled
    else:
        tokens, nt = w.batch.tokens, w.batch.num_tokens
        sampled = w.batch.sampled
    buf = T(tokens, gpu)
    ntg = T(nt, gpu)
    sg = T(sampled, gpu)
    # eager reference on a copy
    ref_buf = buf.clone()
    ref = d.propose_with_update(ntg.clone(), ref_buf, sg)
    ref = [N(x) for x in ref]
    # warm up on scratch state, then capture
    for _ in range(2):
        d.propose_with_update(ntg.clone(), buf.clone(), sg)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    nt_static = ntg.clone()
    with torch.cuda.graph(g):
        out = d.propose_with_update(nt_static, buf, sg)
    for rep in range(4):
        nt_static.copy_(ntg)
        buf.copy_(T(tokens, gpu))
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, ref):
            np.testing.assert_array_equal(N(a), b, err_msg=f"replay {rep}")
        np.testing.assert_array_equal(N(buf), N(ref_buf))
        _ = torch.arange(1000, device=gpu).sum().item()  # eager work


# ------------------------------------------- reference verification loops
def _make(gpu, enable_global=True):
    from suffixgpu_amd import SuffixGPUDrafter
    return SuffixGPUDrafter(k=4, device=gpu, max_pattern_len=8,
                            max_occurrences=16, enable_global=enable_global,
                            global_capacity=1 << 16, delta_capacity=1 << 12,
                            rebuild_threshold=1 << 10)


def _adapter_propose(d, buf, nts, pending):
    n = len(pending)
    buf[0, nts:nts + n] = torch.tensor(pending, dtype=torch.int32,
                                       device=buf.device)
    return d.propose(torch.tensor([nts + n], dtype=torch.int32,
                                  device=buf.device), buf)


def _repetitive_doc(seed, n_blocks=12):
    g = random.Random(seed)
    blocks = [[g.randint(0, 5) for _ in range(6)] for _ in range(4)]
    doc = []
    for _ in range(n_blocks):
        doc.extend(g.choice(blocks))
    return doc


def _nonrepeating_doc(seed, n=30):
    g = random.Random(seed)
    doc = []
    while len(doc) < n:
        t = g.randint(0, 15)
        if len(doc) >= 2 and any(doc[i] == doc[-2] and doc[i + 1] == doc[-1]
                                 and doc[i + 2] == t
                                 for i in range(len(doc) - 2)):
            continue
        doc.append(t)
    return doc


def _spec_loop(d, doc, prompt_len, gpu):
    prompt = doc[:prompt_len]
    target = len(doc) - prompt_len
    buf = torch.zeros(1, len(doc) + 12, dtype=torch.int32, device=gpu)
    buf[0, :prompt_len] = torch.tensor(prompt, dtype=torch.int32)
    gen, pending, steps, acc = [], [doc[prompt_len]], 0, 0
    while len(gen) < target:
        steps += 1
        assert steps < 10000
        draft, nv = _adapter_propose(d, buf, prompt_len + len(gen), pending)
        gen.extend(pending)
        if len(gen) >= target:
            break
        base = prompt_len + len(gen)
        a = 0
        dl = N(draft)[0]
        while a < int(nv[0]) and base + a < len(doc) and dl[a] == doc[base + a]:
            a += 1
        acc += a
        pending = [int(dl[i]) for i in range(a)]
        if base + a < len(doc):
            pending.append(doc[base + a])
        else:
            gen.extend(pending)
            break
    return gen[:target], steps, acc, buf


def test_spec_loop_exact_local(gpu):
    doc = _repetitive_doc(7)
    gen, steps, acc, _ = _spec_loop(_make(gpu, False), doc, 4, gpu)
    assert gen == doc[4:]
    assert steps < len(doc) - 4 and acc > 0


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_spec_loop_exact_random(gpu, seed):
    doc = _nonrepeating_doc(seed, 48)
    gen, _, _, _ = _spec_loop(_make(gpu, False), doc, 6, gpu)
    assert gen == doc[6:]


def test_global_warmup_improves_acceptance(gpu):
    d = _make(gpu)
    doc = _nonrepeating_doc(11, 32)
    accs = []
    for _ in range(2):
        gen, _, acc, buf = _spec_loop(d, doc, 4, gpu)
        assert gen == doc[4:]
        d.harvest_rows([buf[0]], [4 + len(gen)])
        accs.append(acc)
    assert accs[1] > accs[0] and accs[1] >= 8


def test_ingest_then_cross_request_draft(gpu):
    from suffixgpu_amd import SuffixGPUDrafter
    d = SuffixGPUDrafter(k=4, device=gpu, max_pattern_len=8,
                         max_occurrences=8, enable_global=True,
                         global_capacity=1024, delta_capacity=256,
                         rebuild_threshold=100000)
    phrase = [11, 12, 13, 14, 15, 16, 17, 18]
    resp = torch.tensor(phrase * 8, dtype=torch.int32, device=gpu)
    d.ingest_active(["a"], [resp], [len(resp)], chunk=16)
    buf = torch.zeros(1, 32, dtype=torch.int32, device=gpu)
    cur = [99, 98] + phrase[:6]
    buf[0, :len(cur)] = torch.tensor(cur, dtype=torch.int32)
    draft, nv = d.propose(torch.tensor([len(cur)], dtype=torch.int32,
                                       device=gpu), buf,
                          torch.ones(1, dtype=torch.bool, device=gpu))
    n = int(nv[0])
    assert n > 0 and N(draft)[0, :n].tolist() == (phrase[6:] + phrase)[:n]


@pytest.mark.parametrize("enable_global", [False, True])
def test_step_long_rows_vs_oracle(gpu, enable_global):
    """Rows of 40000 tokens (streamed local role) in the fused step, with
    and without the global index (without it, rows this long run the
    1024-thread local-only kernel): rows are windows of the document
    stream at committed lengths around the 16384-position chunk
    boundaries."""
    from suffixgpu_amd import SuffixGPUDrafter
    s, t = 40000, 17
    w, d, o = _global_pair(gpu, seed=9, b=4, s=2048)
    if not enable_global:
        kw = dict(GLOBAL_KW, enable_global=False)
        d, o = SuffixGPUDrafter(device=gpu, **kw), DrafterOracle(**kw)
    stream = np.concatenate(w.active_docs + w.delta_docs).astype(I32)
    rng = np.random.default_rng(9)
    q_list = [0, 3, 16384, 16385, 20000, 39990, s - t, s]
    b = len(q_list)
    rows = np.zeros((b, s), dtype=I32)
    sampled = np.full((b, t), -1, dtype=I32)
    for i, q in enumerate(q_list):
        off = int(rng.integers(0, stream.shape[0] - s - t))
        rows[i] = stream[off:off + s]
        acc = int(rng.integers(0, t + 1))
        sampled[i, :acc] = stream[off + q:off + q + acc][:acc]
    nt = np.array(q_list, dtype=I32)
    tg = T(rows, gpu)
    draft, nv, new = d.propose_with_update(T(nt, gpu), tg, T(sampled, gpu))
    to = rows.copy()
    ed, env, enew = o.propose_with_update(nt, to, sampled)
    np.testing.assert_array_equal(N(tg), to)
    np.testing.assert_array_equal(N(new), enew)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)
    assert (env > 0).sum() > 0


@pytest.mark.parametrize("s", [8192, 16384])
def test_step_dense_grid_vs_oracle(gpu, s):
    """B=100 rows with global memory on make a grid of 300 workgroups,
    more than the CUs: the step then sizes every role for two workgroups
    per CU (at S=16384 the local role streams its row)."""
    w, d, o = _global_pair(gpu, seed=11, b=100, s=s)
    bt = w.batch
    tg = T(bt.tokens, gpu)
    draft, nv, new = d.propose_with_update(T(bt.num_tokens, gpu), tg,
                                           T(bt.sampled, gpu))
    to = bt.tokens.copy()
    ed, env, enew = o.propose_with_update(bt.num_tokens, to, bt.sampled)
    np.testing.assert_array_equal(N(tg), to)
    np.testing.assert_array_equal(N(new), enew)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)
    assert (env > 0).sum() > 10


@pytest.mark.parametrize("b", [180, 256])
def test_step_wave_grid_split_delta_vs_oracle(gpu, b):
    """Batches whose grid runs in waves (3 B > 512) split a 2^16-capacity
    delta over several parts within 1024 workgroups (B=180: 3 parts, 900
    workgroups; B=256: 2 parts, 1024), dispatched by role."""
    w, d, o = _global_pair(gpu, seed=12, b=b, s=2048,
                           delta_capacity=1 << 16)
    assert d.global_index.delta_len > 30000
    bt = w.batch
    tg = T(bt.tokens, gpu)
    draft, nv, new = d.propose_with_update(T(bt.num_tokens, gpu), tg,
                                           T(bt.sampled, gpu))
    to = bt.tokens.copy()
    ed, env, enew = o.propose_with_update(bt.num_tokens, to, bt.sampled)
    np.testing.assert_array_equal(N(tg), to)
    np.testing.assert_array_equal(N(new), enew)
    np.testing.assert_array_equal(N(draft), ed)
    np.testing.assert_array_equal(N(nv), env)
    assert (env > 0).sum() > b // 2
