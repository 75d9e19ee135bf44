"""sfx_propose_step_noalloc (the step with its scratch in a static device
array, for callers that cannot allocate) against sfx_propose_step with a
caller workspace, both called through the C ABI on identical inputs: two
calls in a row, the second with a smaller batch, then a local-only call.
The host-side rejection of batches beyond the static scratch is checked
without a GPU in test_abi.py."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from suffixgpu_amd import synth

pytestmark = pytest.mark.gpu

CFG = dict(k=16, max_pattern_len=32, max_occurrences=128, num_backoff=8,
           max_spec_factor=2.0, min_token_prob=0.1)


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _run(d, ix, tokens, nt, sampled, with_ws):
    """One propose_with_update through the C ABI: (draft, nv, new, rows)."""
    from suffixgpu_amd import _lib
    L = _lib.lib()
    b = tokens.shape[0]
    dev = tokens.device
    rows = tokens.clone()
    bt, keep = _lib.make_batch(rows, nt, sampled=sampled,
                               limit=tokens.shape[1])
    draft = torch.full((b, d.k), -9, dtype=torch.int32, device=dev)
    nv = torch.full((b,), -9, dtype=torch.int32, device=dev)
    new = torch.full((b,), -9, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    ixp = None if ix is None else ctypes.byref(ix)
    if with_ws:
        ws = None
        nbytes = 0
        if ix is not None:
            nbytes = int(L.sfx_step_workspace_size(d._params, b,
                                                   ix.delta_capacity))
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        rc = L.sfx_propose_step(d._params, ixp, bt, draft.data_ptr(),
                                nv.data_ptr(), new.data_ptr(),
                                None if ws is None else ws.data_ptr(),
                                nbytes, st)
    else:
        rc = L.sfx_propose_step_noalloc(d._params, ixp, bt,
                                        draft.data_ptr(), nv.data_ptr(),
                                        new.data_ptr(), st)
    assert rc == 0, rc
    torch.cuda.synchronize()
    del keep
    return [t.cpu().numpy() for t in (draft, nv, new, rows)]


def test_noalloc_step_matches_workspace_step(gpu):
    from suffixgpu_amd import SuffixGPUDrafter
    kw = dict(enable_global=True, global_capacity=1 << 17,
              delta_capacity=1 << 16, rebuild_threshold=1 << 30, **CFG)
    w = synth.global_corpus(seed=12, capacity=kw["global_capacity"],
                            delta_fill=1 << 15, n_docs=60, b=48, s=4096,
                            seq_hi=3000)
    d = SuffixGPUDrafter(device=gpu, **kw)
    d.global_index.load_documents([T(x, gpu) for x in w.active_docs])
    d.global_index.append_documents([T(x, gpu) for x in w.delta_docs])
    ix = d.global_index.index_struct()
    bt = w.batch
    for b in (48, 20):  # the second call is smaller
        args = (T(bt.tokens[:b], gpu), T(bt.num_tokens[:b], gpu),
                T(bt.sampled[:b], gpu))
        got = _run(d, ix, *args, with_ws=False)
        exp = _run(d, ix, *args, with_ws=True)
        for g, e in zip(got, exp):
            np.testing.assert_array_equal(g, e, err_msg=f"B={b}")
        assert (got[1] > 0).sum() > b // 2
    # local-only: no scratch involved, same results
    lw = synth.local_zipf(seed=2, b=16, s=2048, lo=512)
    dl = SuffixGPUDrafter(device=gpu, **CFG)
    args = (T(lw.tokens, gpu), T(lw.num_tokens, gpu), T(lw.sampled, gpu))
    got = _run(dl, None, *args, with_ws=False)
    exp = _run(dl, None, *args, with_ws=True)
    for g, e in zip(got, exp):
        np.testing.assert_array_equal(g, e)
