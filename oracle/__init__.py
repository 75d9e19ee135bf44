"""CPU restatement of the reference drafter's algorithm -- TEST INFRASTRUCTURE.

This package is the oracle: a numpy (and plain-Python for the brute-force
definitions) restatement of zip95297/SuffixGPU's pure-torch/CPU path.  Each
function cites the reference file:line it follows.  It exists only to check
the HIP implementation in ``suffixgpu_amd`` and to time a CPU baseline.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import anything from here; the product package never
does, and fails loudly when its HIP library is missing.

Pinning status (what checks each function against something other than
itself):

* ``naive``          -- textbook brute-force definitions; checked by the
  reference's known-answer tests (tests/test_oracle_kats.py).
* ``sa``             -- suffix array vs brute force sort + uniqueness; interval
  search vs brute-force bounds; golden vectors.
* ``local``          -- match_back / candidates / occurrences vs brute force
  and the local-match KATs; full local propose vs golden vectors written by
  the reference itself.
* ``expand``         -- majority-vote KATs, the pairwise==sort property,
  golden vectors (alpha and weights included).
* ``global_index``   -- global-index KATs and regressions; write-path state
  traces vs golden vectors.
* ``drafter``        -- update_state / propose_with_update KATs; end-to-end
  golden vectors (local-only and local+global).

No function is left "parity unpinned" except the weighted vote's fp32 sum
order (weights are an expand_chain option the drafter never uses): float
sums of weights are compared within the reference's own rtol=1e-4.
"""
