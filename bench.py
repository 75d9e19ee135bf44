"""Drafter benchmark: propose_with_update on one MI355X.

Workload (the drafter's decode shape with global memory on): B=64 request
rows of S=8192 int32 tokens, k=16, max_pattern_len=32, num_backoff=8,
max_occurrences=128, max_spec_factor=2.0, min_token_prob=0.1, and a
2^22-token corpus + SA built from 1024 template-sharing synthetic sequences
plus a half-full 2^16-token delta; each row carries a geometric(0.3)+1
accepted-token sampled block.  One step = update_state + local match +
SA/delta match + merge + expansion + selection, captured once as a HIP
graph and replayed; inputs stay resident in HBM.

Printed: one JSON line with p50 us/step (value), the dominant kernel's
roofline, the SA-build throughput and the CPU baseline (the oracle's numpy
restatement of the same step on this host, on a bounded sample).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

# HIP graph launch path: with CLR's graph packet capture (on by default in
# ROCm 7.2) a replay of the one-kernel step graph spends about 2.6 us more
# between kernels than with it off (pipelined replays 35.4 -> 32.7 us at
# B=64, S=8192).  Read once when the HIP runtime starts, so it is set before
# torch is imported; a value already in the environment is kept.
os.environ.setdefault("DEBUG_CLR_GRAPH_PACKET_CAPTURE", "0")

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = ("propose_with_update p50 µs/step (B=64,S=8192); HBM GB/s; "
          "SA build Mtok/s")
HBM_PEAK_GBPS = 8000.0
CFG = dict(k=16, max_pattern_len=32, max_occurrences=128, num_backoff=8,
           max_spec_factor=2.0, min_token_prob=0.1)
B, S, T_SAMPLED = 64, 8192, 17
CAPACITY, DELTA_CAP, DELTA_FILL = 1 << 22, 1 << 16, 1 << 15


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-steps", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the B=256 S=16384 1000-step decode loop")
    ap.add_argument("--e2e-steps", type=int, default=1000)
    ap.add_argument("--pmc-workload", action="store_true",
                    help="for rocprofv3 --pmc passes: a copy of known size, "
                    "a few step launches, then two SA rebuilds of the "
                    "corpus as the index runs them; prints no JSON")
    ap.add_argument("--sync-check", action="store_true",
                    help="for rocprofv3 --hip-trace: 20 eager "
                    "propose_with_update calls, then 20 graph replays, each "
                    "section between device synchronisations; prints no "
                    "JSON")
    ap.add_argument("--summarize-api", metavar="TRACE_DIR",
                    help="HIP API calls per section of a --sync-check "
                    "trace (rocprofv3 --hip-trace CSV output)")
    ap.add_argument("--summarize-counters", metavar="PMC_DIR",
                    help="mean of every counter per dispatch, per kernel, "
                    "from one rocprofv3 --pmc output of --pmc-workload")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR",
                                                         "WRITE_DIR"),
                    help="turn two rocprofv3 --pmc outputs (FETCH_SIZE, "
                    "WRITE_SIZE) of --pmc-workload into HBM bytes/launch")
    return ap.parse_args()


# --------------------------------------------------------------- roofline
def local_algorithmic_bytes(new_counts, accepted, k, b=None,
                            s=None) -> int:
    """Rows scanned once + sampled block read + scatter writes + draft,
    num_valid and counts (in/out), for b rows of s tokens."""
    b = B if b is None else b
    s = S if s is None else s
    n_eff = np.minimum(new_counts.astype(np.int64), s)
    return int(4 * n_eff.sum() + 4 * b * T_SAMPLED + 4 * accepted.sum()
               + 4 * b * (k + 3))


def reference_probe_footprint(sa, corpus, rpat, plen, P):
    """Distinct SA ranks and corpus positions the reference's merged
    binary search (ceil(log2(N+1)) fixed probes per bound, every length
    1..P) has to read to decide its comparisons."""
    n = sa.shape[0]
    iters = int(np.ceil(np.log2(n + 1)))
    rows = []
    for b in range(rpat.shape[0]):
        for ln in range(1, int(plen[b]) + 1):
            rows.append((b, ln))
    rb = np.array([r[0] for r in rows])
    rl = np.array([r[1] for r in rows])
    m = rb.shape[0]
    pats = np.zeros((m, P), np.int64)
    for j in range(P):
        t = rl - 1 - j
        pats[:, j] = np.where(t >= 0, rpat[rb, np.maximum(t, 0)], 0)
    pats2 = np.concatenate([pats, pats])
    rl2 = np.concatenate([rl, rl])
    upper = np.arange(2 * m) >= m
    lo = np.zeros(2 * m, np.int64)
    hi = np.full(2 * m, n, np.int64)
    ranks, cpos = [], []
    offs = np.arange(P)
    for _ in range(iters):
        mid = np.minimum((lo + hi) // 2, n - 1)
        active = lo < hi
        pos = sa[mid].astype(np.int64)
        idx = pos[:, None] + offs[None, :]
        tok = np.where(idx < n, corpus[np.minimum(idx, n - 1)], -1)
        valid = offs[None, :] < rl2[:, None]
        eq = (tok == pats2) | ~valid
        lcp = np.minimum(np.cumprod(eq, axis=1).sum(1), rl2)
        full = lcp >= rl2
        sp = np.minimum(pos + lcp, n - 1)
        sch = np.where(pos + lcp < n, corpus[sp], -1)
        pch = pats2[np.arange(2 * m), np.minimum(lcp, P - 1)]
        c = np.where(full, 0, np.where(sch < pch, -1, np.where(sch > pch, 1,
                                                                0)))
        go = (c < 0) | (upper & (c == 0))
        ranks.append(mid[active])
        need = np.minimum(lcp + 1, rl2)
        for r in np.flatnonzero(active):
            e = min(int(pos[r]) + int(need[r]), n)
            cpos.append(np.arange(int(pos[r]), e))
        lo = np.where(go, mid + 1, lo)
        hi = np.where(go, hi, mid)
    u_sa = np.unique(np.concatenate(ranks)) if ranks else np.zeros(0)
    u_c = np.unique(np.concatenate(cpos)) if cpos else np.zeros(0)
    return u_sa, u_c


def time_sa_builds(w, dev, side):
    """SA build throughput on a side stream (HIP events): the corpus
    snapshot (docs + SEP + sentinel) and a uniform-random low-repeat
    corpus of the same capacity."""
    import torch
    from suffixgpu_amd import synth
    from suffixgpu_amd.suffix_array import (build_state,
                                            build_suffix_array_into,
                                            build_suffix_array_rounds,
                                            read_build_state,
                                            sa_workspace_bytes)
    flat = np.concatenate([np.append(x, -2) for x in w.active_docs]).astype(
        np.int32)
    m = min(flat.shape[0] + 1, CAPACITY)
    rng = np.random.default_rng(4)
    uniform = rng.integers(0, synth.VOCAB_LARGE, size=CAPACITY).astype(
        np.int32)
    ws = torch.empty(sa_workspace_bytes(CAPACITY), dtype=torch.uint8,
                     device=dev)
    build_ms = {}
    for name, text_np, mm in (("corpus", flat, m), ("uniform", uniform,
                                                     CAPACITY)):
        text = torch.full((CAPACITY,), _lib_pad(), dtype=torch.int32,
                          device=dev)
        text[:text_np.shape[0]].copy_(torch.from_numpy(text_np))
        out = torch.empty(CAPACITY, dtype=torch.int32, device=dev)
        times = []
        for rep in range(3):
            torch.cuda.synchronize()
            side.wait_stream(torch.cuda.current_stream(dev))
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(side):
                e0.record(side)
                build_suffix_array_into(text, mm, out, ws, adaptive=True)
                e1.record(side)
            e1.synchronize()
            times.append(e0.elapsed_time(e1))
        build_ms[name] = (min(times), mm)
        log(f"SA build {name}: m={mm} {min(times):.2f} ms")
        # As the index's background rebuild runs it at steady state: the
        # rounds the previous build needed plus a margin of 2 (flagged as
        # expected to find the array final), with the radix path for the
        # rounds that took it, then the output (the device confirms the
        # array is final).
        prev = read_build_state(ws, mm)
        final, rounds, radix = prev.done, prev.needed + 2, prev.radix_mask & ~1
        fin = prev.needed + 1
        times = []
        for rep in range(3):
            torch.cuda.synchronize()
            side.wait_stream(torch.cuda.current_stream(dev))
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(side):
                e0.record(side)
                build_suffix_array_rounds(text, mm, out, ws, rounds, radix,
                                          fin)
                e1.record(side)
            e1.synchronize()
            times.append(e0.elapsed_time(e1))
        ok, _ = build_state(ws, mm)
        if not (final and ok):
            raise RuntimeError("SA build: hinted rounds did not finish")
        build_ms[name + "_hinted"] = (min(times), rounds)
        build_ms[name + "_radix"] = radix
        log(f"SA rebuild {name} ({rounds} rounds, as the index runs it): "
            f"{min(times):.2f} ms")
        key = "tables" if name == "corpus" else "tables_" + name
        build_ms[key] = index_tables_ms(text, out, dev, side, ws)
        log(f"key rows + n-gram table of the {name} text: {build_ms[key]}")
    del ws
    return build_ms


def index_tables_ms(text, sa, dev, side, ws) -> dict:
    """What a rebuild adds after the suffix array, on the rebuild stream:
    the key rows and the n-gram range table (best of 3, HIP events), the
    table read from the ranks' first four tokens that the key-row launch
    writes into the SA build workspace ``ws``, as the index does."""
    import torch
    from suffixgpu_amd import _lib
    from suffixgpu_amd.global_index import KEY_WIDTH, gram_slots_for
    L = _lib.lib()
    n = text.shape[0]
    keys = torch.empty(n * KEY_WIDTH, dtype=torch.int32, device=dev)
    slots = gram_slots_for(n)
    gram = torch.zeros(int(L.sfx_gram_table_bytes(slots)), dtype=torch.uint8,
                       device=dev)
    res = {"keys": [], "gram": []}
    for _ in range(3):
        torch.cuda.synchronize()
        side.wait_stream(torch.cuda.current_stream(dev))
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        with torch.cuda.stream(side):
            ev[0].record(side)
            _lib.check(L.sfx_sa_keys(text.data_ptr(), sa.data_ptr(), n, n,
                                     KEY_WIDTH, keys.data_ptr(),
                                     ws.data_ptr(), side.cuda_stream),
                       "keys")
            ev[1].record(side)
            _lib.check(L.sfx_gram_build(ws.data_ptr(), 4, n,
                                        gram.data_ptr(), slots,
                                        side.cuda_stream), "gram")
            ev[2].record(side)
        ev[2].synchronize()
        res["keys"].append(ev[0].elapsed_time(ev[1]))
        res["gram"].append(ev[1].elapsed_time(ev[2]))
    # header word 0: the longest run length the table holds (0: unusable)
    kmax = int(gram[0:4].view(torch.int32).item())
    del keys, gram
    return {"key_rows_ms": round(min(res["keys"]), 3),
            "gram_table_ms": round(min(res["gram"]), 3),
            "gram_slots": slots, "gram_table_kmax": kmax}


# ------------------------------------------------------------------ main
def main() -> int:
    args = parse()
    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(*args.summarize_pmc), indent=1))
        return 0
    if args.summarize_counters:
        print(json.dumps(summarize_counters(args.summarize_counters),
                         indent=1))
        return 0
    if args.summarize_api:
        print(json.dumps(summarize_api(args.summarize_api), indent=1))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this drafter benchmark runs on exactly "
                          "one GPU (the workload is one GPU's rows); "
                          f"--gpus {args.gpus} is not supported"}))
        return 2
    import torch

    from suffixgpu_amd import SuffixGPUDrafter, synth
    from suffixgpu_amd import _lib
    from suffixgpu_amd.suffix_array import (build_suffix_array_into,
                                            sa_workspace_bytes)

    dev = torch.device("cuda", 0)
    t0 = time.time()
    w = synth.global_corpus(seed=3, capacity=CAPACITY, delta_fill=DELTA_FILL,
                            n_docs=1024, b=B, s=S, t=T_SAMPLED)
    log(f"workload generated in {time.time() - t0:.1f}s: "
        f"{len(w.active_docs)} corpus docs, {len(w.delta_docs)} delta docs")

    d = SuffixGPUDrafter(device=dev, enable_global=True,
                         global_capacity=CAPACITY, delta_capacity=DELTA_CAP,
                         rebuild_threshold=1 << 30, **CFG)
    gi = d.global_index

    side = torch.cuda.Stream(dev)
    build_ms = None
    if not args.pmc_workload:
        build_ms = time_sa_builds(w, dev, side)

    gi.load_documents([torch.from_numpy(x).to(dev) for x in w.active_docs])
    gi.append_documents([torch.from_numpy(x).to(dev) for x in w.delta_docs])
    torch.cuda.synchronize()
    log(f"index: active_len={gi.active_len} delta_len={gi.delta_len}")
    if args.pmc_workload:
        return pmc_workload(d, w, dev)
    if args.sync_check:
        return sync_check(d, w, dev)

    bt = w.batch
    tokens0 = torch.from_numpy(bt.tokens).to(dev)
    buf = tokens0.clone()
    nt = torch.from_numpy(bt.num_tokens).to(dev)
    sampled = torch.from_numpy(bt.sampled).to(dev)

    # ---- capture one step; replays are identical (counts not fed back).
    for _ in range(3):
        d.propose_with_update(nt, buf.clone(), sampled)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = d.propose_with_update(nt, buf, sampled)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    cur = torch.cuda.current_stream(dev)
    torch.cuda.synchronize()
    tw0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record(cur)
        graph.replay()
        ends[i].record(cur)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - tw0) * 1e3
    per_us = [s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends)]
    p50 = statistics.median(per_us)
    draft, num_valid, new_counts = (x.cpu().numpy() for x in out)
    log(f"step p50 {p50:.2f} us, wall {wall_ms / args.steps * 1e3:.2f} "
        f"us/step, drafting rows {(num_valid > 0).sum()}/{B}, "
        f"mean num_valid {num_valid.mean():.2f}")

    compact = compact_index_step(dev, w, bt, (draft, num_valid),
                                 args.steps, args.warmup)
    log(f"index without search tables: {compact}")

    adapter_p50 = adapter_step_p50(d, dev, bt, args.steps, args.warmup)
    log(f"engine adapter step p50 {adapter_p50:.2f} us (step kernel + count "
        "feedback, captured)")

    # ---- the step kernel launched directly (no graph) between HIP events
    # on its stream, then the local and global kernels launched alone.
    step_us = step_kernel_us(d, dev, tokens0, nt, sampled, args.kernel_reps)
    acc = (bt.sampled != -1).sum(1)
    k_local_us, k_global_us = kernel_timings(d, dev, tokens0, nt, sampled,
                                             args.kernel_reps)
    log(f"kernel avg: step {step_us:.2f} us (local alone {k_local_us:.2f}, "
        f"global alone {k_global_us:.2f})")

    a_local = local_algorithmic_bytes(new_counts, acc, CFG["k"])
    a_global, fp = global_algorithmic_bytes(d, dev, buf, new_counts)
    log(f"algorithmic bytes: local {a_local}, global {a_global} ({fp})")
    step_bytes = a_local + a_global
    achieved = step_bytes / (step_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 2),
                "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 6),
                "traffic": load_traffic("k_step"), "kernel": "k_step",
                "algorithmic_bytes": step_bytes,
                "avg_launch_us": round(step_us, 3)}

    copy_gbps = copy_peak_gbps(dev)
    cold_p50 = cold_step_p50(graph, dev)
    conc = concurrent_rebuild(graph, w, dev, build_ms["corpus_hinted"][1],
                              build_ms["corpus_radix"])
    log(f"copy peak {copy_gbps:.0f} GB/s; cold-cache step p50 "
        f"{cold_p50:.2f} us; rebuild during replays: {conc}")
    c5 = c5_local_step(dev, args.kernel_reps)
    log(f"local step at B={C5_B} S={C5_S}: {c5}")
    e2e = None
    if not args.no_e2e:
        e2e = e2e_loop(dev, args.e2e_steps)
        log(f"e2e decode loop: {e2e}")

    local_cfgs = local_configs(dev, 200, not args.no_cpu)
    sweep = latency_sweep(dev, 50)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(d, w, args.cpu_steps,
                           (draft, num_valid, new_counts))

    sa_corpus_ms, sa_m = build_ms["corpus"]
    sa_uni_ms, _ = build_ms["uniform"]
    sa_reb_ms, sa_reb_rounds = build_ms["corpus_hinted"]
    result = {
        "metric": METRIC,
        "value": round(p50, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms / args.steps, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i32",
        "data": "synthetic",
        "config": {"workload": "propose_with_update, global memory on: "
                   "B=64 S=8192 k=16 P=32 R=128 num_backoff=8 "
                   "spec_factor=2.0 min_prob=0.1, corpus 2^22 (template "
                   "sequences, SA prebuilt) + delta 2^15/2^16, hipGraph "
                   "replay", "global_batch": B, "seq_len": S,
                   "parallelism": "none (1 GPU)",
                   "hip_env": {"DEBUG_CLR_GRAPH_PACKET_CAPTURE": os.environ.get(
                       "DEBUG_CLR_GRAPH_PACKET_CAPTURE")}},
        "step_hbm_gbps": round(step_bytes / (p50 * 1e-6) / 1e9, 3),
        "step_algorithmic_bytes": step_bytes,
        "sa_build_mtok_s": round(sa_m / (sa_corpus_ms * 1e-3) / 1e6, 2),
        "sa_build_uniform_mtok_s": round(CAPACITY / (sa_uni_ms * 1e-3) / 1e6,
                                         2),
        "sa_build_steps_equiv": round(sa_corpus_ms * 1e3 / p50, 1),
        "sa_rebuild_hinted_ms": round(sa_reb_ms, 3),
        "sa_rebuild_hinted_rounds": sa_reb_rounds,
        "sa_rebuild_hinted_mtok_s": round(sa_m / (sa_reb_ms * 1e-3) / 1e6, 2),
        "sa_rebuild_hbm": sa_rebuild_hbm(sa_reb_ms),
        "rebuild_tables": build_ms["tables"],
        "rebuild_tables_uniform": build_ms["tables_uniform"],
        "kernels_us": {"k_step": round(step_us, 3),
                       "k_local_alone": round(k_local_us, 3),
                       "k_global_alone": round(k_global_us, 3)},
        "roofline": roofline,
        "copy_peak_gbps": round(copy_gbps, 1),
        "roofline_frac_of_copy_peak": round(achieved / copy_gbps, 6),
        "cold_cache_step_p50_us": round(cold_p50, 3),
        "adapter_step_p50_us": round(adapter_p50, 3),
        "sa_rebuild_concurrent": conc,
        "c5_local_step": c5,
        "e2e_decode_loop": e2e,
        "local_configs": local_cfgs,
        "latency_sweep": sweep,
        "vram": drafter_device_bytes(d, B, S),
        "compact_index": compact,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


def _lib_pad() -> int:
    return 2 ** 31 - 1


def adapter_step_p50(d, dev, bt, steps: int, warmup: int) -> float:
    """The engine adapter's captured propose (the step plus the copy of the
    new counts into its resident counts) on the same 64 rows: p50 of the
    replays between an event pair; the counts are restored outside it."""
    import torch
    from suffixgpu_amd.adapter import SuffixProposerGPU
    ad = SuffixProposerGPU(k=d.k, max_num_seqs=B, max_model_len=S,
                           device=dev, drafter=d)
    for i in range(B):
        n = int(bt.num_tokens[i])
        ad.add_request(i, bt.tokens[i, :n])
    ad.tokens.copy_(torch.from_numpy(bt.tokens).to(dev))
    counts0 = ad.num_tokens.clone()
    samp = torch.from_numpy(bt.sampled).to(dev)
    for _ in range(3):
        ad.num_tokens.copy_(counts0)
        ad.propose(samp)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ad.propose(samp)
    cur = torch.cuda.current_stream(dev)
    per = []
    for i in range(warmup + steps):
        ad.num_tokens.copy_(counts0)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        g.replay()
        e1.record(cur)
        if i >= warmup:
            per.append((e0, e1))
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) * 1e3 for a, b in per)


def sa_rebuild_hbm(rebuild_ms: float):
    """HBM bytes of one background rebuild of the corpus (rocprofv3 PMC
    summary) over its measured time, against the 8 TB/s peak."""
    t = load_traffic("sa_rebuild")
    if not t:
        return None
    gbps = t / (rebuild_ms * 1e-3) / 1e9
    return {"traffic": t, "achieved_gbps": round(gbps, 1),
            "peak_gbps": HBM_PEAK_GBPS, "frac": round(gbps / HBM_PEAK_GBPS, 4)}



def copy_peak_gbps(dev) -> float:
    """Measured device-to-device copy bandwidth (read + write bytes / s)
    over a 1 GiB int32 buffer, best of 10."""
    import torch
    n = 1 << 28
    src = torch.ones(n, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    times = []
    for _ in range(12):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(src)
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1) * 1e-3)
    del src, dst
    return 2 * 4 * n / min(times[2:]) / 1e9


def cold_step_p50(graph, dev, reps: int = 40) -> float:
    """p50 µs of a replay after a 512 MiB scratch write (outside the timed
    region) has pushed the index, delta and rows out of L2 and MALL."""
    import torch
    scratch = torch.empty(1 << 27, dtype=torch.int32, device=dev)
    per = []
    for i in range(reps):
        scratch.fill_(i)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        e1.synchronize()
        per.append(e0.elapsed_time(e1) * 1e3)
    del scratch
    return statistics.median(per)


def concurrent_rebuild(graph, w, dev, rounds: int, radix: int) -> dict:
    """A 4.19M-token SA rebuild (as the index's background rebuild runs
    it: ``rounds`` doubling rounds, the last two flagged as the margin, the
    radix path for those in the mask ``radix``) enqueued on a side stream
    while the
    captured step replays on the main stream: build time, decode steps
    completed before the build's end event, and the step p50 meanwhile."""
    import torch
    from suffixgpu_amd.suffix_array import (build_state,
                                            build_suffix_array_rounds,
                                            sa_workspace_bytes)
    flat = np.concatenate([np.append(x, -2) for x in w.active_docs]).astype(
        np.int32)
    m = min(flat.shape[0] + 1, CAPACITY)
    text = torch.full((CAPACITY,), 2 ** 31 - 1, dtype=torch.int32,
                      device=dev)
    text[:flat.shape[0]].copy_(torch.from_numpy(flat))
    out = torch.empty(CAPACITY, dtype=torch.int32, device=dev)
    ws = torch.empty(sa_workspace_bytes(CAPACITY), dtype=torch.uint8,
                     device=dev)
    side = torch.cuda.Stream(dev)
    main = torch.cuda.current_stream(dev)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t0.record(main)
    side.wait_stream(main)
    b0 = torch.cuda.Event(enable_timing=True)
    b1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(side):
        b0.record(side)
        build_suffix_array_rounds(text, m, out, ws, rounds, radix,
                                  rounds - 1)
        b1.record(side)
    ends = []
    starts = []
    while len(ends) < 4000:
        s0 = torch.cuda.Event(enable_timing=True)
        s1 = torch.cuda.Event(enable_timing=True)
        s0.record(main)
        graph.replay()
        s1.record(main)
        starts.append(s0)
        ends.append(s1)
        if len(ends) % 8 == 0 and b1.query():
            break
    torch.cuda.synchronize()
    if not build_state(ws, m)[0]:
        raise RuntimeError("concurrent SA rebuild did not finish")
    build_ms = b0.elapsed_time(b1)
    done_at = t0.elapsed_time(b1)
    fin = [t0.elapsed_time(e) for e in ends]
    during = [a.elapsed_time(e) * 1e3 for a, e, f in zip(starts, ends, fin)
              if f <= done_at]
    steps = len(during)
    del text, out, ws
    return {"build_ms": round(build_ms, 3), "m": int(m),
            "steps_during_build": steps,
            "step_p50_us_during_build":
                round(statistics.median(during), 3) if during else None}


def replay_p50(fn, reps: int, warmup: int = 5, before=None):
    """Capture fn() once as a HIP graph; p50 µs of `reps` replays between
    event pairs (``before`` runs outside each timed pair), and the wall µs
    per replay of `reps` replays queued back to back."""
    import torch
    for _ in range(3):
        if before:
            before()
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    cur = torch.cuda.current_stream()
    per = []
    for i in range(warmup + reps):
        if before:
            before()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        g.replay()
        e1.record(cur)
        if i >= warmup:
            per.append((e0, e1))
    torch.cuda.synchronize()
    p50 = statistics.median(a.elapsed_time(b) * 1e3 for a, b in per)
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e6 / reps
    return p50, wall, out, g


def cpu_times(fn, reps: int, warmup: int) -> float:
    """p50 µs of fn() over `reps` calls after `warmup` calls."""
    for _ in range(warmup):
        fn()
    per = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        per.append(time.perf_counter() - t0)
    return statistics.median(per) * 1e6


# The reference's two local-only workloads: propose on B=8 rows of S=2048
# uniform tokens with one support threshold, and propose_with_update on
# B=64 rows of S=8192 Zipf tokens with eight.
CFG1 = dict(k=16, max_pattern_len=32, max_occurrences=128, num_backoff=1,
            max_spec_factor=None, min_token_prob=0.0)


def local_configs(dev, reps: int, cpu: bool) -> dict:
    """GPU graph-replay p50 and the oracle's CPU time (one thread, and all
    cores by row slices) for the two local-only workloads; the GPU output
    of each is compared with the oracle's."""
    import torch
    from oracle.drafter import DrafterOracle
    from oracle.pool import RowPool, default_workers
    from suffixgpu_amd import SuffixGPUDrafter, synth
    res = {}
    for name, w, kw, upd in (
            ("config1", synth.local_uniform(seed=1), CFG1, False),
            ("config2", synth.local_zipf(seed=2), CFG, True)):
        d = SuffixGPUDrafter(device=dev, **kw)
        tok = torch.from_numpy(w.tokens).to(dev)
        nt = torch.from_numpy(w.num_tokens).to(dev)
        if upd:
            samp = torch.from_numpy(w.sampled).to(dev)
            fn = lambda: d.propose_with_update(nt, tok, samp)  # noqa: E731
        else:
            fn = lambda: d.propose(nt, tok)  # noqa: E731
        p50, wall, out, _ = replay_p50(fn, reps)
        o = DrafterOracle(**kw)
        tok_o = w.tokens.copy()
        if upd:
            exp = o.propose_with_update(w.num_tokens, tok_o, w.sampled)
        else:
            exp = o.propose(w.num_tokens, tok_o)
        same = all(np.array_equal(a.cpu().numpy(), e)
                   for a, e in zip(out, exp))
        r = {"b": int(w.tokens.shape[0]), "s": int(w.tokens.shape[1]),
             "op": "propose_with_update" if upd else "propose",
             "gpu_graph_p50_us": round(p50, 3),
             "gpu_graph_wall_us": round(wall, 3),
             "matches_oracle": bool(same)}
        if cpu:
            def one():
                t = w.tokens.copy()
                if upd:
                    o.propose_with_update(w.num_tokens, t, w.sampled)
                else:
                    o.propose(w.num_tokens, t)
            r["cpu_1thread_us"] = round(cpu_times(one, 5 if upd else 20,
                                                  1 if upd else 3), 1)
            with RowPool(kw) as pool:
                def many():
                    t = w.tokens.copy()
                    if upd:
                        pool.propose_with_update(w.num_tokens, t, w.sampled)
                    else:
                        pool.propose(w.num_tokens, t)
                r["cpu_all_cores_us"] = round(cpu_times(many, 20, 3), 1)
                r["cpu_cores"] = pool.workers
        res[name] = r
        log(f"{name}: {r}")
        del d, tok
    return res


# The reference's standalone latency sweep (bench_vs_cpu.py --mode
# latency): propose() on uniform-random rows (vocab 32000, num_tokens in
# [S/2, S)), k=16, max_pattern_len=24, spec_factor 2.0, min_prob 0.1, and
# with global memory a 2^20 corpus / 2^15 delta fed 96 documents of 4096
# tokens.  Its published L20 graph-mode ms/step (RESULTS.md §4):
REF_SWEEP_GRAPH_MS = {
    (False, 4096): (0.10, 0.11, 0.13, 0.16),
    (False, 16384): (0.14, 0.15, 0.15, 0.23),
    (True, 4096): (0.34, 0.38, 0.44, 0.65),
    (True, 16384): (0.38, 0.42, 0.46, 0.74),
}
SWEEP_B = (1, 8, 32, 128)


def latency_sweep(dev, reps: int) -> list:
    import torch
    from suffixgpu_amd import SuffixGPUDrafter
    rng = np.random.default_rng(0)
    kw = dict(k=16, max_pattern_len=24, max_spec_factor=2.0,
              min_token_prob=0.1, global_capacity=1 << 20,
              delta_capacity=1 << 15)
    rows = []
    for glob in (False, True):
        d = SuffixGPUDrafter(device=dev, enable_global=glob,
                             rebuild_stream=torch.cuda.Stream(dev), **kw)
        if glob:
            gi = d.global_index
            gi.blocking_poll = True
            docs = [torch.from_numpy(rng.integers(0, 32000, size=4096)).to(
                dev, torch.int32) for _ in range(96)]
            d.harvest_rows(docs, [4096] * len(docs))
            d.poll()
            torch.cuda.synchronize()
        for s in (4096, 16384):
            for i, b in enumerate(SWEEP_B):
                buf = torch.from_numpy(rng.integers(0, 32000, size=(b, s))).to(
                    dev, torch.int32)
                nt = torch.from_numpy(rng.integers(
                    s // 2, s, size=b).astype(np.int32)).to(dev)
                p50, wall, _, _ = replay_p50(lambda: d.propose(nt, buf), reps)
                rows.append({"global": glob, "s": s, "b": b,
                             "graph_p50_us": round(p50, 2),
                             "graph_wall_us": round(wall, 2),
                             "reference_l20_graph_us":
                                 REF_SWEEP_GRAPH_MS[(glob, s)][i] * 1e3})
        del d
    log("latency sweep: " + "; ".join(
        f"{'g' if r['global'] else 'l'} S={r['s']} B={r['b']}: "
        f"{r['graph_p50_us']}" for r in rows))
    return rows


def compact_index_step(dev, w, bt, ref_out, steps: int,
                       warmup: int) -> dict:
    """The same step with the index built without search tables (no key
    rows, no n-gram tables): the drafter's device memory against the
    reference's, and what the smaller footprint costs per step.  The
    drafts must equal the full index's."""
    import numpy as np
    import torch
    from suffixgpu_amd import SuffixGPUDrafter
    d = SuffixGPUDrafter(device=dev, enable_global=True,
                         global_capacity=CAPACITY, delta_capacity=DELTA_CAP,
                         rebuild_threshold=1 << 30,
                         global_search_tables=False, **CFG)
    gi = d.global_index
    gi.load_documents([torch.from_numpy(x).to(dev) for x in w.active_docs])
    gi.append_documents([torch.from_numpy(x).to(dev) for x in w.delta_docs])
    tokens0 = torch.from_numpy(bt.tokens).to(dev)
    nt = torch.from_numpy(bt.num_tokens).to(dev)
    sampled = torch.from_numpy(bt.sampled).to(dev)
    buf = tokens0.clone()
    p50, wall, out, _ = replay_p50(
        lambda: d.propose_with_update(nt, buf, sampled), steps, warmup,
        before=lambda: buf.copy_(tokens0))
    same = all(np.array_equal(a.cpu().numpy(), b)
               for a, b in zip(out[:2], ref_out[:2]))
    res = {"step_p50_us": round(p50, 3), "wall_us": round(wall, 3),
           "drafts_equal_full_index": bool(same),
           "vram": drafter_device_bytes(d, B, S)}
    del d, gi
    torch.cuda.empty_cache()
    return res


def drafter_device_bytes(d, b: int, s: int) -> dict:
    """Device memory the drafter holds (exact tensor sizes), next to the
    caller's [B, S] token buffer."""
    ws = sum(t.numel() for t in d._ws.values())
    out = {"step_workspaces": ws}
    if d.global_index is not None:
        out.update(d.global_index.device_bytes())
    total = sum(out.values())
    return {"persistent_mb": round(total / 1e6, 1),
            "by_role_mb": {k: round(v / 1e6, 2) for k, v in out.items()},
            "token_buffer_mb": round(b * s * 4 / 1e6, 1)}


def e2e_loop(dev, steps: int) -> dict:
    """Scripted decode loop (B=256, S=16384): captured propose_with_update
    per step with the sampled block and counts fed back on the device,
    16 longest rows harvested into global memory every 64 steps (device
    row indices and lengths: device-side ingest) and reset, background
    rebuilds at delta_capacity // 2 on a side stream, poll() every step."""
    import torch
    from suffixgpu_amd import SuffixGPUDrafter, synth
    t0 = time.time()
    lp = synth.decode_loop(steps=steps)
    gen_s = time.time() - t0
    side = torch.cuda.Stream(dev)
    d = SuffixGPUDrafter(device=dev, enable_global=True,
                         global_capacity=CAPACITY, delta_capacity=DELTA_CAP,
                         rebuild_threshold=DELTA_CAP // 2,
                         rebuild_stream=side, **CFG)
    gi = d.global_index
    tok = torch.from_numpy(lp.tokens).to(dev)
    nt = torch.from_numpy(lp.num_tokens).to(dev)
    samp_all = torch.from_numpy(lp.sampled).to(dev)
    samp = samp_all[0].clone()
    # New requests' rows arrive as an engine stages them: pinned host
    # buffers copied without blocking the host.
    fresh = {i: (torch.tensor(rows, dtype=torch.int64, device=dev),
                 torch.tensor(lengths, dtype=torch.int64, device=dev),
                 torch.from_numpy(new_rows).pin_memory(),
                 torch.from_numpy(new_nt).pin_memory())
             for i, (rows, lengths, new_rows, new_nt)
             in lp.harvests.items()}
    for _ in range(3):
        d.propose_with_update(nt, tok, samp)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = d.propose_with_update(nt, tok, samp)
    torch.cuda.synchronize()
    main = torch.cuda.current_stream(dev)
    evs = []
    swaps = 0
    launches = 0
    nv_log = torch.zeros(steps, lp.tokens.shape[0], dtype=torch.int32,
                         device=dev)
    tw = time.perf_counter()
    for i in range(steps):
        samp.copy_(samp_all[i])
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(main)
        graph.replay()
        e1.record(main)
        evs.append((e0, e1))
        nt.copy_(out[2])
        nv_log[i].copy_(out[1])
        if i in fresh:
            idx, lens, new_rows, new_nt = fresh[i]
            d.harvest_finished(idx, lens, tok)
            tok.index_copy_(0, idx, new_rows.to(dev, non_blocking=True))
            nt.index_copy_(0, idx, new_nt.to(dev, non_blocking=True))
        before = gi._rebuild_event
        d.poll()  # starts the build of a snapshot the device staged
        now = gi._rebuild_event
        swaps += int(before is not None and now is not before)
        launches += int(now is not None and now is not before)
    torch.cuda.synchronize()
    wall = time.perf_counter() - tw
    per = [a.elapsed_time(b) * 1e3 for a, b in evs]
    # The loop above is paced by its Python host work (copies, harvests,
    # poll), so the GPU waits for each launch and the event pairs include
    # the graph launch's host latency.  The same step replayed back to
    # back, with the host queueing ahead, gives the device time per step.
    qevs = [(torch.cuda.Event(enable_timing=True),
             torch.cuda.Event(enable_timing=True)) for _ in range(100)]
    for e0, e1 in qevs:
        e0.record(main)
        graph.replay()
        e1.record(main)
    torch.cuda.synchronize()
    queued = [a.elapsed_time(b) * 1e3 for a, b in qevs]
    return {"workload": "B=256 S=16384 k=16 nb=8 R=128, 1000-step "
                        "captured decode loop, harvest 16 rows / 64 steps "
                        "(device row indices and lengths), rebuild at "
                        "delta_capacity/2 on a side stream",
            "steps": steps, "replay_p50_us": round(statistics.median(per), 3),
            "replay_p99_us": round(float(np.percentile(per, 99)), 3),
            "queued_replay_p50_us": round(statistics.median(queued), 3),
            "wall_us_per_step": round(wall / steps * 1e6, 3),
            "mean_drafted_tokens_per_step":
                round(float(nv_log.sum().item()) / steps, 2),
            "harvests": len(lp.harvests), "rebuilds_launched": launches,
            "swaps": swaps, "active_len": gi.active_len,
            "generate_s": round(gen_s, 2),
            "vram": dict(drafter_device_bytes(d, lp.tokens.shape[0],
                                              lp.tokens.shape[1]),
                         reference_l20_persistent_mb=96.3)}


def launches_us(fn, cur, reps: int) -> float:
    """Average duration of `reps` back-to-back launches of fn on stream
    `cur`, between one pair of HIP events recorded on that stream: the
    launches queue ahead of the GPU, so the events bracket the kernels
    and the gaps between them (an event pair around every launch adds
    ~3 us to each)."""
    import torch
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    for _ in range(reps):
        fn()
    e1.record(cur)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def step_kernel_us(d, dev, tokens0, nt, sampled, reps):
    """Average duration of the fused step kernel: propose_with_update
    launched directly on the current stream `reps` times back to back
    (launches_us)."""
    import torch
    cur = torch.cuda.current_stream(dev)
    buf = tokens0.clone()
    return launches_us(lambda: d.propose_with_update(nt, buf, sampled), cur,
                       reps)


# The local step at the decode-loop shape (B=256 rows of S=16384 tokens,
# num_tokens uniform in [4096, 16384], global memory off): the shape where
# the token rows alone are 16 MiB, for a per-kernel bandwidth fraction.
C5_B, C5_S, C5_LO = 256, 16384, 4096


def c5_local(dev):
    """(drafter, tokens, counts, sampled) of the local-only B=256 S=16384
    step."""
    import torch
    from suffixgpu_amd import SuffixGPUDrafter, synth
    bt = synth.local_zipf(seed=5, b=C5_B, s=C5_S, lo=C5_LO, t=T_SAMPLED)
    d = SuffixGPUDrafter(device=dev, enable_global=False, **CFG)
    return (d, torch.from_numpy(bt.tokens).to(dev),
            torch.from_numpy(bt.num_tokens).to(dev),
            torch.from_numpy(bt.sampled).to(dev))


def c5_local_step(dev, reps: int) -> dict:
    """Kernel time (HIP events, direct launches), algorithmic bytes and
    the HBM roofline fraction of the local step at B=256, S=16384."""
    d, tok, nt, sampled = c5_local(dev)
    us = step_kernel_us(d, dev, tok, nt, sampled, reps)
    buf = tok.clone()
    _, _, new = d.propose_with_update(nt, buf, sampled)
    acc = (sampled.cpu().numpy() != -1).sum(1)
    nbytes = local_algorithmic_bytes(new.cpu().numpy(), acc, CFG["k"],
                                     C5_B, C5_S)
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"workload": f"local-only propose_with_update, B={C5_B} "
                        f"S={C5_S}, num_tokens U[{C5_LO},{C5_S}]",
            "kernel_us": round(us, 3), "algorithmic_bytes": nbytes,
            "achieved_gbps": round(gbps, 1),
            "frac": round(gbps / HBM_PEAK_GBPS, 5),
            "traffic": load_traffic("k_step_c5_local")}


# Calibration copy for the PMC passes: bitwise_not over 2^26 int32 reads
# and writes exactly 256 MiB each.
PMC_COPY_ELEMS = 1 << 26
PMC_STEP_LAUNCHES = 10
PMC_SA_BUILDS = 2
# kernels of one suffix-array build (csrc/sa_build.hip)
SA_BUILD_KERNELS = ("k_sa_", "k_rs_", "k_grp_", "k_pos_")
# what a rebuild adds after the suffix array: key rows, n-gram table
TABLE_KERNELS = ("k_rank_keys", "k_gram_")


def pmc_workload(d, w, dev) -> int:
    import torch
    from suffixgpu_amd import _lib
    src = torch.randint(0, 1 << 30, (PMC_COPY_ELEMS,), dtype=torch.int32,
                        device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    bt = w.batch
    buf = torch.from_numpy(bt.tokens).to(dev)
    nt = torch.from_numpy(bt.num_tokens).to(dev)
    sampled = torch.from_numpy(bt.sampled).to(dev)
    for _ in range(PMC_STEP_LAUNCHES):
        d.propose_with_update(nt, buf, sampled)
    torch.cuda.synchronize()
    from suffixgpu_amd.suffix_array import (build_suffix_array_rounds,
                                            read_build_state,
                                            sa_workspace_bytes)
    flat = np.concatenate([np.append(x, -2) for x in w.active_docs]).astype(
        np.int32)
    m = min(flat.shape[0] + 1, CAPACITY)
    text = torch.full((CAPACITY,), _lib_pad(), dtype=torch.int32, device=dev)
    text[:flat.shape[0]].copy_(torch.from_numpy(flat))
    out = torch.empty(CAPACITY, dtype=torch.int32, device=dev)
    ws = torch.empty(sa_workspace_bytes(CAPACITY), dtype=torch.uint8,
                     device=dev)
    build_suffix_array_rounds(text, m, out, ws, 40)
    torch.cuda.synchronize()
    prev = read_build_state(ws, m)
    needed, radix = prev.needed, prev.radix_mask & ~1
    from suffixgpu_amd.global_index import KEY_WIDTH, gram_slots_for
    L = _lib.lib()
    keys = torch.empty(CAPACITY * KEY_WIDTH, dtype=torch.int32, device=dev)
    slots = gram_slots_for(CAPACITY)
    gram = torch.zeros(int(L.sfx_gram_table_bytes(slots)), dtype=torch.uint8,
                       device=dev)
    st = _lib.stream_of(dev)
    for _ in range(PMC_SA_BUILDS):
        build_suffix_array_rounds(text, m, out, ws, needed + 2, radix,
                                  needed + 1)
        # the key rows and n-gram table the index builds after it
        _lib.check(L.sfx_sa_keys(text.data_ptr(), out.data_ptr(), CAPACITY,
                                 m, KEY_WIDTH, keys.data_ptr(),
                                 ws.data_ptr(), st), "keys")
        _lib.check(L.sfx_gram_build(ws.data_ptr(), 4, m, gram.data_ptr(),
                                    slots, st), "gram")
    torch.cuda.synchronize()
    del keys, gram
    c5d, c5t, c5n, c5s = c5_local(dev)
    for _ in range(PMC_STEP_LAUNCHES):
        c5d.propose_with_update(c5n, c5t, c5s)
    torch.cuda.synchronize()
    log(f"pmc workload done: 3 calibration copies of {PMC_COPY_ELEMS * 4} "
        f"bytes, {PMC_STEP_LAUNCHES} step launches, {PMC_SA_BUILDS} SA "
        f"rebuilds of m={m} ({needed + 2} rounds) with key rows and "
        "n-gram table")
    return 0


SYNC_CHECK_STEPS = 20


def sync_check(d, w, dev) -> int:
    """Host-side API calls of the step, for a HIP API trace: eager
    propose_with_update calls, then replays of one captured step, each
    section bracketed by device synchronisations.  The step itself must
    make no synchronising call and no device-to-host copy."""
    import torch
    bt = w.batch
    buf = torch.from_numpy(bt.tokens).to(dev)
    nt = torch.from_numpy(bt.num_tokens).to(dev)
    sampled = torch.from_numpy(bt.sampled).to(dev)
    for _ in range(3):
        d.propose_with_update(nt, buf, sampled)
    torch.cuda.synchronize()
    for _ in range(SYNC_CHECK_STEPS):
        d.propose_with_update(nt, buf, sampled)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        d.propose_with_update(nt, buf, sampled)
    graph.replay()
    torch.cuda.synchronize()
    for _ in range(SYNC_CHECK_STEPS):
        graph.replay()
    torch.cuda.synchronize()
    # Device-side ingest: harvest_finished with device rows and lengths
    # (16 rows of the batch per call); the first call uploads the host
    # doc-length lists, then the timed section must read nothing back.
    rows = torch.arange(16, device=dev)
    lengths = nt[:16].clone()
    d.harvest_finished(rows, lengths, buf)
    torch.cuda.synchronize()
    for _ in range(SYNC_CHECK_STEPS):
        d.harvest_finished(rows, lengths, buf)
    torch.cuda.synchronize()
    log(f"sync check done: {SYNC_CHECK_STEPS} eager steps, "
        f"{SYNC_CHECK_STEPS} graph replays, {SYNC_CHECK_STEPS} device "
        "harvests")
    return 0


# HIP API calls that block the host on the device or copy to the host.
_BLOCKING = ("Synchronize", "hipMemcpy", "hipEventQuery", "hipStreamQuery",
             "hipMallocHost", "hipHostMalloc", "hipMalloc", "hipFree")


def summarize_api(trace_dir: str) -> dict:
    """Per section of a --sync-check run (the spans between consecutive
    hipDeviceSynchronize calls of the main thread), the HIP API calls made,
    and which of them would block or allocate."""
    import csv
    from collections import Counter
    files = sorted(Path(trace_dir).rglob("*hip_api_trace.csv"))
    if not files:
        raise SystemExit(f"no hip_api_trace.csv under {trace_dir}")
    calls = []
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                calls.append((int(r["Start_Timestamp"]), r["Thread_Id"],
                              r["Function"]))
    calls.sort()
    syncs = [c for c in calls if c[2] == "hipDeviceSynchronize"]
    main_tid = Counter(c[1] for c in syncs).most_common(1)[0][0]
    seq = [c for c in calls if c[1] == main_tid]
    marks = [i for i, c in enumerate(seq) if c[2] == "hipDeviceSynchronize"]
    sections = []
    for a, b in zip(marks, marks[1:]):
        hist = Counter(c[2] for c in seq[a + 1:b])
        if not hist:
            continue
        sections.append({
            "calls": dict(hist.most_common()),
            "blocking_or_allocating": sorted(
                n for n in hist if any(x in n for x in _BLOCKING))})
    # The last two sections are the timed eager calls and the replays
    # (capture and its first replay sit between them).
    eager = [s for s in sections
             if s["calls"].get("hipExtLaunchKernel", 0)
             + s["calls"].get("hipLaunchKernel", 0)
             + s["calls"].get("hipModuleLaunchKernel", 0)
             == SYNC_CHECK_STEPS]
    replay = [s for s in sections
              if s["calls"].get("hipGraphLaunch", 0) == SYNC_CHECK_STEPS]
    # The last section: the device harvests (three ingest launches each,
    # then the nine of the delta token index's rebuild).
    harvest = [s for s in sections
               if s["calls"].get("hipLaunchKernel", 0) >= 3 * SYNC_CHECK_STEPS
               and s["calls"].get("hipLaunchKernel", 0)
               % SYNC_CHECK_STEPS == 0
               and not s["calls"].get("hipGraphLaunch", 0)]
    return {"steps_per_section": SYNC_CHECK_STEPS,
            "eager_steps": eager[-1] if eager else None,
            "graph_replays": replay[-1] if replay else None,
            "device_harvests": harvest[-1] if harvest else None,
            "sections": len(sections)}


def summarize_counters(out_dir: str) -> dict:
    """{"kernel grid=G": {"dispatches": n, counter: mean per dispatch}}
    over every counter in one rocprofv3 --pmc CSV output directory (values
    summed over the counter's instances within a dispatch)."""
    import csv
    from collections import defaultdict
    files = sorted(Path(out_dir).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {out_dir}")
    per = defaultdict(float)            # (dispatch, kernel, counter) -> sum
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                name = r["Kernel_Name"].split("(")[0].replace("void ", "")
                name += f" grid={r.get('Grid_Size', '?')}"
                per[(int(r["Dispatch_Id"]), name, r["Counter_Name"])] += \
                    float(r["Counter_Value"])
    agg = defaultdict(lambda: defaultdict(list))
    for (disp, name, ctr), v in per.items():
        agg[name][ctr].append(v)
    out = {}
    for name, ctrs in sorted(agg.items()):
        n = max(len(v) for v in ctrs.values())
        out[name] = {"dispatches": n}
        out[name].update({c: round(sum(v) / len(v), 1)
                          for c, v in sorted(ctrs.items())})
    return out


def _pmc_rows(out_dir: str, counter: str):
    """(kernel name, value) per dispatch of one counter from a rocprofv3
    --pmc CSV output directory."""
    import csv
    files = sorted(Path(out_dir).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {out_dir}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r.get("Counter_Name") == counter:
                    rows.append((int(r.get("Dispatch_Id", len(rows))),
                                 r["Kernel_Name"],
                                 float(r["Counter_Value"])))
    rows.sort()
    return [(k, v) for _, k, v in rows]


def summarize_pmc(fetch_dir: str, write_dir: str) -> dict:
    """HBM bytes per step launch from FETCH_SIZE / WRITE_SIZE (KiB per
    dispatch), each scaled by what it reads for the calibration copy of
    known size (256 MiB read, 256 MiB written)."""
    known = PMC_COPY_ELEMS * 4
    out = {}
    for name, d_, counter in (("fetch", fetch_dir, "FETCH_SIZE"),
                              ("write", write_dir, "WRITE_SIZE")):
        rows = _pmc_rows(d_, counter)
        cal = [v for k, v in rows if "bitwise_not" in k]
        # the first PMC_STEP_LAUNCHES step launches are the B=64 global-on
        # step; the B=256 S=16384 local step launches k_local_wide (one
        # 1024-thread workgroup per row)
        steps = [v for k, v in rows if "k_step" in k]
        step = steps[:PMC_STEP_LAUNCHES]
        c5 = [v for k, v in rows if "k_local_wide" in k]
        # SA builds in dispatch order, each starting with k_sa_range; the
        # last PMC_SA_BUILDS are the rebuilds as the index runs them
        builds: list[list[float]] = []
        tables: list[list[float]] = []
        for k, v in rows:
            if "k_sa_range" in k:
                builds.append([])
                tables.append([])
            if builds and any(p in k for p in SA_BUILD_KERNELS):
                builds[-1].append(v)
            if tables and any(p in k for p in TABLE_KERNELS):
                tables[-1].append(v)
        if not cal or not step or len(builds) < PMC_SA_BUILDS:
            raise SystemExit(f"{counter}: calibration, k_step or SA build "
                             "dispatches missing")
        cal_b = statistics.median(cal) * 1024.0
        scale = known / cal_b
        step_b = statistics.mean(step) * 1024.0
        sa_b = statistics.mean(
            sum(b) for b in builds[-PMC_SA_BUILDS:]) * 1024.0
        c5_b = statistics.mean(c5) * 1024.0 if c5 else 0.0
        tab_b = statistics.mean(
            sum(b) for b in tables[-PMC_SA_BUILDS:]) * 1024.0
        out[name] = {"counter": counter, "calibration_bytes": cal_b,
                     "scale": scale, "step_raw_bytes": step_b,
                     "step_bytes": step_b * scale,
                     "dispatches": len(step),
                     "sa_build_bytes": sa_b * scale,
                     "c5_local_dispatches": len(c5),
                     "c5_local_bytes": c5_b * scale,
                     "rebuild_tables_bytes": tab_b * scale}
    total = out["fetch"]["step_bytes"] + out["write"]["step_bytes"]
    sa_total = out["fetch"]["sa_build_bytes"] + out["write"]["sa_build_bytes"]
    c5_total = out["fetch"]["c5_local_bytes"] + out["write"]["c5_local_bytes"]
    tab_total = (out["fetch"]["rebuild_tables_bytes"]
                 + out["write"]["rebuild_tables_bytes"])
    return {"k_step": round(total), "sa_rebuild": round(sa_total),
            "rebuild_tables": round(tab_total),
            "k_step_c5_local": round(c5_total) or None, "detail": out}


def row_tails(counts, rows, P):
    """Each row's last min(count, P) tokens, left-aligned in a [B, P]
    int32 tensor (zero after them), and those lengths as int64: the query
    form of the global kernel, for timing it and counting its bytes."""
    import torch
    q = counts.to(torch.int64)
    n = q.clamp(max=P)
    j = torch.arange(P, device=rows.device, dtype=torch.int64)
    src = (q - n).unsqueeze(1) + j.unsqueeze(0)
    keep = j.unsqueeze(0) < n.unsqueeze(1)
    vals = rows.gather(1, src.clamp(0, rows.shape[1] - 1))
    return (torch.where(keep, vals, torch.zeros_like(vals)).to(torch.int32)
            .contiguous(), n.contiguous())


def kernel_timings(d, dev, tokens0, nt, sampled, reps):
    """Average duration of the local and the global kernel, each launched
    alone on the current stream (launches_us)."""
    import torch

    from suffixgpu_amd import _lib
    L = _lib.lib()
    cur = torch.cuda.current_stream(dev)
    b = tokens0.shape[0]
    buf = tokens0.clone()
    bt, keep = _lib.make_batch(buf, nt, sampled=sampled,
                               limit=tokens0.shape[1])
    draft = torch.empty(b, d.k, dtype=torch.int32, device=dev)
    nv = torch.empty(b, dtype=torch.int32, device=dev)
    newc = torch.empty(b, dtype=torch.int32, device=dev)
    p_local = _lib.make_params(d.k, d.max_pattern_len,
                               d.local_kernel.max_occurrences,
                               d.local_kernel.min_match_len,
                               d.local_kernel.support_thresholds, (),
                               d.max_spec_factor, d.max_spec_offset,
                               d.min_token_prob, d.vote_smoothing_alpha)

    def local_launch():
        _lib.check(L.sfx_propose_step(p_local, None, bt, draft.data_ptr(),
                                      nv.data_ptr(), newc.data_ptr(), None,
                                      0, cur.cuda_stream), "local")

    # the global kernel, query form: tails of the updated rows
    upd = tokens0.clone()
    new = d.update_state(nt, upd, sampled)
    tails, tail_len = row_tails(new, upd, d.max_pattern_len)
    gi = d.global_index
    caps = [int(x) for x in d._global_caps.tolist()]
    pg = _lib.make_params(d.k, d.max_pattern_len, gi.max_occurrences, 1,
                          (1,), caps, d.max_spec_factor, d.max_spec_offset,
                          d.min_token_prob, d.vote_smoothing_alpha)
    outs = {n: torch.empty(sh, dtype=dt, device=dev) for n, sh, dt in (
        ("draft", (b, d.k), torch.int32), ("emit", (b,), torch.int64),
        ("draft_len", (b,), torch.int64), ("draft_occ", (b,), torch.int64),
        ("draft_score", (b,), torch.float32))}
    go = _lib.SfxGlobalOut()
    for n, t in outs.items():
        setattr(go, n, t.data_ptr())
    nbytes = int(L.sfx_global_query_workspace_size(pg, b,
                                                    gi.delta_capacity))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    ix = gi.index_struct()

    def global_launch():
        _lib.check(L.sfx_global_query(pg, ix, tails.data_ptr(), b,
                                      tails.shape[1], tail_len.data_ptr(),
                                      go, ws.data_ptr(), nbytes,
                                      cur.cuda_stream), "global")

    res = [launches_us(fn, cur, reps) for fn in (local_launch, global_launch)]
    del keep
    return res[0], res[1]


def global_algorithmic_bytes(d, dev, buf, new_counts):
    """4*delta_len + 4*|SA ranks| + 4*|corpus positions| the reference's
    search and continuation gathers must read for this batch."""
    import torch
    gi = d.global_index
    P = d.max_pattern_len
    q = torch.from_numpy(new_counts.astype(np.int64)).to(dev)
    tails, tail_len = row_tails(q, buf, P)
    res = gi._run_query(tails, tail_len, P, d._global_caps,
                        want=("len", "occ", "sa_start", "sa_end", "sa_len",
                              "d_len"))
    sa = gi.sa.cpu().numpy()
    corpus = gi.corpus.cpu().numpy()
    tl = tail_len.cpu().numpy()
    tn = tails.cpu().numpy().astype(np.int64)
    rpat = np.zeros((tn.shape[0], P), np.int64)
    for j in range(P):
        idx = tl - 1 - j
        rpat[:, j] = np.where(idx >= 0, tn[np.arange(tn.shape[0]),
                                           np.clip(idx, 0, P - 1)], -3)
    u_sa, u_c = reference_probe_footprint(sa, corpus, rpat, np.minimum(tl, P),
                                          P)
    u_sa = set(u_sa.tolist())
    u_c = set(u_c.tolist())
    ml = res["len"].cpu().numpy()
    sl = res["sa_len"].cpu().numpy()
    dl = res["d_len"].cpu().numpy()
    s0 = res["sa_start"].cpu().numpy()
    s1 = res["sa_end"].cpu().numpy()
    R, K, N = gi.max_occurrences, gi.k, gi.capacity
    for b in range(ml.shape[0]):
        for c in range(ml.shape[1]):
            if ml[b, c] == 0 or not (sl[b, c] >= dl[b, c] and sl[b, c] > 0):
                continue
            ilen = int(s1[b, c] - s0[b, c])
            cnt = min(ilen, R)
            for r in range(cnt):
                idx = (int(s0[b, c]) + (r * ilen) // R if ilen > R
                       else int(s0[b, c]) + r)
                u_sa.add(idx)
                p0 = int(sa[idx]) + int(ml[b, c])
                u_c.update(range(p0, min(p0 + K, N)))
    a = 4 * gi.delta_len + 4 * len(u_sa) + 4 * len(u_c)
    return int(a), {"delta_len": gi.delta_len, "u_sa": len(u_sa),
                    "u_corpus": len(u_c)}


def load_traffic(kernel: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(kernel)
    except (OSError, ValueError):
        return None


def cpu_baseline(d, w, steps, gpu_out):
    """The oracle (numpy restatement of the reference's CPU path) timed on
    this host on the same batch and index state: every host core (row
    slices in worker processes, `steps` steps after 3) and one thread (a
    few steps).  The index arrays are the GPU-built ones, loaded into the
    oracle (its own builds are checked by the config parity tests); the
    first CPU step is compared with the GPU step."""
    from oracle.drafter import DrafterOracle
    from oracle.pool import RowPool
    gi = d.global_index
    kw = dict(enable_global=True, global_capacity=CAPACITY,
              delta_capacity=DELTA_CAP, rebuild_threshold=1 << 30, **CFG)
    index = {"corpus": gi.corpus.cpu().numpy(), "sa": gi.sa.cpu().numpy(),
             "delta": gi.delta[:gi.delta_len].cpu().numpy(),
             "active_len": gi.active_len, "delta_len": gi.delta_len}
    o = DrafterOracle(**kw)
    og = o.global_index
    og.corpus[:] = index["corpus"]
    og.sa[:] = index["sa"]
    og.delta[:gi.delta_len] = index["delta"]
    og.active_len = gi.active_len
    og.delta_len = gi.delta_len
    bt = w.batch
    tok = bt.tokens.copy()
    first = o.propose_with_update(bt.num_tokens, tok, bt.sampled)
    same = all(np.array_equal(a, b) for a, b in zip(first, gpu_out))

    def one():
        o.propose_with_update(bt.num_tokens, bt.tokens.copy(), bt.sampled)
    one_us = cpu_times(one, 3, 0)
    with RowPool(kw, index=index) as pool:
        def many():
            pool.propose_with_update(bt.num_tokens, bt.tokens.copy(),
                                     bt.sampled)
        us = cpu_times(many, steps, 3)
        cores = pool.workers
    log(f"cpu baseline: {us / 1e3:.1f} ms/step on {cores} cores, "
        f"{one_us / 1e3:.1f} ms/step on one thread; matches GPU: {same}")
    return {"value": round(us, 1), "unit": "us/step", "cores": cores,
            "kind": "port",
            "sample": f"{steps} propose_with_update steps of the same B=64 "
                      "batch and index (the numpy oracle, rows split over "
                      f"{cores} worker processes), after 3 warm-up steps; "
                      f"host has {os.cpu_count()} logical CPUs",
            "one_thread_us": round(one_us, 1),
            "matches_gpu_step": bool(same)}


if __name__ == "__main__":
    sys.exit(main())
