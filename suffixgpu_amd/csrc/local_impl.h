// Local-role device code: one 512-thread workgroup per request row.
// Included by local.hip (standalone kernel) and step.hip (fused step).
#pragma once

#include "pick.h"
#include "sfx_common.h"
#include "step_ws.h"

namespace sfx {

enum LocalMode { kLocalGather = 0, kLocalForward = 1, kLocalStep = 2 };

struct LocalArgs {
  sfx_params p;
  sfx_batch bt;
  int mode;
  int global_on;
  int64_t* cand_out;   // gather
  int32_t* cont_out;
  int64_t* occ_out;
  int32_t* draft;      // forward / step
  int32_t* num_valid;
  int64_t* len_out;    // forward
  int64_t* occ1_out;
  float* score_out;
  int32_t* new_counts;  // step
  StepWs ws;
  int chunk;  // 0: the whole row is staged in LDS; else streamed in chunks
  int mb_full;  // streamed: LDS holds the match lengths of the whole row
};

struct LocalLayout {
  int row, mb, pat, hist, cand, found, thr, scan, occ, A, H, chain, nv,
      score, misc, total;
};

__host__ __device__ inline int lds_take(int& off, int bytes) {
  const int o = off;
  off += (bytes + 15) & ~15;
  return o;
}

// compact_first_r reads whole 16-byte words of every thread's segment.
__host__ __device__ inline int mb_bytes(int n, int nthreads) {
  const int seg = (((n + nthreads - 1) / nthreads) + 15) & ~15;
  return seg * nthreads;
}

// Tokens staged ahead of a streamed chunk: the pattern length rounded up
// to a whole 16-byte word.
__host__ __device__ inline int stream_halo(int P) { return (P + 3) & ~3; }

// chunk == 0: the row (S tokens) and its match lengths live in LDS.
// chunk > 0: LDS holds one chunk of positions and the stream_halo(P)
// tokens before it, and the match lengths of that chunk (mb_full == 0) or
// of the whole row (mb_full == 1).
__host__ __device__ inline LocalLayout local_layout(int S, int P, int C,
                                                    int R, int K, int nwaves,
                                                    int chunk = 0,
                                                    int mb_full = 0) {
  const int nthreads = nwaves * kWave;
  const int span = chunk > 0 && !mb_full ? chunk : S;
  LocalLayout L;
  int off = 0;
  L.row = lds_take(off, (chunk > 0 ? chunk + stream_halo(P) : S) * 4);
  L.mb = lds_take(off, mb_bytes(span, nthreads));
  L.pat = lds_take(off, P * 4);
  L.hist = lds_take(off, (P + 1) * 4);
  L.cand = lds_take(off, C * 4);
  L.found = lds_take(off, C * 4);
  L.thr = lds_take(off, C * 4);
  L.scan = lds_take(off, 2 * 4 * nwaves * 8);
  L.occ = lds_take(off, C * R * 4);
  L.A = lds_take(off, nwaves * ((R + 3) & ~3) * 4);
  L.H = lds_take(off, nwaves * 2 * kHashSlots * 4);
  L.chain = lds_take(off, C * K * 4);
  L.nv = lds_take(off, C * 4);
  L.score = lds_take(off, C * 4);
  L.misc = lds_take(off, 64);
  L.total = off;
  return L;
}

constexpr int kLocalThreads = 512;
// The local-only decode step over rows of kWideMinSeq tokens or more runs
// one 1024-thread workgroup per row: the row scans (match lengths,
// histogram, first-R compaction) spread over 16 waves, and a CU holds one
// such row.  At B = 256, S = 16384 the step measured 33.6 us against
// 38.6 us with 512 threads; at S = 4096 it was 1.3 us slower (the row
// scans are short and the 16-wave barriers cost more), at S = 16384 and
// B <= 128 the same.
constexpr int kWideThreads = 1024;
constexpr int64_t kWideMinSeq = 8192;

// kStream: the row stays in HBM.  match_back is computed over chunks of
// a.chunk positions staged through LDS.  With a.mb_full the match lengths
// of the whole row stay in LDS and one ordered pass compacts them, as for
// a row held whole; otherwise the chunks are staged once to histogram the
// match lengths and once more, in order, to compact the first R ends per
// candidate with the counts carried from chunk to chunk (stopping once
// every candidate holds R).  The expansion reads continuations from HBM.
template <bool kStream, int NT = kLocalThreads>
__device__ __forceinline__ void local_body(const LocalArgs& a,
                                           unsigned char* smem, int b) {
  constexpr int NW = NT / kWave;
  const sfx_params& p = a.p;
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int ln = tid % kWave;
  const int S = (int)a.bt.seq;
  const int P = p.max_pattern_len;
  const int C = p.num_thresholds;
  const int R = p.max_occurrences;
  const int K = p.k;
  const bool mb_full = kStream && a.mb_full;
  const LocalLayout L = local_layout(S, P, C, R, K, NW, kStream ? a.chunk : 0,
                                     mb_full ? 1 : 0);
  int32_t* row = (int32_t*)(smem + L.row);  // the row, or a staged chunk
  uint8_t* mbuf = (uint8_t*)(smem + L.mb);
  int32_t* pat = (int32_t*)(smem + L.pat);
  int32_t* hist = (int32_t*)(smem + L.hist);
  int32_t* cand = (int32_t*)(smem + L.cand);
  int32_t* found = (int32_t*)(smem + L.found);
  int32_t* thr_lds = (int32_t*)(smem + L.thr);
  uint32_t* scan = (uint32_t*)(smem + L.scan);
  int32_t* occ = (int32_t*)(smem + L.occ);
  int32_t* Abuf = (int32_t*)(smem + L.A);
  int32_t* chain = (int32_t*)(smem + L.chain);
  int32_t* res_nv = (int32_t*)(smem + L.nv);
  float* res_score = (float*)(smem + L.score);
  int* misc = (int*)(smem + L.misc);

  SFX_TRACE_POINT(0);
  if (tid < C) thr_lds[tid] = p.thresholds[tid];
  const RowState st = row_state(a.bt, b);
  const int64_t q = st.q;

  // Stage the row, then apply this step's scatter (proposer.py:162-184).
  // Only positions below min(q, S) are ever read (match_back, pattern and
  // continuations all stop at q), so the rest of the row stays in HBM.
  int32_t* grow = a.bt.tokens + (int64_t)b * S;
  const bool vec4 = (S & 3) == 0 && (((uintptr_t)grow) & 15) == 0;
  if (!kStream) {
    const int qs = (int)(q < 0 ? 0 : (q < S ? q : S));
    if (vec4) {
      // Four 16-byte loads in flight per thread before their LDS stores.
      const int4* src = reinterpret_cast<const int4*>(grow);
      int4* dst = reinterpret_cast<int4*>(row);
      const int n4 = (qs + 3) / 4;
      int i = tid;
      for (; i + 3 * NT < n4; i += 4 * NT) {
        const int4 v0 = src[i];
        const int4 v1 = src[i + NT];
        const int4 v2 = src[i + 2 * NT];
        const int4 v3 = src[i + 3 * NT];
        dst[i] = v0;
        dst[i + NT] = v1;
        dst[i + 2 * NT] = v2;
        dst[i + 3 * NT] = v3;
      }
      for (; i < n4; i += NT) dst[i] = src[i];
    } else {
      for (int i = tid; i < qs; i += NT) row[i] = grow[i];
    }
    __syncthreads();
  }
  if (a.bt.sampled) {
    const int32_t* sp = a.bt.sampled + (int64_t)b * a.bt.num_sampled;
    for (int64_t j = tid; j < a.bt.num_sampled; j += NT) {
      const int64_t pos = st.base + j;
      const int32_t v = sp[j];
      if (j < st.cnt && v != -1 && pos < S && pos >= 0) {
        if (!kStream) row[pos] = v;
        grow[pos] = v;
      }
    }
    if (a.new_counts && tid == 0) a.new_counts[b] = (int32_t)q;
  }
  __syncthreads();

  if (a.mode == kLocalStep && !st.mask) {
    for (int j = tid; j < K; j += NT) a.draft[(int64_t)b * K + j] = -1;
    if (tid == 0) a.num_valid[b] = 0;
    return;
  }

  SFX_TRACE_POINT(1);
  // Newest-first pattern, -2 fill (local_matcher.py:103-112).
  const int32_t* src_row = kStream ? grow : row;
  for (int t = tid; t < P; t += NT) {
    const int64_t idx = q - 1 - t;
    pat[t] = idx >= 0 ? src_row[idx < S - 1 ? idx : S - 1] : -2;
  }
  for (int i = tid; i <= P; i += NT) hist[i] = 0;
  __syncthreads();

  // Streamed rows: positions 0 .. qe - 1 can match (mb is zero from q on);
  // chunk [c0, cend) stages x(c0 - halo) .. x(cend - 2), -1 before the row.
  const int CH = kStream ? a.chunk : S;
  const int halo = kStream ? stream_halo(P) : 0;
  const int qe = (int)(q < 0 ? 0 : (q < S ? q : S));
  auto stage_chunk = [&](int c0, int cend) {
    const int j0 = c0 - halo;
    const int nw = (cend - 1 - j0 + 3) / 4;
    for (int k = tid; k < nw; k += NT) {
      const int j = j0 + 4 * k;
      int4 v;
      if (vec4 && j >= 0 && j + 3 < S) {
        v = reinterpret_cast<const int4*>(grow)[j >> 2];
      } else {
        v.x = j < 0 ? -1 : (j < S ? grow[j] : 0);
        v.y = j + 1 < 0 ? -1 : (j + 1 < S ? grow[j + 1] : 0);
        v.z = j + 2 < 0 ? -1 : (j + 2 < S ? grow[j + 2] : 0);
        v.w = j + 3 < 0 ? -1 : (j + 3 < S ? grow[j + 3] : 0);
      }
      reinterpret_cast<int4*>(row)[k] = v;
    }
  };
  // match_back of positions c0 .. cend - 1 from the staged chunk.
  auto chunk_match = [&](int c0, int cend, bool count) {
    for (int i = c0 + tid; i < cend; i += NT) {
      const int k = i - 1 - (c0 - halo);  // row index of x(i - 1)
      int m = 0;
      while (m < P && row[k - m] == pat[m]) ++m;
      mbuf[mb_full ? i : i - c0] = (uint8_t)m;
      if (count && m > 0) atomicAdd(&hist[m], 1);
    }
  };

  // match_back, zero at i >= q (local_matcher.py:114-132).
  if (kStream) {
    for (int c0 = 0; c0 < qe; c0 += CH) {
      const int cend = c0 + CH < qe ? c0 + CH : qe;
      stage_chunk(c0, cend);
      __syncthreads();
      chunk_match(c0, cend, true);
      __syncthreads();
    }
  } else {
    // Four ends i0 .. i0 + 3 per thread from two 16-byte LDS reads: x(i - 1)
    // is tested against the newest pattern token first and only ends that
    // pass walk further back.  Match lengths are stored as one u32 of four
    // bytes; positions from qe on are never read (the compaction stops
    // there).  Every nonzero length adds one to the histogram with an LDS
    // atomic.
    // The first four pattern tokens are tested at every end without a
    // branch (two 16-byte reads give x(i0 - 4) .. x(i0 + 3)); only ends
    // matching all four walk further back.  On rows whose newest token is
    // frequent most ends match one token, so the walk's setup would run in
    // most waves' iterations.
    const int32_t p0 = pat[0];
    const int32_t p1 = P > 1 ? pat[1] : 0;
    const int32_t p2 = P > 2 ? pat[2] : 0;
    const int32_t p3 = P > 3 ? pat[3] : 0;
    const int4* row4 = reinterpret_cast<const int4*>(row);
    const int ng = (qe + 3) / 4;
    // Ends that match all four first tokens are queued per wave (in the
    // wave's expansion scratch, free until the expansion) and walked after
    // the scan, one per lane, so a wave pays for its longest walk rather
    // than for every group and end position that holds one.  A full queue
    // walks in place.
    constexpr int kWalkQ = 256;
    int32_t* wq = (int32_t*)(smem + L.H) + wv * 2 * kHashSlots;
    int32_t* wq_n = wq + kWalkQ;
    if (ln == 0) *wq_n = 0;
    auto walk = [&](int i) -> int {
      // Walk back four tokens per step from m = 4: the four row tokens and
      // pattern tokens of a step are independent LDS reads.
      const int base = i - 1;  // row index of x(i - 1)
      int m = 4;
      while (m < P) {
        int32_t x4[4], p4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int j = base - m - k;
          x4[k] = j >= 0 ? row[j] : -1;
          p4[k] = pat[m + k < P ? m + k : P - 1];
        }
        int k = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          k += (k == e && m + e < P && x4[e] == p4[e]) ? 1 : 0;
        m += k;
        if (k < 4) break;
      }
      return m;
    };
    for (int g = tid; g - tid < ng; g += NT) {
      uint32_t word = 0;
      uint32_t queued = 0;
      if (g < ng) {
        const int i0 = 4 * g;
        const int4 lo4 = g > 0 ? row4[g - 1] : make_int4(-1, -1, -1, -1);
        const int4 hi4 = row4[g];
        // w[k] = x(i0 - 4 + k); end i0 + u reads x(i0 + u - 1 - t) =
        // w[3 + u - t] for pattern token t
        const int32_t w[8] = {lo4.x, lo4.y, lo4.z, lo4.w,
                              hi4.x, hi4.y, hi4.z, hi4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const bool e0 = i0 + u < qe && w[3 + u] == p0;
          const bool e1 = e0 && P > 1 && w[2 + u] == p1;
          const bool e2 = e1 && P > 2 && w[1 + u] == p2;
          const bool e3 = e2 && P > 3 && w[u] == p3;
          int m = (int)e0 + (int)e1 + (int)e2 + (int)e3;
          if (e3 && P > 4) {
            const int slot = atomicAdd(wq_n, 1);
            if (slot < kWalkQ) {
              wq[slot] = i0 + u;  // walked below; m stays 4 until then
              queued |= 1u << u;
            } else {
              m = walk(i0 + u);
            }
          }
          word |= (uint32_t)m << (8 * u);
        }
        *reinterpret_cast<uint32_t*>(mbuf + i0) = word;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int m = (int)((word >> (8 * u)) & 0xffu);
        if (m > 0 && !((queued >> u) & 1u)) atomicAdd(&hist[m], 1);
      }
    }
    // The wave's queued walks (its own LDS writes: in issue order).
    wave_lds_sync();
    const int nq = min(*wq_n, kWalkQ);
    for (int k = ln; k < nq; k += kWave) {
      const int i = wq[k];
      const int m = walk(i);
      mbuf[i] = (uint8_t)m;
      atomicAdd(&hist[m], 1);
    }
    __syncthreads();
  }

  SFX_TRACE_POINT(2);
  // Candidates: thr-th largest match_back = largest L with #{mb >= L} >=
  // thr; zero below min_match_len or when masked; adjacent duplicates
  // zeroed (local_matcher.py:134-157).  Wave 0: suffix sums of the
  // histogram, then one ballot per threshold (#{mb >= L} is monotone in L,
  // so the largest qualifying L is the number of qualifying L).
  if (wv == 0) {
    // P <= 64: lane ln holds #{mb >= P - ln} in a register (one DPP scan);
    // longer patterns keep the suffix counts in hist[].
    const bool in_reg = P <= kWave;
    int sfx = 0;
    if (in_reg) {
      const int Lv = P - ln;
      sfx = (int)wave_incl_scan(Lv >= 1 ? (uint32_t)hist[Lv] : 0u);
    }
    int carry = 0;
    for (int top = in_reg ? 0 : P; top >= 1; top -= kWave) {
      const int Lv = top - ln;
      int x = Lv >= 1 ? hist[Lv] : 0;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (ln >= o) x += y;
      }
      x += carry;
      if (Lv >= 1) hist[Lv] = x;
      carry = __shfl(x, kWave - 1);
    }
    wave_lds_sync();
    // Lane c holds threshold c, copied to LDS at the start of the block
    // (a varying index into the kernel arguments is a vector load from the
    // argument segment in device memory; issued there, its latency hides
    // behind the row staging).
    const int thr_l = ln < C ? thr_lds[ln] : (int)0x80000000;
    if (in_reg) {
      // Eight thresholds per step, unrolled: each takes one ballot, and the
      // min_match_len, mask and duplicate rules are scalar selects, with no
      // branch per threshold.  A threshold above S qualifies no L.
      const int mml = p.min_match_len;
      const bool live = ln < P;
      int prev_raw = -1;
      for (int c0 = 0; c0 < C; c0 += 8) {
        int outv = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int thr = __builtin_amdgcn_readlane(thr_l, c0 + j);
          const int t = thr < 1 ? 1 : thr;
          int v = popc(ballot(live && sfx >= t));
          if (!(thr <= S && v >= mml && st.mask)) v = 0;
          const int raw = v;
          if (c0 + j > 0 && raw == prev_raw) v = 0;
          prev_raw = raw;
          outv = ln == j ? v : outv;
        }
        if (ln < 8 && c0 + ln < C) cand[c0 + ln] = outv;
      }
    } else {
      const int maxthr = (int)(wave_all_max((uint32_t)thr_l ^ 0x80000000u) ^
                               0x80000000u);
      const int w = min(maxthr, S);
      int prev_raw = -1;
      for (int c = 0; c < C; ++c) {
        const int thr = __builtin_amdgcn_readlane(thr_l, c);
        int v = 0;
        if (thr <= w) {
          const int t = thr < 1 ? 1 : thr;
          for (int base = 1; base <= P; base += kWave) {
            const int Lv = base + ln;
            v += popc(ballot(Lv <= P && hist[Lv] >= t));
          }
        }
        if (!(v >= p.min_match_len && st.mask)) v = 0;
        const int raw = v;
        if (c > 0 && raw == prev_raw) v = 0;
        prev_raw = raw;
        if (ln == 0) cand[c] = v;
      }
    }
  }
  __syncthreads();

  SFX_TRACE_POINT(3);
  // First R ascending ends per candidate (triton_kernels.py:217-243
  // semantics): one ordered pass per group of 8 candidates.
  if (!kStream || mb_full) {
    for (int g0 = 0; g0 < C; g0 += 8)
      compact_first_r<NT>(mbuf, qe, cand + g0, min(8, C - g0), R,
                          occ + g0 * R, 0, found + g0, scan, (g0 >> 3) & 1);
    __syncthreads();
  } else {
    // Chunks in ascending order; a single chunk's match lengths are still
    // in LDS from the histogram pass.
    for (int c = tid; c < C; c += NT) found[c] = 0;
    __syncthreads();
    for (int c0 = 0; c0 < qe; c0 += CH) {
      const int cend = c0 + CH < qe ? c0 + CH : qe;
      if (qe > CH) {
        stage_chunk(c0, cend);
        __syncthreads();
        chunk_match(c0, cend, false);
        __syncthreads();
      }
      for (int g0 = 0; g0 < C; g0 += 8)
        compact_first_r<NT, true>(mbuf, cend - c0, cand + g0, min(8, C - g0),
                                  R, occ + g0 * R, c0, found + g0, scan,
                                  (g0 >> 3) & 1);
      __syncthreads();
      bool open = false;
      for (int c = 0; c < C; ++c) open |= cand[c] > 0 && found[c] < R;
      if (!open) break;
    }
  }

  SFX_TRACE_POINT(4);
  if (a.mode == kLocalGather) {
    for (int c = tid; c < C; c += NT) {
      if (a.cand_out) a.cand_out[(int64_t)b * C + c] = cand[c];
      if (a.occ_out) a.occ_out[(int64_t)b * C + c] = min(found[c], R);
    }
    if (a.cont_out) {
      const int total = C * R * K;
      int32_t* out = a.cont_out + (int64_t)b * total;
      for (int e = tid; e < total; e += NT) {
        const int c = e / (R * K);
        const int r = (e / K) % R;
        const int j = e % K;
        int32_t v = -1;
        if (r < min(found[c], R)) {
          const int64_t idx = (int64_t)occ[c * R + r] + j;
          if (idx < q) v = src_row[idx < S - 1 ? idx : S - 1];
        }
        out[e] = v;
      }
    }
    return;
  }

  // One wave per candidate: majority-vote expansion from the LDS row (HBM
  // when streamed).
  for (int c = wv; c < C; c += NW) {
    const int cv = cand[c];
    const int64_t oc = cv > 0 ? (int64_t)min(found[c], R) : 0;
    const int64_t cap = spec_cap(p, cv);
    const int32_t* oc_list = occ + c * R;
    auto cont_at = [&](int r, int d) -> int32_t {
      const int64_t idx = (int64_t)oc_list[r] + d;
      return idx < q ? src_row[idx < S - 1 ? idx : S - 1] : -1;
    };
    const ExpandResult er = expand_wave<false>(
        cont_at, NoWeight(), R, oc, K, cap, p.min_token_prob, p.alpha,
        Abuf + wv * ((R + 3) & ~3), nullptr,
        (int32_t*)(smem + L.H) + wv * 2 * kHashSlots, chain + c * K);
    if (ln == 0) {
      res_nv[c] = er.nv;
      res_score[c] = er.score;
    }
    if (c < 6) SFX_TRACE_WAVE(10 + c);
  }
  __syncthreads();

  SFX_TRACE_POINT(5);
  // select_local_best (local_matcher.py:245-263).
  if (tid == 0) {
    int best = 0;
    float bkey = local_key(res_score[0], cand[0]);
    for (int c = 1; c < C; ++c) {
      const float key = local_key(res_score[c], cand[c]);
      if (key > bkey) {
        bkey = key;
        best = c;
      }
    }
    const int64_t cap = spec_cap(p, cand[best]);
    const int64_t cap0 = cap > 0 ? cap : 0;
    misc[0] = best;
    misc[1] = (int)((int64_t)res_nv[best] < cap0 ? res_nv[best] : cap0);
  }
  __syncthreads();
  const int best = misc[0];
  const int emit = misc[1];
  const int32_t* bchain = chain + best * K;

  if (a.mode == kLocalForward) {
    for (int j = tid; j < K; j += NT)
      a.draft[(int64_t)b * K + j] = j < emit ? bchain[j] : -1;
    if (tid == 0) {
      a.num_valid[b] = emit;
      if (a.len_out) a.len_out[b] = cand[best];
      if (a.occ1_out)
        a.occ1_out[b] = cand[best] > 0 ? min(found[best], R) : 0;
      if (a.score_out) a.score_out[b] = res_score[best];
    }
    return;
  }

  // Decode step.
  if (!a.global_on) {
    for (int j = tid; j < K; j += NT)
      a.draft[(int64_t)b * K + j] = j < emit ? bchain[j] : -1;
    if (tid == 0) a.num_valid[b] = emit;
    return;
  }
  for (int j = tid; j < K; j += NT)
    ws_store(a.ws.l_chain + (int64_t)b * K + j, bchain[j]);
  if (tid == 0) {
    ws_store(a.ws.l_emit + b, emit);
    ws_store(a.ws.l_score + b, res_score[best]);
  }
  if (block_arrive<false>(a.ws.pick + b, 3u, misc + 2))
    final_pick(p, a.ws, b, a.draft, a.num_valid, misc + 4);
}

// The local-only decode step with kWideThreads per row (local.hip); -1
// when its layout does not fit a CU's LDS (the caller keeps the fused
// step's 512-thread form).
int launch_local_step(LocalArgs a, hipStream_t stream);

}  // namespace sfx
