// Global-role device code: SA-search and delta-scan workgroups per query
// row, and the merge run by whichever of the two finishes second.
// Included by global.hip (standalone kernel) and step.hip (fused step).
#pragma once

#include "gram.h"
#include "pick.h"
#include "sa_search.h"
#include "sfx_common.h"
#include "step_ws.h"

namespace sfx {

constexpr int kGlobalThreads = 512;
constexpr int kSearchGroup = 16;

struct GlobalArgs {
  sfx_params p;
  sfx_index ix;
  int64_t B;
  int step;
  sfx_batch bt;
  const int32_t* query;
  int64_t qwidth;
  const int64_t* qlen;
  sfx_global_out out;
  int need_expand;
  int32_t* draft;
  int32_t* num_valid;
  StepWs ws;
  int merge_waves;
  int mb_lds;  // bytes of LDS for a delta part's match lengths (0: workspace)
  int dparts;  // delta workgroups per row (delta_parts_for)
  int dchunk;  // delta positions staged in LDS at a time (0: kDeltaChunk)
  int dend;    // step: the parts' end lists are copied into LDS at the join
};

struct GlobalLayout {
  int rpat, lb, ub, found, scan, red, misc, lo, ulo, umap, dlen, dcnt, dpc,
      dmap,
      sal, sas, sae, caps, pre, dtok, dmb, mpos, mcache, mA, mH, dend, chain,
      nv, score, rlen, rocc, total;
};

// Delta tokens staged per chunk, at least (after a halo of P rounded up to
// 4 tokens): the host grows the chunk while the layout fits, up to a whole
// part; a part's match_back bytes stay in LDS up to kMbLdsMax positions,
// longer parts keep them in the workspace.
constexpr int kDeltaChunk = 8192;
constexpr int kMbLdsMax = (int)kDeltaMbLdsMax;
// With the delta token index: match lengths of this many bucket entries
// stay in LDS at a time (longer buckets are compacted chunk by chunk).
constexpr int kDixList = 16384;

__host__ __device__ inline int g_take(int& off, int bytes) {
  const int o = off;
  off += (bytes + 15) & ~15;
  return o;
}

// Shared header, then a union: the SA/delta role buffers are dead by the
// time the block (if it arrives second) merges the row.
// dparts > 0 (decode step): the merge side also holds every delta part's
// end lists, copied in at the parts' join.
// dindex: the delta role reads the delta token index; dtok then holds the
// bucket entries' match lengths and dmb their compacted list indices.
__host__ __device__ inline GlobalLayout global_layout(int P, int C, int R,
                                                      int K, int nmw,
                                                      int mb_lds,
                                                      int dchunk = 0,
                                                      int dparts = 0,
                                                      int dindex = 0) {
  constexpr int NW = kGlobalThreads / kWave;
  const int Rp = (R + 3) & ~3;
  GlobalLayout L;
  int off = 0;
  L.rpat = g_take(off, P * 4);
  L.lb = g_take(off, P * 8);
  L.ub = g_take(off, P * 8);
  L.found = g_take(off, C * 4);
  L.scan = g_take(off, 2 * 4 * NW * 8);
  L.red = g_take(off, NW * 4);
  L.misc = g_take(off, 64);
  L.lo = g_take(off, C * 4);
  L.ulo = g_take(off, (C + 1) * 4);
  L.umap = g_take(off, C * 4);
  L.dlen = g_take(off, C * 4);
  L.dcnt = g_take(off, C * 4);
  L.dpc = g_take(off, C * kMaxDeltaParts * 4);
  L.dmap = g_take(off, C * kMaxDeltaParts * 4);
  L.sal = g_take(off, C * 4);
  L.sas = g_take(off, C * 4);
  L.sae = g_take(off, C * 4);
  L.caps = g_take(off, C * 4);
  L.pre = g_take(off, C * 4);
  L.chain = g_take(off, C * K * 4);
  L.nv = g_take(off, C * 4);
  L.score = g_take(off, C * 4);
  L.rlen = g_take(off, C * 4);
  L.rocc = g_take(off, C * 4);
  const int ubase = off;
  if (dindex) {
    L.dtok = g_take(off, kDixList);
    L.dmb = g_take(off, C * R * 4);
  } else {
    L.dtok = g_take(off, ((dchunk > 0 ? dchunk : kDeltaChunk) +
                          ((P + 3) & ~3)) * 4);
    L.dmb = g_take(off, mb_lds);
  }
  const int delta_end = off;
  off = ubase;
  L.mpos = g_take(off, nmw * Rp * 4);
  L.mcache = g_take(off, nmw * R * (K + 1) * 4);
  L.mA = g_take(off, nmw * Rp * 4);
  L.mH = g_take(off, nmw * 2 * kHashSlots * 4);
  L.dend = g_take(off, dparts * C * R * 4);
  L.total = off > delta_end ? off : delta_end;
  return L;
}

// Stage x(c0 - halo) .. x(cend - 2) of the delta into dtok as 16-byte
// words.  Words wholly inside the delta go from memory straight into LDS
// (global_load_lds_dwordx4: no registers, so every load of the chunk is in
// flight at once); the edge words -- before position 0 (-1) or past the
// capacity (0) -- are formed here.  The caller waits for the loads
// (wait_all_loads) and syncs the block before reading dtok.
// Waves from `wfirst` on issue the loads (a wave's loads complete in
// order, so waves that load anything they need sooner stay out of it).
__device__ __forceinline__ void delta_stage(const GlobalArgs& a,
                                            int32_t* dtok, int64_t c0,
                                            int64_t cend, int halo,
                                            int wfirst = 0) {
  const int64_t D = a.ix.delta_capacity;
  const int64_t j0 = c0 - halo;
  const int nk4 = (int)((cend - 1 - j0 + 3) / 4);
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  if (wv < wfirst) return;
  const int4* d4 = reinterpret_cast<const int4*>(a.ix.delta);
  const int stride = kGlobalThreads - wfirst * kWave;
  for (int w0 = (wv - wfirst) * kWave; w0 < nk4; w0 += stride) {
    const int w = w0 + ln;  // one wave covers 64 consecutive words
    const int64_t j = j0 + 4 * (int64_t)w;
    if (w < nk4) {
      if (j >= 0 && j + 3 < D) {
        __builtin_amdgcn_global_load_lds(
            (const void*)(d4 + (j >> 2)),
            (__attribute__((address_space(3))) void*)(dtok + 4 * w0), 16, 0,
            0);
      } else {
        int4 v;
        v.x = j < 0 ? -1 : (j < D ? a.ix.delta[j] : 0);
        v.y = j + 1 < 0 ? -1 : (j + 1 < D ? a.ix.delta[j + 1] : 0);
        v.z = j + 2 < 0 ? -1 : (j + 2 < D ? a.ix.delta[j + 2] : 0);
        v.w = j + 3 < 0 ? -1 : (j + 3 < D ? a.ix.delta[j + 3] : 0);
        reinterpret_cast<int4*>(dtok)[w] = v;
      }
    }
  }
}

// Every load this wave issued has landed (memory-to-LDS ones included).
__device__ __forceinline__ void wait_all_loads() {
  __builtin_amdgcn_s_waitcnt(0);
}

// A delta part's chunk of positions [c0, c0 + dchunk) clipped to phi.
__device__ __forceinline__ int64_t delta_chunk_end(const GlobalArgs& a,
                                                   int64_t c0, int64_t phi) {
  const int64_t ch = a.dchunk > 0 ? a.dchunk : kDeltaChunk;
  return c0 + ch < phi ? c0 + ch : phi;
}

// [plo, phi) of this row's delta part `part` over the live delta.
__device__ __forceinline__ void delta_part_of(const GlobalArgs& a, int part,
                                              int64_t* plo, int64_t* phi) {
  const int64_t D = a.ix.delta_capacity;
  int64_t dl = *a.ix.delta_len;
  dl = dl < 0 ? 0 : (dl > D ? D : dl);
  delta_part_range(dl + 1, a.dparts, part, plo, phi);
}

// The part's thresholds min(part_max, cap) per cap (lo[c]), numbered by
// distinct value in cap order: list u serves every cap with umap[c] = u,
// ulo[u] is its threshold and ulo[C] the number of lists.  Caps are
// non-increasing (the drafter's cap set), so equal thresholds are adjacent
// and wave 0 numbers the distinct ones with one ballot; any other cap
// order takes thread 0's search.  The caller syncs the block after it.
__device__ __forceinline__ void delta_thresholds(const int32_t* caps, int C,
                                                 int part_max, int32_t* lo,
                                                 int32_t* ulo,
                                                 int32_t* umap) {
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  if (wv == 0) {
    const int t = ln < C ? min(part_max, caps[ln]) : 0;
    const int tp = __shfl_up(t, 1);
    const bool sorted = ballot(ln > 0 && ln < C && t > tp) == 0ull;
    if (sorted) {
      const bool fresh = ln < C && (ln == 0 || t != tp);
      const uint64_t fm = ballot(fresh);
      if (ln < C) {
        const int u = rank_lt(fm) + (fresh ? 0 : -1);
        lo[ln] = t;
        umap[ln] = u;
        if (fresh) ulo[u] = t;
      }
      if (ln == 0) ulo[C] = popc(fm);
    } else if (ln == 0) {
      int nu = 0;
      for (int c = 0; c < C; ++c) {
        const int tc = min(part_max, caps[c]);
        lo[c] = tc;
        int u = 0;
        while (u < nu && ulo[u] != tc) ++u;
        if (u == nu) ulo[nu++] = tc;
        umap[c] = u;
      }
      ulo[C] = nu;
    }
  }
}

// ---- Delta role with the delta token index (one workgroup per row): the
// ends i = q + 1 for the positions q in the bucket of the newest pattern
// token rpat[0] (sfx_delta_index_build), ascending -- and end 0 when that
// token is -1, since x(j) = -1 before position 0 -- are the only ends
// whose match length can be nonzero.  Each entry's match length compares
// the delta in memory with the pattern, eight tokens a step (an entry of
// another token in the bucket stops at the first); then the same ordered
// pass as the scan extracts the first R ends per distinct threshold from
// the entries' match lengths, and the entries' list indices are mapped to
// their ends (global_index.py:465-546 computes the same lengths over
// every end).
__device__ __forceinline__ void delta_role_indexed(const GlobalArgs& a,
                                                   const GlobalLayout& L,
                                                   unsigned char* smem,
                                                   int b,
                                                   const int32_t* rpat) {
  constexpr int NT = kGlobalThreads;
  constexpr int NW = NT / kWave;
  const sfx_params& p = a.p;
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int ln = tid % kWave;
  const int P = p.max_pattern_len;
  const int C = p.num_caps;
  const int R = p.max_occurrences;
  const int64_t D = a.ix.delta_capacity;
  int32_t* found = (int32_t*)(smem + L.found);
  uint32_t* scan = (uint32_t*)(smem + L.scan);
  int32_t* red = (int32_t*)(smem + L.red);
  int32_t* lo_lds = (int32_t*)(smem + L.lo);
  uint8_t* lmb = (uint8_t*)(smem + L.dtok);
  int32_t* lend = (int32_t*)(smem + L.dmb);
  const int64_t slot = b;  // one part per row
  int64_t dl64 = *a.ix.delta_len;
  dl64 = dl64 < 0 ? 0 : (dl64 > D ? D : dl64);
  const int dl = (int)dl64;  // the index covers at most 2^30 positions
  const int hb = __builtin_ctzll((unsigned long long)a.ix.delta_buckets);
  const int32_t r0 = rpat[0];
  const uint32_t bk = delta_bucket(r0, hb);
  const uint32_t s0 = a.ix.delta_start[bk];
  const uint32_t s1 = a.ix.delta_start[bk + 1];
  const int has0 = r0 == -1 ? 1 : 0;
  const int n = (int)(s1 > s0 ? s1 - s0 : 0) + has0;
  const int4* ent = reinterpret_cast<const int4*>(a.ix.delta_entries) + s0;
  const int32_t* delta = a.ix.delta;
  // Entry j: {q, x(q), x(q - 1), x(q - 2)} for the end q + 1; entry 0 is
  // the end 0 (q = -1) when has0.
  auto entry = [&](int j) -> int4 {
    return has0 ? (j == 0 ? make_int4(-1, -1, -1, -1) : ent[j - 1]) : ent[j];
  };
  // The match length of the end after q, continuing from m leading
  // matches: x(q - m) .. x(q - m - 3) against rpat[m ..], four independent
  // loads a step; x(j) = -1 before position 0.
  auto mb_from = [&](int q, int m) -> int {
    while (m < P) {
      int32_t x[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = q - m - k;
        x[k] = j >= 0 ? delta[j] : -1;
      }
      int n4 = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        n4 += (n4 == k && m + k < P && x[k] == rpat[m + k]) ? 1 : 0;
      m += n4;
      if (n4 < 4) break;
    }
    return m;
  };
  // Match lengths of entries jb + u * NT + tid (u < 4) of [.., j1) into
  // lmb[j - lbase] (where below kDixList): the four entries -- position
  // and first three tokens each -- are loaded together, and only entries
  // matching all three walk on in the delta.  Returns the largest length.
  auto mb4 = [&](int jb, int j1, int lbase) -> int {
    int4 e[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = jb + u * NT + tid;
      e[u] = j < j1 ? entry(j) : make_int4(dl, 0, 0, 0);
    }
    int mx4 = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      // (q >= dl: past the delta, or an index for a longer delta)
      int m = e[u].x >= dl
                  ? 0
                  : (e[u].y != r0 ? 0
                                  : (P < 2 || e[u].z != rpat[1]
                                         ? 1
                                         : (P < 3 || e[u].w != rpat[2] ? 2
                                                                       : 3)));
      if (m == 3 && P > 3) m = mb_from(e[u].x, 3);
      const int j = jb + u * NT + tid;
      if (j < j1 && j - lbase < kDixList) lmb[j - lbase] = (uint8_t)m;
      mx4 = max(mx4, m);
    }
    return mx4;
  };
  // Match lengths of the first chunk of entries (kept for the compaction
  // when the bucket fits it) and the largest over all entries.
  int mx = 0;
  for (int jb = 0; jb < n; jb += 4 * NT) mx = max(mx, mb4(jb, n, 0));
  mx = (int)wave_all_max((uint32_t)mx);
  if (ln == 0) red[wv] = mx;
  __syncthreads();
  int part_max = 0;
  for (int w = 0; w < NW; ++w) part_max = max(part_max, red[w]);
  SFX_TRACE_POINT(2);
  const int32_t* caps = (const int32_t*)(smem + L.caps);
  int32_t* ulo = (int32_t*)(smem + L.ulo);
  int32_t* umap = (int32_t*)(smem + L.umap);
  delta_thresholds(caps, C, part_max, lo_lds, ulo, umap);
  __syncthreads();
  const int nu = ulo[C];
  if (n <= kDixList) {
    for (int g0 = 0; g0 < nu; g0 += 8)
      compact_first_r<NT>(lmb, n, ulo + g0, min(8, nu - g0), R,
                          lend + g0 * R, 0, found + g0, scan, (g0 >> 3) & 1);
  } else {
    // Chunks of entries in order, their match lengths computed again, with
    // the kept counts carried; done once every list holds R.
    for (int u = tid; u < nu; u += NT) found[u] = 0;
    for (int j0 = 0; j0 < n; j0 += kDixList) {
      const int cnt = n - j0 < kDixList ? n - j0 : kDixList;
      __syncthreads();  // the previous chunk's compaction read lmb
      for (int jb = j0; jb < j0 + cnt; jb += 4 * NT) mb4(jb, j0 + cnt, j0);
      __syncthreads();
      for (int g0 = 0; g0 < nu; g0 += 8)
        compact_first_r<NT, true>(lmb, cnt, ulo + g0, min(8, nu - g0), R,
                                  lend + g0 * R, j0, found + g0, scan,
                                  (g0 >> 3) & 1);
      __syncthreads();
      bool open = false;
      for (int u = 0; u < nu; ++u) open |= ulo[u] > 0 && found[u] < R;
      if (!open) break;
    }
  }
  __syncthreads();
  SFX_TRACE_POINT(3);
  // list indices -> ends, for the combine and the gather
  for (int e = tid; e < nu * R; e += NT) {
    const int u = e / R;
    if (e - u * R < found[u])
      ws_store(a.ws.d_end + (slot * C + u) * R + (e - u * R),
               entry(lend[e]).x + 1);
  }
  for (int c = tid; c < C; c += NT) {
    ws_store(a.ws.d_cnt + slot * C + c, lo_lds[c] > 0 ? found[umap[c]] : 0);
    ws_store(a.ws.d_map + slot * C + c, umap[c]);
  }
  if (tid == 0) ws_store(a.ws.d_mx + slot, part_max);
}

// ---- Delta role, one part of the row: match_back over ends i in
// [lo, hi) of 0 .. delta_len, with the delta staged through LDS in 16-byte
// words (chunks of kDeltaChunk positions after a halo of P rounded up to
// 4), kept as u8 in LDS (kMbLds) or the workspace; then one ordered pass
// extracts the part's first R ends per cap with mb >= min(part max, cap).
// Caps whose thresholds are equal (every cap at or above the part's
// longest match, and the repeated smallest caps) share one list, so the
// pass runs once per distinct threshold.  The merge keeps a part's list
// only where that threshold equals the row's min(max mb, cap) -- any other
// part has no end that reaches it -- and concatenates the kept lists in
// part order (global_index.py:465-546).
template <bool kMbLds>
__device__ __forceinline__ void delta_role(const GlobalArgs& a,
                                           const GlobalLayout& L,
                                           unsigned char* smem, int b,
                                           int part, const int32_t* rpat) {
  constexpr int NT = kGlobalThreads;
  constexpr int NW = NT / kWave;
  const sfx_params& p = a.p;
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int ln = tid % kWave;
  const int P = p.max_pattern_len;
  const int C = p.num_caps;
  const int R = p.max_occurrences;
  const int KD = a.dparts;
  const int64_t D = a.ix.delta_capacity;
  int32_t* found = (int32_t*)(smem + L.found);
  uint32_t* scan = (uint32_t*)(smem + L.scan);
  int32_t* red = (int32_t*)(smem + L.red);
  int* misc = (int*)(smem + L.misc);
  int32_t* lo_lds = (int32_t*)(smem + L.lo);
  int32_t* dtok = (int32_t*)(smem + L.dtok);
  const int64_t slot = (int64_t)b * KD + part;
  uint8_t* mb = kMbLds ? (uint8_t*)(smem + L.dmb)
                       : a.ws.d_mb + slot * delta_mb_stride(
                                                delta_part_cap(D, KD));
  int64_t plo, phi;
  delta_part_of(a, part, &plo, &phi);
  const int halo = (P + 3) & ~3;
  const int32_t r0 = rpat[0];
  const int32_t r1 = P > 1 ? rpat[1] : 0;
  const int32_t r2 = P > 2 ? rpat[2] : 0;
  const int32_t r3 = P > 3 ? rpat[3] : 0;
  int mx = 0;
  // The first chunk's loads were issued before the row setup (global_body)
  // so that their latency overlaps it; each later chunk is staged after
  // the previous one's scan.
  for (int64_t c0 = plo; c0 < phi; ) {
    const int64_t cend = delta_chunk_end(a, c0, phi);
    if (c0 != plo) delta_stage(a, dtok, c0, cend, halo);
    wait_all_loads();
    __syncthreads();
    // Ends i0 .. i0 + 3 (i0 = c0 + 4g) from two 16-byte LDS reads, which
    // give x(i0 - 4) .. x(i0 + 3) (the halo is at least 4): the four
    // newest pattern tokens are tested at every end without a branch, and
    // only ends matching all four walk further back, four tokens a step.
    const int ng = (int)((cend - c0 + 3) / 4);
    for (int g = tid; g < ng; g += NT) {
      const int k = 4 * g + halo;  // dtok index of x(i0)
      const int4 lo4 = reinterpret_cast<const int4*>(dtok)[(k >> 2) - 1];
      const int4 hi4 = reinterpret_cast<const int4*>(dtok)[k >> 2];
      // w[j] = x(i0 - 4 + j); end i0 + u reads x(i0 + u - 1 - t) =
      // w[3 + u - t] for pattern token t
      const int32_t w[8] = {lo4.x, lo4.y, lo4.z, lo4.w,
                            hi4.x, hi4.y, hi4.z, hi4.w};
      const int64_t i0 = c0 + 4 * (int64_t)g;
      uint32_t word = 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool e0 = i0 + u < cend && w[3 + u] == r0;
        const bool e1 = e0 && P > 1 && w[2 + u] == r1;
        const bool e2 = e1 && P > 2 && w[1 + u] == r2;
        const bool e3 = e2 && P > 3 && w[u] == r3;
        int m = (int)e0 + (int)e1 + (int)e2 + (int)e3;
        if (e3 && P > 4) {
          const int base = k - 1 + u;  // dtok index of x(i - 1)
          while (m < P) {
            int32_t x4[4], p4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int j = base - m - e;
              x4[e] = j >= 0 ? dtok[j] : -1;
              p4[e] = rpat[m + e < P ? m + e : P - 1];
            }
            int n4 = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              n4 += (n4 == e && m + e < P && x4[e] == p4[e]) ? 1 : 0;
            m += n4;
            if (n4 < 4) break;
          }
        }
        word |= (uint32_t)m << (8 * u);
        mx = max(mx, m);
      }
      *reinterpret_cast<uint32_t*>(mb + (i0 - plo)) = word;
    }
    __syncthreads();
    c0 = cend;
  }
  // match lengths are >= 0: the unsigned DPP max is the signed one
  mx = (int)wave_all_max((uint32_t)mx);
  if (ln == 0) red[wv] = mx;
  __syncthreads();
  int part_max = 0;
  for (int w = 0; w < NW; ++w) part_max = max(part_max, red[w]);
  SFX_TRACE_POINT(2);
  const int32_t* caps = (const int32_t*)(smem + L.caps);
  int32_t* ulo = (int32_t*)(smem + L.ulo);
  int32_t* umap = (int32_t*)(smem + L.umap);
  delta_thresholds(caps, C, part_max, lo_lds, ulo, umap);
  __syncthreads();
  const int nu = ulo[C];
  for (int g0 = 0; g0 < nu; g0 += 8)
    compact_first_r<NT, false, true>(
        mb, phi - plo, ulo + g0, min(8, nu - g0), R,
        a.ws.d_end + (slot * C + g0) * R, (int32_t)plo, found + g0, scan,
        (g0 >> 3) & 1);
  __syncthreads();
  SFX_TRACE_POINT(3);
  for (int c = tid; c < C; c += NT) {
    ws_store(a.ws.d_cnt + slot * C + c, lo_lds[c] > 0 ? found[umap[c]] : 0);
    ws_store(a.ws.d_map + slot * C + c, umap[c]);
  }
  if (tid == 0) ws_store(a.ws.d_mx + slot, part_max);
}

// Row-level delta result per cap from the parts (run by the merging
// workgroup): dlen[c] = min(max mb, cap), dpc[c][k] = part k's kept hits,
// dcnt[c] = min(sum, R), dmap[c][k] = part k's list index for cap c.
__device__ __forceinline__ void delta_combine(const GlobalArgs& a, int b,
                                              const int32_t* caps,
                                              int32_t* dlen, int32_t* dcnt,
                                              int32_t* dpc, int32_t* dmap) {
  const int C = a.p.num_caps;
  const int R = a.p.max_occurrences;
  const int KD = a.dparts;
  for (int c = threadIdx.x; c < C; c += blockDim.x) {
    const int cap = caps[c];
    // every part's maximum and count in one round of loads (the parts
    // wrote them from other workgroups: each read goes past this L2)
    int pmx[kMaxDeltaParts], pcnt[kMaxDeltaParts], pmap[kMaxDeltaParts];
    int mx = 0;
#pragma unroll
    for (int k = 0; k < kMaxDeltaParts; ++k) {
      const int64_t slot = (int64_t)b * KD + k;
      pmx[k] = k < KD ? a.ws.d_mx[slot] : 0;
      pcnt[k] = k < KD ? a.ws.d_cnt[slot * C + c] : 0;
      pmap[k] = k < KD ? a.ws.d_map[slot * C + c] : 0;
      mx = max(mx, pmx[k]);
    }
    const int lo = min(mx, cap);
    int total = 0;
#pragma unroll
    for (int k = 0; k < kMaxDeltaParts; ++k) {
      if (k >= KD) break;
      const bool keep = lo > 0 && min(pmx[k], cap) == lo;
      const int h = keep ? pcnt[k] : 0;
      dpc[c * kMaxDeltaParts + k] = h;
      dmap[c * kMaxDeltaParts + k] = pmap[k];
      total += h;
    }
    dlen[c] = lo;
    dcnt[c] = total < R ? total : R;
  }
}

// End position of the row's r-th delta hit for cap c (r < dcnt[c]).
__device__ __forceinline__ int32_t delta_end_at(const GlobalArgs& a, int b,
                                                int c, int r,
                                                const int32_t* dpc) {
  const int C = a.p.num_caps;
  const int R = a.p.max_occurrences;
  const int KD = a.dparts;
  int k = 0;
  while (k < KD - 1 && r >= dpc[c * kMaxDeltaParts + k]) {
    r -= dpc[c * kMaxDeltaParts + k];
    ++k;
  }
  const int64_t slot = (int64_t)b * KD + k;
  return a.ws.d_end[(slot * C + a.ws.d_map[slot * C + c]) * R + r];
}

// Position of the r-th SA sample of the interval [s, s + ilen): stride
// ilen / R when it is longer than R (global_index.py:339-352).
__device__ __forceinline__ int32_t sa_sample(const GlobalArgs& a, int64_t s,
                                             int64_t ilen, int r) {
  const int R = a.p.max_occurrences;
  const int64_t N = a.ix.capacity;
  int64_t idx = ilen > R ? s + ((int64_t)r * ilen) / R : s + r;
  idx = idx < 0 ? 0 : (idx > N - 1 ? N - 1 : idx);
  return a.ix.sa[idx];
}

// One wave: the continuation block of one candidate (src 1: the SA
// interval [sa_s, sa_s + ilen), sampled with stride ilen / R when longer
// than R (global_index.py:339-352); src 2: the row's delta ends minus len)
// gathered into LDS -- tokens in range, not PAD, not negative, else -1
// (:443-463) -- optionally copied to cont_out [R, K], then (expand) the
// majority-vote expansion into chain_out.
// slot: the wave whose LDS areas hold the block (-1: the calling wave's);
// gathered: the block is already there (an early gather), only expand.
__device__ __forceinline__ ExpandResult gather_expand(
    const GlobalArgs& a, const GlobalLayout& L, unsigned char* smem, int b,
    int c, int src, int len, int occ, int64_t sa_s, int64_t ilen,
    const int32_t* dpc, int32_t* cont_out, bool expand, int32_t* chain_out,
    const int32_t* dend = nullptr, int slot = -1, bool gathered = false) {
  const sfx_params& p = a.p;
  const int ln = lane_id();
  const int wv = slot >= 0 ? slot : (int)(threadIdx.x / kWave);
  const int R = p.max_occurrences;
  const int K = p.k;
  const int Rp = (R + 3) & ~3;
  const int64_t N = a.ix.capacity;
  const int64_t D = a.ix.delta_capacity;
  int32_t* mpos = (int32_t*)(smem + L.mpos) + wv * Rp;
  int32_t* mcache = (int32_t*)(smem + L.mcache) + (int64_t)wv * R * (K + 1);
  // delta: each part's list index for this cap, read with the parts'
  // counts by delta_combine (one dependent load per hit here)
  const int32_t* dmap = (const int32_t*)(smem + L.dmap) + c * kMaxDeltaParts;
  const int Kp = K + 1;
  if (!gathered) {
    for (int r = ln; r < occ; r += kWave) {
      int32_t pos;
      if (src == 1) {
        pos = sa_sample(a, sa_s, ilen, r);
      } else {
        int k = 0, rr = r;
        while (k < a.dparts - 1 && rr >= dpc[c * kMaxDeltaParts + k]) {
          rr -= dpc[c * kMaxDeltaParts + k];
          ++k;
        }
        const int m = dmap[k];
        const int64_t slot = (int64_t)b * a.dparts + k;
        // the end lists: copied into LDS at the parts' join (dend), or read
        // from the workspace
        const int32_t end_r =
            dend ? dend[(k * p.num_caps + m) * R + rr]
                 : a.ws.d_end[(slot * p.num_caps + m) * R + rr];
        const int64_t e = (int64_t)end_r - len;
        pos = (int32_t)(e < 0 ? 0 : e);
      }
      mpos[r] = pos;
    }
    wave_lds_sync();
    SFX_TRACE_POINT(10);
    const int32_t* srcbuf = src == 1 ? a.ix.corpus : a.ix.delta;
    const int64_t nbuf = src == 1 ? N : D;
    int64_t slen = N;
    if (src == 2) {
      slen = *a.ix.delta_len;
      slen = slen < 0 ? 0 : (slen > D ? D : slen);
    }
    // One occurrence row per lane: its K tokens are independent loads.  Rows
    // are K + 1 words apart in LDS (an odd stride), so the lanes' reads and
    // writes of one depth fall in distinct banks.
    for (int r = ln; r < occ; r += kWave) {
      const int64_t base = (int64_t)mpos[r] + len;
      int32_t* dst = mcache + r * Kp;
      for (int j0 = 0; j0 < K; j0 += 16) {
        int32_t v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int64_t idx = base + j0 + u;
          v[u] = -1;
          if (j0 + u < K && idx < slen && idx >= 0)
            v[u] = srcbuf[idx < nbuf - 1 ? idx : nbuf - 1];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u)
          if (j0 + u < K)
            dst[j0 + u] = (v[u] != kPad && v[u] >= 0) ? v[u] : -1;
      }
    }
  }
  wave_lds_sync();
  SFX_TRACE_POINT(11);
  if (cont_out)
    for (int e = ln; e < R * K; e += kWave)
      cont_out[e] = e < occ * K ? mcache[(e / K) * Kp + e % K] : -1;
  ExpandResult er{0, 0.0f};
  if (expand) {
    const int64_t cap = spec_cap(p, len);
    auto cont_at = [&](int r, int d) -> int32_t { return mcache[r * Kp + d]; };
    er = expand_wave<false>(cont_at, NoWeight(), R, occ, K, cap,
                            p.min_token_prob, p.alpha,
                            (int32_t*)(smem + L.mA) + wv * Rp, nullptr,
                            (int32_t*)(smem + L.mH) + wv * 2 * kHashSlots,
                            chain_out);
  }
  SFX_TRACE_POINT(12);
  return er;
}

// Decode step: expansions of one source's candidate for every cap
// (src 1: SA, lens/s/e per cap in LDS; src 2: delta, lens/counts per cap
// and the per-part hit counts).  Caps with the same length share one
// candidate, so each run of equal lengths is expanded once (one wave per
// run) and its result written for every cap of the run to nv/score/chain
// [B,C(,K)] in the workspace.  Called by the whole block.
__device__ __forceinline__ void source_expand(
    const GlobalArgs& a, const GlobalLayout& L, unsigned char* smem, int b,
    int src, const int32_t* lens, const int32_t* aux0, const int32_t* aux1,
    const int32_t* dpc, int32_t* nv_out, float* score_out,
    int32_t* chain_out, const int32_t* needed = nullptr,
    const int32_t* pre = nullptr) {
  const sfx_params& p = a.p;
  const int C = p.num_caps;
  const int R = p.max_occurrences;
  const int K = p.k;
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  const int nmw = a.merge_waves;
  int32_t* chain = (int32_t*)(smem + L.chain);
  for (int c = wv; c < C && wv < nmw; c += nmw) {
    const int len = lens[c];
    if (c > 0 && lens[c - 1] == len) continue;  // expanded by the run head
    int end = c + 1;
    while (end < C && lens[end] == len) ++end;
    if (needed) {  // no cap of the run can pick this candidate
      bool any = false;
      for (int cc = c; cc < end; ++cc) any = any || needed[cc] != 0;
      if (!any) continue;
    }
    ExpandResult er{0, 0.0f};
    if (len > 0) {
      int occ;
      int64_t s0 = 0, ilen = 0;
      if (src == 1) {
        s0 = aux0[c];
        ilen = (int64_t)aux1[c] - s0;
        occ = (int)(ilen < R ? ilen : R);
      } else {
        occ = aux0[c];
      }
      er = gather_expand(a, L, smem, b, c, src, len, occ, s0, ilen, dpc,
                         nullptr, true, chain + c * K,
                         src == 2 && a.dend
                             ? (const int32_t*)(smem + L.dend)
                             : nullptr,
                         -1, pre && pre[c] == len);
    }
    wave_lds_sync();  // lane 0 wrote the chain
    for (int cc = c; cc < end; ++cc) {
      const int64_t i = (int64_t)b * C + cc;
      for (int d = ln; d < K; d += kWave)
        if (d < er.nv) ws_store(chain_out + i * K + d, chain[c * K + d]);
      if (ln == 0) {
        ws_store(nv_out + i, er.nv);
        ws_store(score_out + i, er.score);
      }
    }
  }
}

// The key rows the index's selector word names (sfx_index.key_select).
// A nonzero selector names the second buffer, which may be NULL: no key
// rows while they are being rebuilt.
__device__ __forceinline__ const int32_t* live_keys(const sfx_index& ix) {
  if (ix.key_select && *ix.key_select != 0) return ix.sa_key_alt;
  return ix.sa_key;
}

// The n-gram range table of the live suffix array, or NULL.
__device__ __forceinline__ const void* live_gram(const sfx_index& ix) {
  if (ix.key_select && *ix.key_select != 0) return ix.gram_alt;
  return ix.gram;
}

// role 0: SA search; role 1 .. dparts: delta part role - 1.
// kEarly: the decode step's SA workgroup may gather short caps' blocks
// early.  Off in the streamed step kernel (rows beyond the LDS layout, as
// in the B=256 S=16384 decode loop, whose grid runs in waves with two
// workgroups per CU): there it measured slower, the loop's replay p50
// 50.4-51.0 -> 53.4-54.4 us.
template <bool kEarly = true>
__device__ __forceinline__ void global_body(const GlobalArgs& a,
                                            unsigned char* smem, int b,
                                            int role) {
  constexpr int NT = kGlobalThreads;
  constexpr int NW = NT / kWave;
  const sfx_params& p = a.p;
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int ln = tid % kWave;
  const int P = p.max_pattern_len;
  const int C = p.num_caps;
  const int R = p.max_occurrences;
  const int K = p.k;
  const int Rp = (R + 3) & ~3;
  const bool dindex = a.ix.delta_entries != nullptr;
  const GlobalLayout L =
      global_layout(P, C, R, K, a.merge_waves, a.mb_lds, a.dchunk,
                    a.dend ? a.dparts : 0, dindex ? 1 : 0);
  int32_t* rpat = (int32_t*)(smem + L.rpat);
  int64_t* lbs = (int64_t*)(smem + L.lb);
  int64_t* ubs = (int64_t*)(smem + L.ub);
  int32_t* found = (int32_t*)(smem + L.found);
  uint32_t* scan = (uint32_t*)(smem + L.scan);
  int32_t* red = (int32_t*)(smem + L.red);
  int* misc = (int*)(smem + L.misc);
  const int64_t N = a.ix.capacity;
  const int64_t D = a.ix.delta_capacity;
  SFX_TRACE_POINT(0);
  // The caps, read by thread index later (delta thresholds, combine): a
  // varying index into the kernel arguments is a vector load from device
  // memory, so it is issued once here, ahead of the first barrier.
  if (tid < C) ((int32_t*)(smem + L.caps))[tid] = p.caps[tid];
  // A delta part's first chunk goes from memory into LDS while the row's
  // pattern is read: the waves past the pattern's threads load the delta
  // length and issue it (a wave's loads complete in order, so they read
  // nothing of the row themselves); delta_role waits for it.  dtok lies
  // past the header the setup writes.
  const int wpat = (P + kWave - 1) / kWave;  // waves holding pattern threads
  auto stage_first_chunk = [&]() {
    if (role > 0 && wv >= wpat && !dindex) {
      int64_t plo, phi;
      delta_part_of(a, role - 1, &plo, &phi);
      if (plo < phi)
        delta_stage(a, (int32_t*)(smem + L.dtok), plo,
                    delta_chunk_end(a, plo, phi), (P + 3) & ~3, wpat);
    }
  };

  // Query tail, newest first: rpat[t] = tail token t back from the end;
  // -3 past the start (global_index.py:493-501).
  int64_t qlen = 0;
  if (a.step) {
    if (role > 0 && wv >= wpat && !dindex) {
      stage_first_chunk();
    } else {
      const RowState st = row_state(a.bt, b);
      if (tid == 0) misc[12] = st.mask ? 1 : 0;
      const int64_t q = st.q;
      qlen = q < P ? q : P;
      if (st.mask)
        for (int t = tid; t < P; t += NT) {
          const int64_t idx = q - 1 - t;
          int32_t v = -3;
          if (idx >= 0) {
            const int64_t x = idx < a.bt.seq - 1 ? idx : a.bt.seq - 1;
            v = updated_token(a.bt, b, st, x);
          }
          rpat[t] = v;
        }
    }
  } else {
    qlen = a.qlen[b];
    stage_first_chunk();
    const int64_t Q = a.qwidth;
    for (int t = tid; t < P; t += NT) {
      const int64_t idx = qlen - 1 - t;
      int32_t v = -3;
      if (idx >= 0) v = a.query[(int64_t)b * Q + (idx < Q - 1 ? idx : Q - 1)];
      rpat[t] = v;
    }
  }
  // (plen is read by the SA role, whose waves all read the row)
  const int plen = (int)(qlen < 0 ? 0 : (qlen < P ? qlen : P));
  __syncthreads();
  if (a.step && !misc[12]) {  // masked rows: the local kernel writes them
    wait_all_loads();  // no load into this block's LDS outlives it
    return;
  }
  SFX_TRACE_POINT(1);

  if (role == 0) {
    // ---- SA interval search for every suffix length of the tail.
    constexpr int G = kSearchGroup;
    const int ngroups = NT / G;
    const int g = tid / G;
    const int32_t* keys = live_keys(a.ix);
    // The n-gram table narrows each search to the ranks that share its
    // pattern's first min(l, kmax) tokens (the whole answer for
    // l <= kmax, the longest run length the table holds); without a
    // usable table every search spans [0, N).
    const void* gram = live_gram(a.ix);
    int kg = gram ? (int)reinterpret_cast<const GramHeader*>(gram)->kmax : 0;
    kg = kg < kGramMax ? kg : kGramMax;
    if (kg <= 0) gram = nullptr;
    for (int l = g + 1; l <= P; l += ngroups) {
      int64_t lo = 0, hi = 0;
      if (l <= plen) {
        auto pat_at = [&](int j) -> int32_t { return rpat[l - 1 - j]; };
        uint32_t r0 = 0, r1 = (uint32_t)N;
        int found = -1;
        const int k = l < kg ? l : kg;
        int32_t t[4] = {0, 0, 0, 0};
        bool real = true;
#pragma unroll
        for (int j = 0; j < kGramMax; ++j) {
          if (j < k) {
            t[j] = pat_at(j);
            real = real && gram_real(t[j]);
          }
        }
        if (gram && real)
          found = gram_lookup<G>(gram, a.ix.gram_slots, t[0], t[1], t[2],
                                 t[3], k, r0, r1);
        if (found == 0) {
          lo = hi = 0;  // no suffix starts with the first k tokens
        } else if (found == 1 && l == k) {
          lo = r0;
          hi = r1;
        } else {
          if (found != 1) {
            r0 = 0;
            r1 = (uint32_t)N;
          }
          kary_bounds<G>(a.ix.sa, a.ix.corpus, N, keys, (int)a.ix.key_width,
                         pat_at, l, lo, hi, r0, r1);
        }
      }
      if (tid % G == 0) {
        lbs[l - 1] = lo;
        ubs[l - 1] = hi;
      }
    }
    // Early gathers (decode step).  With one length per search group,
    // wave 0's groups search lengths 1 .. 4, which the n-gram table
    // answers with one lookup, and wave 0 then waits for the longest
    // searches.  Meanwhile it gathers the continuation block of one cap
    // whose candidate it already knows (cap <= the table's longest run
    // length) into the LDS area of the wave that will expand it: wave c
    // for the run of equal candidate lengths that cap c heads.  A cap
    // whose run head it cannot know yet (the cap before lies beyond the
    // table) is gathered as if it were one; pre[c] is the length gathered
    // for cap c, -1 for none.
    int32_t* pre = (int32_t*)(smem + L.pre);
    const int nmw = a.merge_waves;
    const bool early = kEarly && a.step && gram && ngroups >= P;
    if (early && wv == 0) {
      wave_lds_sync();  // this wave's groups wrote lengths 1 .. 4
      // One gather: the smallest cap's (its short candidate has the most
      // distinct continuations, the longest expansion).  A second one
      // held the block barrier past the longest searches (two gathers of
      // about 3.8 us each from 3.6 us, searches ending at 7.5-9.3 us).
      int prev = -1;  // candidate length of cap c - 1, if known
      int gc = -1, glen = 0;  // the cap to gather and its candidate length
      for (int c = 0; c < C; ++c) {
        const int cap = p.caps[c];
        int best = -1;
        if (cap <= kg) {
          const int l = ln + 1;
          const bool f = l <= kg && l <= cap && l <= plen &&
                         ubs[l - 1] > lbs[l - 1];
          const uint64_t m = ballot(f);
          best = m ? 64 - __builtin_clzll(m) : 0;
        }
        if (best > 0 && c < nmw && best != prev) {
          gc = c;
          glen = best;
        }
        if (ln == 0) pre[c] = -1;
        prev = best;
      }
      if (gc >= 0) {
        const int64_t s0 = lbs[glen - 1];
        const int64_t ilen = ubs[glen - 1] - s0;
        gather_expand(a, L, smem, b, gc, 1, glen,
                      (int)(ilen < R ? ilen : R), s0, ilen, nullptr, nullptr,
                      false, nullptr, nullptr, gc, false);
        if (ln == 0) pre[gc] = glen;
      }
    }
    __syncthreads();
    SFX_TRACE_POINT(2);
    // Each cap takes its longest non-empty interval (sa_search.py:
    // 137-163); wave w selects caps w, w + NW, ...
    int32_t* sal = (int32_t*)(smem + L.sal);
    int32_t* sas = (int32_t*)(smem + L.sas);
    int32_t* sae = (int32_t*)(smem + L.sae);
    const int32_t* capl = (const int32_t*)(smem + L.caps);  // LDS copy
    for (int c = wv; c < C; c += NW) {
      const int cap = capl[c];
      int best = 0;
      for (int base = 1; base <= P; base += kWave) {
        const int l = base + ln;
        const bool f = l <= P && l <= cap && l <= plen &&
                       ubs[l - 1] > lbs[l - 1];
        const uint64_t m = ballot(f);
        if (m) best = base + 63 - __builtin_clzll(m);
      }
      if (ln == 0) {
        const int64_t s0 = best ? lbs[best - 1] : 0;
        const int64_t e0 = best ? ubs[best - 1] : 0;
        sal[c] = best;
        sas[c] = (int32_t)s0;
        sae[c] = (int32_t)e0;
        ws_store(a.ws.sa_len + (int64_t)b * C + c, best);
        ws_store(a.ws.sa_s + (int64_t)b * C + c, (int32_t)s0);
        ws_store(a.ws.sa_e + (int64_t)b * C + c, (int32_t)e0);
        // for the delta workgroups (decode step): a word of its own per
        // cap, so a reader sees either 0 or the length, no fence needed
        if (a.step)
          ws_store(a.ws.sa_known + (int64_t)b * SFX_MAX_CANDIDATES + c,
                   best + 1);
        if (!a.step) {  // query outputs (none in a decode step)
          if (a.out.sa_len) a.out.sa_len[(int64_t)b * C + c] = best;
          if (a.out.sa_start) a.out.sa_start[(int64_t)b * C + c] = s0;
          if (a.out.sa_end) a.out.sa_end[(int64_t)b * C + c] = e0;
        }
      }
    }
    if (a.step) {
      // Decode step: expand the SA candidate of every cap now, while the
      // delta and local workgroups are still running.
      __syncthreads();
      source_expand(a, L, smem, b, 1, sal, sas, sae, nullptr,
                    a.ws.sa_nv, a.ws.sa_score, a.ws.sa_chain, nullptr,
                    early ? pre : nullptr);
      SFX_TRACE_POINT(4);
      if (block_arrive<false>(a.ws.pick + b, 3u, misc + 1))
        final_pick(p, a.ws, b, a.draft, a.num_valid, misc + 4);
      return;
    }
  } else {
    if (dindex)
      delta_role_indexed(a, L, smem, b, rpat);
    else if (a.mb_lds)
      delta_role<true>(a, L, smem, b, role - 1, rpat);
    else
      delta_role<false>(a, L, smem, b, role - 1, rpat);
    if (a.step) {
      // Decode step: the last delta part combines the parts and expands
      // the delta candidate of every cap.
      if (a.dparts > 1) {
        if (!block_arrive(a.ws.djoin + b, (unsigned)a.dparts, misc + 1))
          return;
      } else {
        __syncthreads();  // this block's own part results
      }
      SFX_TRACE_POINT(4);
      int32_t* dlen = (int32_t*)(smem + L.dlen);
      int32_t* dcnt = (int32_t*)(smem + L.dcnt);
      int32_t* dpc = (int32_t*)(smem + L.dpc);
      // Every part's end lists go into LDS in the same round of loads as
      // the parts' maxima and counts, so the gather reads its positions
      // there instead of one more dependent round from the workspace.
      const int nend = a.dend ? a.dparts * C * R : 0;
      const int32_t* ends = a.ws.d_end + (int64_t)b * a.dparts * C * R;
      int32_t* dend = (int32_t*)(smem + L.dend);
      constexpr int kPre = 4;
      int32_t pre[kPre];
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        const int e = tid + u * NT;
        pre[u] = e < nend ? ends[e] : 0;
      }
      // The SA lengths its workgroup has published so far (agent-scope
      // loads: it wrote them from another CU), with the same round.
      int sa1 = 0;
      if (tid < C)
        sa1 = __hip_atomic_load(
            a.ws.sa_known + (int64_t)b * SFX_MAX_CANDIDATES + tid,
            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      delta_combine(a, b, (const int32_t*)(smem + L.caps), dlen, dcnt, dpc,
                    (int32_t*)(smem + L.dmap));
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        const int e = tid + u * NT;
        if (e < nend) dend[e] = pre[u];
      }
      for (int e = tid + kPre * NT; e < nend; e += NT) dend[e] = ends[e];
      __syncthreads();
      // A cap's delta candidate counts only when its match is longer than
      // the SA's (global_index.py:321-325); where the SA length is known
      // and at least as long, its expansion is skipped (the pick never
      // reads it).
      int32_t* need = (int32_t*)(smem + L.found);
      for (int c = tid; c < C; c += NT) {
        ws_store(a.ws.dl_c + (int64_t)b * C + c, dlen[c]);
        need[c] = sa1 == 0 || dlen[c] > sa1 - 1;
      }
      __syncthreads();
      SFX_TRACE_POINT(5);
      source_expand(a, L, smem, b, 2, dlen, dcnt, nullptr, dpc, a.ws.dn_nv,
                    a.ws.dn_score, a.ws.dn_chain, need);
      SFX_TRACE_POINT(6);
      if (block_arrive<false>(a.ws.pick + b, 3u, misc + 2))
        final_pick(p, a.ws, b, a.draft, a.num_valid, misc + 4);
      return;
    }
  }

  // ---- Query: the last of the SA and delta workgroups merges the row.
  SFX_TRACE_POINT(4);
  if (!block_arrive(a.ws.join + b, 1u + (unsigned)a.dparts, misc + 1))
    return;
  SFX_TRACE_POINT(5);
  int32_t* dlen = (int32_t*)(smem + L.dlen);
  int32_t* dcnt = (int32_t*)(smem + L.dcnt);
  int32_t* dpc = (int32_t*)(smem + L.dpc);
  delta_combine(a, b, (const int32_t*)(smem + L.caps), dlen, dcnt, dpc,
                (int32_t*)(smem + L.dmap));
  __syncthreads();
  if (a.out.d_len || a.out.d_cnt)
    for (int c = tid; c < C; c += NT) {
      if (a.out.d_len) a.out.d_len[(int64_t)b * C + c] = dlen[c];
      if (a.out.d_cnt) a.out.d_cnt[(int64_t)b * C + c] = dcnt[c];
    }
  if (a.out.d_pos)
    for (int e = tid; e < C * R; e += NT) {
      const int c = e / R;
      const int r = e % R;
      int64_t v = 0;
      if (r < dcnt[c]) v = (int64_t)delta_end_at(a, b, c, r, dpc) - dlen[c];
      a.out.d_pos[((int64_t)b * C + c) * R + r] = v < 0 ? 0 : v;
    }

  const int nmw = a.merge_waves;
  int32_t* chain = (int32_t*)(smem + L.chain);
  int32_t* res_nv = (int32_t*)(smem + L.nv);
  float* res_score = (float*)(smem + L.score);
  int32_t* res_len = (int32_t*)(smem + L.rlen);
  int32_t* res_occ = (int32_t*)(smem + L.rocc);
  for (int c = wv; c < C && wv < nmw; c += nmw) {
    // Source selection per cap, before and after dedup (:321-337).
    auto pre = [&](int cc, int& len, int& src) {
      const int sl = a.ws.sa_len[(int64_t)b * C + cc];
      const int dl_c = dlen[cc];
      const bool use_sa = sl >= dl_c && sl > 0;
      const bool use_d = dl_c > sl && dl_c > 0;
      len = use_sa ? sl : (use_d ? dl_c : 0);
      src = (use_sa ? 1 : 0) + (use_d ? 2 : 0);
    };
    int len, src;
    pre(c, len, src);
    if (c > 0) {
      int plen0, psrc;
      pre(c - 1, plen0, psrc);
      if (len == plen0 && src == psrc && len > 0) {
        len = 0;
        src = 0;
      }
    }
    const int64_t sa_s = a.ws.sa_s[(int64_t)b * C + c];
    const int64_t ilen = (int64_t)a.ws.sa_e[(int64_t)b * C + c] - sa_s;
    int occ = 0;
    if (src == 1) occ = (int)(ilen < R ? ilen : R);
    if (src == 2) occ = dcnt[c];
    int32_t* cont_out =
        a.out.cont ? a.out.cont + ((int64_t)b * C + c) * R * K : nullptr;
    const ExpandResult er =
        gather_expand(a, L, smem, b, c, src, len, occ, sa_s, ilen, dpc,
                      cont_out, a.need_expand != 0, chain + c * K);
    if (ln == 0) {
      if (a.out.len) a.out.len[(int64_t)b * C + c] = len;
      if (a.out.occ) a.out.occ[(int64_t)b * C + c] = occ;
      res_nv[c] = er.nv;
      res_score[c] = er.score;
      res_len[c] = len;
      res_occ[c] = occ;
    }
  }
  if (!a.need_expand) return;
  __syncthreads();
  SFX_TRACE_POINT(6);
  // Best cap: first argmax of the raw score (global_index.py:427-436).
  if (tid == 0) {
    int best = 0;
    for (int c = 1; c < C; ++c)
      if (res_score[c] > res_score[best]) best = c;
    const int64_t cap = spec_cap(p, res_len[best]);
    const int64_t cap0 = cap > 0 ? cap : 0;
    misc[2] = best;
    misc[3] = (int)((int64_t)res_nv[best] < cap0 ? res_nv[best] : cap0);
  }
  __syncthreads();
  const int best = misc[2];
  const int emit = misc[3];
  const int32_t* bchain = chain + best * K;
  if (a.out.draft)
    for (int j = tid; j < K; j += NT)
      a.out.draft[(int64_t)b * K + j] = j < emit ? bchain[j] : -1;
  if (tid == 0) {
    if (a.out.emit) a.out.emit[b] = emit;
    if (a.out.draft_len) a.out.draft_len[b] = res_len[best];
    if (a.out.draft_occ) a.out.draft_occ[b] = res_occ[best];
    if (a.out.draft_score) a.out.draft_score[b] = res_score[best];
  }
}

}  // namespace sfx
