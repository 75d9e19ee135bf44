// Suffix-array interval search by a group of G lanes (k-ary search).
//
// The reference resolves each bound with ceil(log2(n+1)) dependent binary
// probes, each an SA read followed by corpus reads (suffix_gpu/
// sa_search.py:66-107).  Here G lanes probe G ranks of the current range
// at once, so one round of loads cuts the range (G+1)-fold; lower and
// upper bound share their probes until their ranges separate, then each
// gets G/2 lanes.  With a key array (the first kw tokens of every rank's
// suffix, built with the suffix array) a probe is a single row load.  Only
// the exact bounds are returned, which is all the reference's result
// depends on.
#pragma once

#include "sfx_common.h"

namespace sfx {

// -1 / 0 / +1: suffix at sa[rank] < pattern / starts with it / > pattern.
// Corpus reads at or past n compare as -1 (sa_search.py:25-63).
template <class PatFn>
__device__ __forceinline__ int cmp_suffix(const int32_t* __restrict__ sa,
                                          const int32_t* __restrict__ corpus,
                                          int64_t n, int64_t rank,
                                          PatFn pat_at, int plen) {
  const int64_t pos = sa[rank];
  for (int j0 = 0; j0 < plen; j0 += 4) {
    int32_t t[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t idx = pos + j0 + u;
      t[u] = idx < n ? corpus[idx > 0 ? idx : 0] : -1;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + u;
      if (j >= plen) return 0;
      const int32_t pj = pat_at(j);
      if (t[u] != pj) return t[u] < pj ? -1 : 1;
    }
  }
  return 0;
}

// The same comparison from the rank's key row: keys[rank * kw + j] holds
// corpus[sa[rank] + j] (or -1 past the end) for j < kw, so patterns of up
// to kw tokens are decided by one row load (kw * 4 bytes, one line for
// kw = 32); longer patterns continue in the corpus.  pt holds the first
// min(plen, 32) pattern tokens in registers, so the token loop waits on
// nothing but the row.
template <class PatFn>
__device__ __forceinline__ int cmp_suffix_key(
    const int32_t* __restrict__ keys, int kw,
    const int32_t* __restrict__ sa, const int32_t* __restrict__ corpus,
    int64_t n, int64_t rank, const int32_t (&pt)[32], PatFn pat_at,
    int plen) {
  const int4* row = reinterpret_cast<const int4*>(keys + rank * kw);
  const int kn = plen < kw ? plen : kw;
  int4 w[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    if (4 * q < kn) w[q] = row[q];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int t4[4] = {w[q].x, w[q].y, w[q].z, w[q].w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = 4 * q + u;
      if (j >= kn) break;
      if (t4[u] != pt[j]) return t4[u] < pt[j] ? -1 : 1;
    }
  }
  if (plen <= kw) return 0;
  const int64_t pos = sa[rank];
  for (int j = kw; j < plen; ++j) {
    const int64_t idx = pos + j;
    const int32_t t = idx < n ? corpus[idx] : -1;
    const int32_t pj = pat_at(j);
    if (t != pj) return t < pj ? -1 : 1;
  }
  return 0;
}

// Probe k of a range [lo, hi) cut by NP probes: lo + floor((hi - lo) *
// (k + 1) c / 2^32) with c = floor(2^32 / (NP + 1)), one 32x32->64
// multiply (ranks stay below 2^31).  kc = (k + 1) c < 2^32, so the probes
// ascend with k and stay below hi, which is all the search needs.
__device__ __forceinline__ uint32_t kary_at(uint32_t lo, uint32_t hi,
                                            uint32_t kc) {
  return lo + (uint32_t)(((uint64_t)(hi - lo) * kc) >> 32);
}

// Narrow [lo, hi] (answer inside; ranks < lo false, >= hi true) with the
// predicate bits of np probes of scale c (bit k = probe k true).
__device__ __forceinline__ void kary_narrow(uint32_t& lo, uint32_t& hi,
                                            uint32_t bits, int np,
                                            uint32_t c) {
  const int k = bits ? __builtin_ctz(bits) : np;  // first true probe
  const uint32_t nlo = k > 0 ? kary_at(lo, hi, (uint32_t)k * c) + 1 : lo;
  const uint32_t nhi = bits ? kary_at(lo, hi, (uint32_t)(k + 1) * c) : hi;
  lo = nlo;
  hi = nhi;
}

// Exact lower bound (first rank with cmp >= 0) and upper bound (first rank
// with cmp > 0) of one pattern.  Called by all G lanes of an aligned group
// with identical arguments; returns the bounds on every lane of the group.
// keys (kw = key width, 4 <= kw <= 32, kw % 4 == 0) may be NULL: then the
// comparison reads sa and the corpus.  n < 2^31.  The search runs inside
// [r0, r1], which must hold both bounds (every rank below r0 compares
// below the pattern, every rank from r1 on above it); [0, n] always does.
//
// The groups of a wave are in different phases (both bounds on one range,
// one bound left, or the bounds split), so each lane's probe and both
// bounds' updates are computed for every phase with selects: no phase
// branches for the wave to run one after another.
template <int G, class PatFn>
__device__ __forceinline__ void kary_bounds(
    const int32_t* __restrict__ sa, const int32_t* __restrict__ corpus,
    int64_t n, const int32_t* __restrict__ keys, int kw, PatFn pat_at,
    int plen, int64_t& lower, int64_t& upper, uint32_t r0, uint32_t r1) {
  static_assert(G >= 2 && G <= 32 && (64 % G) == 0, "group size");
  constexpr int H = G / 2;
  constexpr uint32_t cG = (uint32_t)((1ull << 32) / (G + 1));
  constexpr uint32_t cH = (uint32_t)((1ull << 32) / (H + 1));
  const int ln = lane_id();
  const int gl = ln % G;
  const int gbase = ln - gl;
  int32_t pt[32];
  if (keys) {
#pragma unroll
    for (int j = 0; j < 32; ++j) pt[j] = j < plen ? pat_at(j) : 0;
  }
  uint32_t lo1 = r0, hi1 = r1, lo2 = r0, hi2 = r1;
  while (lo1 < hi1 || lo2 < hi2) {
    const bool shared = lo1 == lo2 && hi1 == hi2;
    const bool only1 = !shared && lo2 == hi2;
    const bool only2 = !shared && lo1 == hi1;
    const bool split = !shared && !only1 && !only2;
    // G probes over the one live range, or G/2 per bound once they split
    const bool upper_half = split && gl >= H;
    const bool use2 = only2 || upper_half;
    const uint32_t c = split ? cH : cG;
    const int np = split ? H : G;
    const int k = upper_half ? gl - H : gl;
    const int64_t probe = (int64_t)kary_at(use2 ? lo2 : lo1, use2 ? hi2 : hi1,
                                           (uint32_t)(k + 1) * c);
    const int cv =
        keys ? cmp_suffix_key(keys, kw, sa, corpus, n, probe, pt, pat_at,
                              plen)
             : cmp_suffix(sa, corpus, n, probe, pat_at, plen);
    const uint64_t m1 = ballot(cv >= 0);
    const uint64_t m2 = ballot(cv > 0);
    const uint32_t full = G == 32 ? 0xffffffffu : ((1u << G) - 1u);
    const uint32_t half = (1u << H) - 1u;
    const uint32_t g1 = (uint32_t)(m1 >> gbase) & full;
    const uint32_t g2 = (uint32_t)(m2 >> gbase) & full;
    uint32_t l1 = lo1, h1 = hi1, l2 = lo2, h2 = hi2;
    kary_narrow(l1, h1, split ? (g1 & half) : g1, np, c);
    kary_narrow(l2, h2, split ? ((g2 >> H) & half) : g2, np, c);
    if (!only2) {
      lo1 = l1;
      hi1 = h1;
    }
    if (!only1) {
      lo2 = l2;
      hi2 = h2;
    }
  }
  lower = lo1;
  upper = lo2;
}

}  // namespace sfx
