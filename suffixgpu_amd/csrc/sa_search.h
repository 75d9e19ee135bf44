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

// Key-row comparison of a group's G probes at once (G % 8 == 0, keys not
// NULL).  Instruction i loads the rows of probes i * G/8 .. + G/8 - 1, one
// 16-byte part per lane: lanes 8s .. 8s + 7 of the group read probe
// i * G/8 + s's row, so each load instruction of the wave touches one
// line per 8 lanes.  (With one row per lane it touched 64 lines, and the
// CU's vector L1 serves the distinct lines of an instruction one after
// another: the waves of a workgroup then queued behind each other, about
// 0.4 us apart.)  Two ballots per instruction give every row's first
// differing token and its sign; each lane keeps its own probe's result
// (probe gl: instruction gl / (G/8), octet gl % (G/8)) and finishes it in
// the corpus when the pattern is longer than the row and the row ties.
// pc holds pattern tokens 4 * (gl % 8) .. + 3.  probe_of(q) is probe q's
// rank.  Returns -1 / 0 / +1 for the lane's own probe.
template <int G, class ProbeFn, class PatFn>
__device__ __forceinline__ int cmp_probes_key(
    const int32_t* __restrict__ keys, int kw,
    const int32_t* __restrict__ sa, const int32_t* __restrict__ corpus,
    int64_t n, ProbeFn probe_of, const int32_t (&pc)[4], PatFn pat_at,
    int plen) {
  constexpr int kParts = 8;             // 16-byte parts of a 128-byte row
  constexpr int kRows = G / kParts;     // rows per load instruction
  constexpr int kInstr = G / kRows;     // load instructions per round
  static_assert(G % kParts == 0, "whole rows per group");
  const int ln = lane_id();
  const int gl = ln % G;
  const int gbase = ln - gl;
  const int part = gl % kParts;
  const int sub = gl / kParts;
  const int kn = plen < kw ? plen : kw;
  const bool live = 4 * part < kn;
  int4 v[kInstr];
#pragma unroll
  for (int i = 0; i < kInstr; ++i) {
    v[i] = make_int4(0, 0, 0, 0);
    if (live) {
      const int64_t pr = probe_of(i * kRows + sub);
      v[i] = reinterpret_cast<const int4*>(keys + pr * kw)[part];
    }
  }
  int cv = 0;
#pragma unroll
  for (int i = 0; i < kInstr; ++i) {
    const int32_t t4[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
    bool mis = false, neg = false;
#pragma unroll
    for (int j = 3; j >= 0; --j) {  // the lowest differing token wins
      if (live && 4 * part + j < kn && t4[j] != pc[j]) {
        mis = true;
        neg = t4[j] < pc[j];
      }
    }
    const uint64_t bm = ballot(mis);
    const uint64_t bn = ballot(mis && neg);
    const int ob = gbase + kParts * (gl % kRows);  // own probe's octet
    const uint32_t seg = (uint32_t)(bm >> ob) & 0xffu;
    const int lb = seg ? __builtin_ctz(seg) : 0;
    const bool nb = (bn >> (ob + lb)) & 1ull;
    const int r = seg == 0 ? 0 : (nb ? -1 : 1);
    cv = i == gl / kRows ? r : cv;
  }
  if (cv != 0 || plen <= kw) return cv;
  const int64_t pos = sa[probe_of(gl)];
  for (int j = kw; j < plen; ++j) {
    const int64_t idx = pos + j;
    const int32_t t = idx < n ? corpus[idx] : -1;
    const int32_t pj = pat_at(j);
    if (t != pj) return t < pj ? -1 : 1;
  }
  return 0;
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
  constexpr bool kCoop = G % 8 == 0;  // rows read by lane octets
  int32_t pt[kCoop ? 4 : 32];
  if (keys) {
    // cooperative: pattern tokens 4 * (gl % 8) .. + 3; else all of them
    const int j0 = kCoop ? 4 * (gl % 8) : 0;
#pragma unroll
    for (int j = 0; j < (kCoop ? 4 : 32); ++j)
      pt[j] = j0 + j < plen ? pat_at(j0 + j) : 0;
  }
  uint32_t lo1 = r0, hi1 = r1, lo2 = r0, hi2 = r1;
  while (lo1 < hi1 || lo2 < hi2) {
    const bool shared = lo1 == lo2 && hi1 == hi2;
    const bool only1 = !shared && lo2 == hi2;
    const bool only2 = !shared && lo1 == hi1;
    const bool split = !shared && !only1 && !only2;
    // G probes over the one live range, or G/2 per bound once they split
    const uint32_t c = split ? cH : cG;
    const int np = split ? H : G;
    // probe q of the group (lane q's own probe)
    auto probe_of = [&](int q) -> int64_t {
      const bool uh = split && q >= H;
      const bool u2 = only2 || uh;
      const int kq = uh ? q - H : q;
      return (int64_t)kary_at(u2 ? lo2 : lo1, u2 ? hi2 : hi1,
                              (uint32_t)(kq + 1) * c);
    };
    int cv;
    if constexpr (kCoop) {
      cv = keys ? cmp_probes_key<G>(keys, kw, sa, corpus, n, probe_of, pt,
                                    pat_at, plen)
                : cmp_suffix(sa, corpus, n, probe_of(gl), pat_at, plen);
    } else {
      cv = keys ? cmp_suffix_key(keys, kw, sa, corpus, n, probe_of(gl), pt,
                                 pat_at, plen)
                : cmp_suffix(sa, corpus, n, probe_of(gl), pat_at, plen);
    }
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
