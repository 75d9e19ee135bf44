// Shared device helpers for the gfx950 drafter kernels: wave64 primitives,
// the fp32 rules of the chain score, and the wave-level majority-vote
// chain expansion used by the local, global and standalone expand paths.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "suffixgpu_amd.h"

// Phase timestamps for profiling builds (-DSFX_TRACE): thread 0 of each
// block stores wall_clock64() into sfx_trace_buf[block * 16 + slot].
#ifdef SFX_TRACE
extern __constant__ uint64_t* sfx_trace_buf;
#define SFX_TRACE_POINT(slot)                                          \
  do {                                                                 \
    if (threadIdx.x == 0 && sfx_trace_buf)                             \
      sfx_trace_buf[(uint64_t)blockIdx.x * 16 + (slot)] = wall_clock64(); \
  } while (0)
// Lane 0 of the calling wave stores instead (per-wave phase ends).
#define SFX_TRACE_WAVE(slot)                                           \
  do {                                                                 \
    if (__lane_id() == 0 && sfx_trace_buf)                             \
      sfx_trace_buf[(uint64_t)blockIdx.x * 16 + (slot)] = wall_clock64(); \
  } while (0)
// Per-wave counters of the last expansion (8 u64 per wave of 8).
extern __constant__ uint64_t* sfx_trace_stats;
#define SFX_TRACE_STAT(idx, val)                                       \
  do {                                                                 \
    if (__lane_id() == 0 && sfx_trace_stats)                           \
      sfx_trace_stats[((uint64_t)blockIdx.x * 8 + threadIdx.x / 64) * 8 + \
                      (idx)] = (uint64_t)(val);                        \
  } while (0)
#else
#define SFX_TRACE_POINT(slot) \
  do {                        \
  } while (0)
#define SFX_TRACE_WAVE(slot) \
  do {                       \
  } while (0)
#define SFX_TRACE_STAT(idx, val) \
  do {                           \
  } while (0)
#endif

namespace sfx {

constexpr int kWave = 64;
constexpr int32_t kPad = 0x7fffffff;  // corpus fill past the end
constexpr int32_t kSep = -2;          // document separator

// ------------------------------------------------------------ wave64 ops
__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

__device__ __forceinline__ int popc(uint64_t m) { return __popcll(m); }

// Number of set bits of m in lanes below the calling lane.
__device__ __forceinline__ int rank_lt(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi(
      (unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = __shfl_xor(v, o);
    v = w > v ? w : v;
  }
  return v;
}

__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

// Order LDS traffic of the calling wave (writes before later reads).
// Inclusive prefix sum over the 64 lanes of a wave with DPP row shifts and
// row broadcasts (no LDS traffic).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf,
                                             false);  // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf,
                                             false);  // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf,
                                             false);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf,
                                             false);  // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf,
                                             false);  // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf,
                                             false);  // row_bcast:31
  return v;
}

// Lane l of each row of 16 lanes takes lane l - 1's value; lane 0 of each
// row takes `first`.
__device__ __forceinline__ float lane_shr1(float v, float first) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, first),
                                         __builtin_bit_cast(int, v), 0x111,
                                         0xf, 0xf, false));  // row_shr:1
}

// Inclusive max-scan over the 64 lanes of a wave (unsigned; lanes shifted
// in from outside a row contribute 0).
__device__ __forceinline__ uint32_t wave_incl_max(uint32_t v) {
  uint32_t t;
  t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false);
  v = v > t ? v : t;
  t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false);
  v = v > t ? v : t;
  t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false);
  v = v > t ? v : t;
  t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false);
  v = v > t ? v : t;
  t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);
  v = v > t ? v : t;
  t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);
  v = v > t ? v : t;
  return v;
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ int64_t load_count(const void* p, int is64,
                                              int64_t i) {
  return is64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

// ------------------------------------------------- workspace handover
// Stores of data that another workgroup of the same launch reads after a
// handover (block_arrive): agent-scope relaxed atomic stores, which write
// through to memory, so the release's L2 write-back finds little dirty
// data (a release after 32 KiB of plain stores per workgroup measured
// ~9K cycles, after the same stores written through ~2K).
__device__ __forceinline__ void ws_store(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ws_store(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The matching reads after a handover without the acquire's cache
// invalidation (block_arrive<false>): agent-scope relaxed atomic loads,
// which read the coherent copy that the writers' stores and release
// reached, not a line a cache of this XCD may still hold.
__device__ __forceinline__ int32_t ws_load(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ws_load(const float* p) {
  return __uint_as_float(__hip_atomic_load(
      reinterpret_cast<uint32_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
      __HIP_MEMORY_SCOPE_AGENT));
}

// ------------------------------------------------------------ fp32 rules
// The chain probability and scores follow torch's fp32 CPU arithmetic:
// every operation rounds to fp32 (no FMA contraction; the library is built
// with -ffp-contract=off as well) and the division is IEEE-correct.

// max(0, floor(fl32(f) * fl32(L) + fl32(off))) as int64
// (suffix_gpu/local_matcher.py:76-81).  Float->int64 conversions that
// overflow produce INT64_MIN on the reference's x86 host and then clamp to
// 0; the same happens here.
__device__ __forceinline__ int64_t spec_cap(const sfx_params& p,
                                            int64_t len) {
  if (!p.has_spec_factor) return p.k;
  float v = __fadd_rn(__fmul_rn(p.spec_factor, (float)len), p.spec_offset);
  if (!(v < 9.2233720368547758e18f)) return 0;  // overflow or NaN
  if (!(v >= 0.0f)) return 0;
  return (int64_t)floorf(v);
}

// score + fl32(fl32(len) * fl32(1e-6)) (local_matcher.py:259-260).
__device__ __forceinline__ float local_key(float score, int64_t len) {
  return __fadd_rn(score, __fmul_rn((float)len, 1e-6f));
}

// ---------------------------------------------------- majority-vote expand
struct ExpandResult {
  int nv;       // number of valid chain slots (a prefix)
  float score;  // sum of the chain probability over valid slots < cap
};

// max votes first, then the smallest (signed) token
__device__ __forceinline__ bool vote_better(int cnt, int tok, int bcnt,
                                            int btok) {
  return cnt > bcnt || (cnt == bcnt && tok < btok);
}

// ---------------------------------------------------------- vote helpers
// Uniform maximum of an unsigned value over the wave.
__device__ __forceinline__ uint32_t wave_all_max(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_max(v),
                                             kWave - 1);
}

// Uniform minimum of a signed value over the wave.
__device__ __forceinline__ int32_t wave_all_min(int32_t v) {
  const uint32_t m = wave_all_max(~((uint32_t)v ^ 0x80000000u));
  return (int32_t)(~m ^ 0x80000000u);
}

constexpr int kHashSlots = 256;  // per wave LDS area H: 2 * kHashSlots ints
constexpr int kVoteSlots = 2 * kHashSlots;

__device__ __forceinline__ int vote_slot(int32_t v) {
  return (int)(((uint32_t)v * 0x9E3779B1u) >> 23);  // 9 bits
}

// Folds the vote over the rows' values v0, v1 (-1: no vote) into the
// running best (bcnt, btok): most rows, then the smallest value.  The rows
// of btok are counted already.  Every row adds one to its value's slot of
// an LDS count table H (kVoteSlots ints, by hash; plain atomics, no
// probing), so a slot's count bounds the count of each value in it from
// above.  The value with the largest bound (the smallest value on ties) is
// counted exactly with two ballots; when the bound was exact no other
// value can beat it, otherwise values are taken in bound order until no
// remaining bound can beat the best.
__device__ __forceinline__ void count_vote(int32_t v0, int32_t v1,
                                           int32_t* H, int& bcnt, int& btok) {
  const int ln = lane_id();
  int4* H4 = reinterpret_cast<int4*>(H);
  H4[ln] = make_int4(0, 0, 0, 0);
  H4[ln + kWave] = make_int4(0, 0, 0, 0);
  wave_lds_sync();
  const bool a0 = v0 != -1;
  const bool a1 = v1 != -1;
  const int h0 = vote_slot(v0);
  const int h1 = vote_slot(v1);
  if (a0) atomicAdd(&H[h0], 1);
  if (a1) atomicAdd(&H[h1], 1);
  wave_lds_sync();
  const bool known = bcnt > 0;
  uint32_t u0 = a0 && !(known && v0 == btok) ? (uint32_t)H[h0] : 0u;
  uint32_t u1 = a1 && !(known && v1 == btok) ? (uint32_t)H[h1] : 0u;
  wave_lds_sync();  // the table is rewritten by the next call
  while (true) {
    const uint32_t mu = wave_all_max(u0 > u1 ? u0 : u1);
    if (mu == 0u || (int)mu < bcnt) break;
    const int32_t t0 = u0 == mu ? v0 : 0x7fffffff;
    const int32_t t1 = u1 == mu ? v1 : 0x7fffffff;
    const int32_t x = wave_all_min(t0 < t1 ? t0 : t1);
    if ((int)mu == bcnt && x > btok) break;
    const int c = popc(ballot(v0 == x)) + popc(ballot(v1 == x));
    if (vote_better(c, x, bcnt, btok)) {
      bcnt = c;
      btok = x;
    }
    if ((uint32_t)c == mu) break;  // an exact bound: x beats the rest
    u0 = v0 == x ? 0u : u0;
    u1 = v1 == x ? 0u : u1;
  }
}

// Depths of one segment of the unit vote (below).
constexpr int kSegDepths = 16;

// Wave-cooperative depth-wise majority vote of one candidate
// (suffix_gpu/expand.py:59-147 == triton_kernels.py:139-215).
//
// Occurrence r (< R) is row r of the candidate's continuation block;
// cont_at(r, d) returns its token at depth d (any d < K) and is only
// called for rows r < occ.  chain_out[0..K) receives the chain (-1 past
// the first invalid depth).
//
// Unit votes with R <= 128 (two rows per lane) run in segments of up to
// kSegDepths depths.  A segment starts at depth d from r*, the first row
// on the chain (it agreed with every winner so far) that holds a token at
// d.  Each row finds the first depth of the window where its token differs
// from r*'s (its LDS tokens loaded eight at a time, compared by selects,
// no cross-lane step), and an LDS histogram of these agreement lengths and
// one DPP scan give, for every depth j of the window, g_j rows holding
// r*'s token among those still on the chain and x_j rows there holding
// another token.  Where g_j > x_j, r*'s token wins the full vote outright
// whatever the others hold, with count g_j and denominator
// g_j + x_j + alpha: every depth's factor is then one lane of a single
// vector division (exactly 1, skipped, when x_j and alpha are 0), and the
// chain probability and score are the same fp32 products and sums in
// depth order, computed lane after lane with DPP shifts.  So a run of
// majority depths costs a fixed number of steps, not one dependent
// ballot-and-divide round per depth.  A segment starts only where depth d
// holds a majority for r*'s token (two ballots); a depth without one takes
// a full vote, after which another segment starts when a single row is
// left, all voters agreed, or the depth had a majority after a segment of
// several depths -- else the next depth is voted in full too.  The tokens
// of the next depth are in flight during a full vote, and a segment that
// stops at a depth without a majority hands that depth's tokens on.
//
// The full vote: the first voter's value is counted with two ballots and
// settles a depth where it holds a majority; otherwise every value is
// counted at once (count_vote).  Larger R and weighted votes compact the
// active rows into A (row order) and count by broadcast LDS reads.  A
// holds R ints; W (weighted votes only) R floats, both LDS.  H is a
// per-wave LDS area of 2 * kHashSlots ints.
template <bool kWeighted, class ContFn, class WeightFn>
__device__ __forceinline__ ExpandResult expand_wave(ContFn cont_at,
                                                    WeightFn weight_at,
                                    int R, int64_t occ, int K, int64_t cap,
                                    float min_prob, float alpha, int* A,
                                    float* W, int32_t* H,
                                    int32_t* chain_out) {
  const int ln = lane_id();
  float prob = 1.0f;
  float score = 0.0f;
  int nv = 0;
  int d = 0;
#ifdef SFX_TRACE
  const uint64_t t_start = wall_clock64();
  const uint64_t c_start = __builtin_amdgcn_s_memtime();
  int st_hash = 0, st_full = 0, st_seg = 0;
#endif
  if (!kWeighted && R <= 2 * kWave) {
    const int r0 = ln;
    const int r1 = ln + kWave;
    const bool in0 = r0 < R && (int64_t)r0 < occ;
    const bool in1 = r1 < R && (int64_t)r1 < occ;
    // Tokens at depth d of the rows on the chain (they agreed with every
    // winner so far), -1 for the others and for rows without a token there
    // (they leave the chain at d).
    int v0 = in0 && K > 0 ? cont_at(r0, 0) : -1;
    int v1 = in1 && K > 0 ? cont_at(r1, 0) : -1;
    bool ended = false;
    bool vote = false;  // depth d is voted in full
    int last_run = kSegDepths;  // depths the last segment settled
    while (!ended && d < K) {
      if (vote) {
        // ---- one full vote at depth d over the rows on the chain; the
        // voters' tokens at depth d + 1 (a superset of the survivors') are
        // loaded meanwhile
#ifdef SFX_TRACE
        ++st_full;
#endif
        const bool nx = d + 1 < K;
        const int n0 = nx && v0 != -1 ? cont_at(r0, d + 1) : -1;
        const int n1 = nx && v1 != -1 ? cont_at(r1, d + 1) : -1;
        const uint64_t rem0 = ballot(v0 != -1);
        const uint64_t rem1 = ballot(v1 != -1);
        const int nact = popc(rem0) + popc(rem1);
        if (nact == 0) break;
        const float denom = __fadd_rn((float)(nact > 1 ? nact : 1), alpha);
        // The first voter's value, counted with two ballots, settles a
        // depth where it holds a majority; otherwise every value is counted
        // at once.
        int btok = rem0 ? __builtin_amdgcn_readlane(v0, __builtin_ctzll(rem0))
                        : __builtin_amdgcn_readlane(v1, __builtin_ctzll(rem1));
        int bcnt = popc(ballot(v0 == btok)) + popc(ballot(v1 == btok));
        if (2 * bcnt <= nact) {
#ifdef SFX_TRACE
          ++st_hash;
#endif
          count_vote(v0, v1, H, bcnt, btok);
        }
        const float vf = (float)bcnt;
        prob = __fmul_rn(prob, __fdiv_rn(vf, denom));
        const bool valid = (vf > 0.0f) && (prob >= min_prob);
        if (!valid) break;
        if (ln == 0) chain_out[d] = btok;
        if ((int64_t)d < cap) score = __fadd_rn(score, prob);
        v0 = v0 != -1 && v0 == btok ? n0 : -1;
        v1 = v1 != -1 && v1 == btok ? n1 : -1;
        ++d;
        // A segment pays off over a run of majority depths: the next depth
        // starts one when a single row is left (the bcnt winners stay),
        // every voter agreed here, or this depth had a majority after a
        // segment of several depths; otherwise it is voted in full as well.
        vote = !(bcnt == 1 || bcnt == nact ||
                 (2 * bcnt > nact && last_run >= 4));
        continue;
      }
      // ---- one segment: depths d .. d + W - 1 against r*, the first row
      // on the chain with a token at d
      const uint64_t s0 = ballot(v0 != -1);
      const uint64_t s1 = ballot(v1 != -1);
      if (!(s0 | s1)) break;  // no row votes: the chain ends
#ifdef SFX_TRACE
      ++st_seg;
#endif
      const bool p0 = v0 != -1;
      const bool p1 = v1 != -1;
      const int rs = s0 ? __builtin_ctzll(s0) : kWave + __builtin_ctzll(s1);
      const int nP = popc(s0) + popc(s1);
      {
        // Depth d itself without a majority for r*'s token: no segment
        const int a0 = __builtin_amdgcn_readlane(s0 ? v0 : v1, rs & 63);
        const int g0 = popc(ballot(v0 == a0)) + popc(ballot(v1 == a0));
        if (2 * g0 <= nP) {
          vote = true;
          continue;
        }
      }
      const int W = K - d < kSegDepths ? K - d : kSegDepths;
      // lane j < W: r*'s token at depth d + j; no row agrees with r* from
      // its first -1 on (We >= 1: r* holds a token at d)
      const int refv = ln < W ? cont_at(rs, d + ln) : -1;
      const uint64_t rend = ballot(ln < W && refv == -1);
      const int We = rend ? __builtin_ctzll(rend) : W;
      // Agreement of each row with r*: the first depth of the window where
      // its token differs and that token, found by visiting the depths from
      // the last, eight loads in flight per row (rows off the chain read
      // r*'s tokens and are dropped below; depths past the window reread
      // its last one).
      const int q0 = p0 ? r0 : rs;
      const int q1 = p1 ? r1 : rs;
      int au0 = W, au1 = W, dt0 = -1, dt1 = -1;
      auto agree8 = [&](int jb, auto two) {
        int t0[8], t1[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int jj = jb + u < W ? jb + u : W - 1;
          t0[u] = cont_at(q0, d + jj);
          if (two) t1[u] = cont_at(q1, d + jj);
        }
#pragma unroll
        for (int u = 7; u >= 0; --u) {
          const int a = __builtin_amdgcn_readlane(refv, jb + u);
          au0 = t0[u] != a ? jb + u : au0;
          dt0 = t0[u] != a ? t0[u] : dt0;
          if (two) {
            au1 = t1[u] != a ? jb + u : au1;
            dt1 = t1[u] != a ? t1[u] : dt1;
          }
        }
      };
      static_assert(kSegDepths == 16, "two batches of eight depths");
      // (depth We itself is scanned too: a vote there takes its tokens)
      if (s1 != 0) {
        if (We >= 8) agree8(8, std::true_type());
        agree8(0, std::true_type());
      } else {
        if (We >= 8) agree8(8, std::false_type());
        agree8(0, std::false_type());
      }
      // agreement lengths within the window (-1 off the chain)
      const int ag0 = p0 ? (au0 < We ? au0 : We) : -1;
      const int ag1 = p1 ? (au1 < We ? au1 : We) : -1;
      // Every row on the chain agreeing with r* through the window (one
      // wave minimum): each depth j < We has all of them voting for r*'s
      // token and no other vote, so with alpha 0 its factor is exactly 1
      // and the probability stays; the depth We (if < W) has no majority.
      const int amin = wave_all_min(min(ag0 >= 0 ? ag0 : 0x7fffffff,
                                        ag1 >= 0 ? ag1 : 0x7fffffff));
      int m;
      float pv;
      if (amin >= We && alpha == 0.0f) {
        m = We;
        pv = prob;
      } else {
        // Per depth j (lane j): g rows holding r*'s token at depth d + j
        // among those still on the chain there (agreement > j), x rows
        // there voting for another token (agreement == j, a token there).
        // r*'s token wins outright when g > x, with the full vote's count g
        // and denominator g + x.  The agreement histogram (hg) and the
        // voters' one (hx) are counted in H.
        int* hg = H;
        int* hx = H + 32;
        H[ln] = 0;
        wave_lds_sync();
        if (ag0 >= 0) {
          atomicAdd(&hg[ag0], 1);
          if (ag0 < We && dt0 != -1) atomicAdd(&hx[ag0], 1);
        }
        if (ag1 >= 0) {
          atomicAdd(&hg[ag1], 1);
          if (ag1 < We && dt1 != -1) atomicAdd(&hx[ag1], 1);
        }
        wave_lds_sync();
        const int gv =
            nP - (int)wave_incl_scan(ln < 32 ? (uint32_t)hg[ln] : 0u);
        const int xv = ln < 32 ? hx[ln] : 0;
        const uint64_t maj = ballot(ln < We && gv > xv);
        m = __builtin_ctzll(~maj);  // <= We (lanes >= We: 0)
        // g / (g + 0) is exactly 1: no division then
        float f = 1.0f;
        if (xv != 0 || alpha != 0.0f)
          f = __fdiv_rn((float)gv, __fadd_rn((float)(gv + xv), alpha));
        // Lane j: the chain probability after depth d + j, the fp32
        // product in depth order -- each step takes the left neighbour's
        // product (lane 0: the probability before the window), so after
        // step s lanes 0 .. s hold their final values.
        pv = f;
#pragma unroll
        for (int sb = 0; sb < kSegDepths; sb += 4) {
          if (sb >= m) break;
#pragma unroll
          for (int s = sb; s < sb + 4; ++s)
            pv = __fmul_rn(lane_shr1(pv, prob), f);
        }
      }
      const uint64_t okp = ballot(ln < m && pv >= min_prob);
      const int jn = __builtin_ctzll(~okp);  // depths kept, <= m
      // the score: the same in-order fp32 sum over depths below cap
      const int64_t room = cap - (int64_t)d;
      const int lim = room < (int64_t)jn ? (room < 0 ? 0 : (int)room) : jn;
      if (lim > 0) {
        const float av = ln < lim ? pv : 0.0f;
        float sv = av;
#pragma unroll
        for (int sb = 0; sb < kSegDepths; sb += 4) {
          if (sb >= lim) break;
#pragma unroll
          for (int s = sb; s < sb + 4; ++s)
            sv = __fadd_rn(lane_shr1(sv, score), av);
        }
        score = __builtin_bit_cast(
            float,
            __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), lim - 1));
      }
      if (jn > 0)
        prob = __builtin_bit_cast(
            float,
            __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv), jn - 1));
      if (ln < jn) chain_out[d + ln] = refv;
      last_run = jn;
      const bool k0 = ag0 >= jn;
      const bool k1 = ag1 >= jn;
      if (jn < m) {
        ended = true;  // the chain probability fell below min_prob
      } else if (jn < W) {
        // Depth d + jn has no majority for r*'s token: voted in full, with
        // the tokens there already known -- r*'s for rows that agree with
        // it there, else the row's first differing token.
        vote = true;
        const int rj = __builtin_amdgcn_readlane(refv, jn);
        v0 = k0 ? (au0 > jn ? rj : dt0) : -1;
        v1 = k1 ? (au1 > jn ? rj : dt1) : -1;
      } else if (d + jn < K) {
        v0 = k0 ? cont_at(r0, d + jn) : -1;
        v1 = k1 ? cont_at(r1, d + jn) : -1;
      }
      d += jn;
    }
    nv = d;
  } else {
    const int nslot = (R + kWave - 1) / kWave;  // <= 32 (R <= 2048)
    uint32_t ok = 0;
    for (int s = 0; s < nslot; ++s) {
      int r = s * kWave + ln;
      if (r < R && (int64_t)r < occ) ok |= 1u << s;
    }
    for (; d < K; ++d) {
      int nact = 0;
      for (int s = 0; s < nslot; ++s) {
        const int r = s * kWave + ln;
        const bool okr = (ok >> s) & 1u;
        int c = -1;
        if (okr) c = cont_at(r, d);
        const bool act = okr && c != -1;
        const uint64_t m = ballot(act);
        if (act) {
          const int pos = nact + rank_lt(m);
          A[pos] = c;
          if (kWeighted) W[pos] = weight_at(r);
        }
        nact += popc(m);
        if (!act) ok &= ~(1u << s);
      }
      wave_lds_sync();
      if (nact == 0) break;
      uint64_t best = 0;
      for (int i = ln; i < nact; i += kWave) {
        const int x = A[i];
        uint32_t vbits;
        if (!kWeighted) {
          int v = 0;
          int j = 0;
          for (; j + 4 <= nact; j += 4) {
            const int4 q = *reinterpret_cast<const int4*>(A + j);
            v += (q.x == x) + (q.y == x) + (q.z == x) + (q.w == x);
          }
          for (; j < nact; ++j) v += (A[j] == x);
          vbits = (uint32_t)v;
        } else {
          float v = 0.0f;
          for (int j = 0; j < nact; ++j)
            if (A[j] == x) v = __fadd_rn(v, W[j]);
          vbits = __float_as_uint(v);
        }
        const uint64_t key =
            ((uint64_t)vbits << 32) |
            (uint64_t)(0xffffffffu - ((uint32_t)x ^ 0x80000000u));
        best = key > best ? key : best;
      }
      best = wave_max_u64(best);
      const uint32_t vbits = (uint32_t)(best >> 32);
      const int tok = (int)((0xffffffffu - (uint32_t)best) ^ 0x80000000u);
      float vf;
      float denom;
      if (!kWeighted) {
        vf = (float)(int)vbits;
        denom = __fadd_rn((float)(nact > 1 ? nact : 1), alpha);
      } else {
        vf = __uint_as_float(vbits);
        float a = 0.0f;
        for (int j = 0; j < nact; ++j) a = __fadd_rn(a, W[j]);
        denom = __fadd_rn(a, alpha);
      }
      prob = __fmul_rn(prob, __fdiv_rn(vf, denom));
      const bool valid = (vf > 0.0f) && (prob >= min_prob);
      if (!valid) break;
      if (ln == 0) chain_out[d] = tok;
      if ((int64_t)d < cap) score = __fadd_rn(score, prob);
      ++nv;
      for (int s = 0; s < nslot; ++s) {
        if ((ok >> s) & 1u) {
          if (cont_at(s * kWave + ln, d) != tok) ok &= ~(1u << s);
        }
      }
      wave_lds_sync();
    }
  }
  for (int dd = d + ln; dd < K; dd += kWave) chain_out[dd] = -1;
#ifdef SFX_TRACE
  SFX_TRACE_STAT(0, occ);
  SFX_TRACE_STAT(1, st_seg);
  SFX_TRACE_STAT(2, st_full + 1000 * st_hash);
  SFX_TRACE_STAT(6, wall_clock64() - t_start);
  SFX_TRACE_STAT(7, nv);
#endif
  ExpandResult res;
  res.nv = nv;
  res.score = score;
  return res;
}

struct NoWeight {
  __device__ float operator()(int) const { return 0.0f; }
};

// ------------------------------------------------- ordered compaction
// Inclusive prefix sum over the 16 lanes of each row (DPP row shifts).
__device__ __forceinline__ uint32_t row16_incl_scan(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf,
                                             false);  // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf,
                                             false);  // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf,
                                             false);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf,
                                             false);  // row_shr:8
  return v;
}

// Block-wide exclusive prefix sums of up to 8 per-thread counters (those
// with on[c]; the others read 0), and their block totals, with one
// barrier: the waves' inclusive scans leave each wave's totals in
// `scratch` (8 * (NT/64) u32 of LDS), and every wave then scans the
// waves' totals itself -- lane w holds wave w's, one 16-lane scan per
// counter -- instead of every thread adding up all the waves.  A
// following call must use another scratch area (or come after a barrier):
// waves leave while slower ones still read this one's.
template <int NT>
__device__ __forceinline__ void block_exscan8(const uint32_t (&v)[8],
                                              const bool (&on)[8],
                                              uint32_t (&pre)[8],
                                              uint32_t (&tot)[8],
                                              uint32_t* scratch) {
  constexpr int NW = NT / kWave;
  static_assert(NW <= 16, "one row of 16 lanes holds the waves' totals");
  const int ln = lane_id();
  const int wv = threadIdx.x / kWave;
  uint32_t inc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) inc[c] = on[c] ? wave_incl_scan(v[c]) : 0u;
  if (ln == kWave - 1) {
    reinterpret_cast<uint4*>(scratch + wv * 8)[0] =
        make_uint4(inc[0], inc[1], inc[2], inc[3]);
    reinterpret_cast<uint4*>(scratch + wv * 8)[1] =
        make_uint4(inc[4], inc[5], inc[6], inc[7]);
  }
  __syncthreads();
  uint4 lo = make_uint4(0u, 0u, 0u, 0u), hi = lo;
  if (ln < NW) {
    lo = reinterpret_cast<const uint4*>(scratch + ln * 8)[0];
    hi = reinterpret_cast<const uint4*>(scratch + ln * 8)[1];
  }
  const uint32_t t8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    uint32_t before = 0, all = 0;
    if (on[c]) {
      const uint32_t x = row16_incl_scan(t8[c]);
      before = wv > 0 ? (uint32_t)__builtin_amdgcn_readlane((int)x, wv - 1)
                      : 0u;
      all = (uint32_t)__builtin_amdgcn_readlane((int)x, NW - 1);
    }
    pre[c] = before + inc[c] - v[c];
    tot[c] = all;
  }
}

// Per-byte test x >= t (1 <= t <= 255) on four u8 match lengths at once,
// as 0x80 flags.  With s = (x & 0x7f) + add (add = 128 - t for t < 128,
// 256 - t otherwise; never carries out of the byte), bit 7 of s is the
// carry of the low seven bits of x - t, and the carry out of the byte --
// no borrow, x >= t -- is x7 | s7 for t < 128 and x7 & s7 for t >= 128.
struct ByteGe {
  uint32_t add;  // per-byte constant replicated into all four bytes
  bool hi;       // t >= 128
  bool on;       // t >= 1
};
__device__ __forceinline__ ByteGe byte_ge_init(int t) {
  ByteGe g;
  g.on = t > 0;
  g.hi = t >= 128;
  const uint32_t a = t <= 0 ? 0u : (g.hi ? 256u - t : 128u - t);
  g.add = a * 0x01010101u;
  return g;
}
__device__ __forceinline__ uint32_t bytes_ge(uint32_t x, const ByteGe& g) {
  const uint32_t s = (x & 0x7f7f7f7fu) + g.add;
  return (g.hi ? (x & s) : (x | s)) & 0x80808080u;
}

// Clears the bytes of a 16-byte word from byte r (0 < r < 16) on.
__device__ __forceinline__ uint4 clear_from(uint4 q, int r) {
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int keep = r - 4 * k;
    if (keep <= 0) w[k] = 0u;
    else if (keep < 4) w[k] &= (1u << (8 * keep)) - 1u;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// First R ascending positions i in [0, n) with mb[i] >= thr[c], for up to
// 8 thresholds (thr[c] <= 0 disables c).  mb holds u8 match lengths, is
// 16-byte aligned and readable up to the last thread segment's end (bytes
// from n on are ignored).  One ordered
// pass: every thread owns a 16-byte-aligned segment read as uint4 words,
// counts bytes >= thr four at a time (all-zero words skipped), one block
// scan gives each thread its output offsets, then it writes its hits
// below R.  out[c * R + slot] = out_base + position; count[c] =
// min(hits, R).  With kAcc the call continues an earlier one over the
// preceding positions: count[c] holds the hits kept so far, new hits take
// the slots after them and count[c] = min(count[c] + hits, R) (the calls
// are separated by a barrier).  thr is LDS holding nthr thresholds; out
// and count may be LDS or global.  scratch holds 2 * 8 * (NT/64) u32 of
// LDS: consecutive calls alternate its halves (buf 0, 1, 0, ...) or are
// separated by a barrier.  kWsOut: out is workspace another workgroup
// reads after a handover (ws_store).  All threads of the block must call
// it.
template <int NT, bool kAcc = false, bool kWsOut = false, typename MbPtr>
__device__ __forceinline__ void compact_first_r(MbPtr mb, int64_t n,
                                                const int* thr, int nthr,
                                                int R, int32_t* out,
                                                int32_t out_base, int* count,
                                                uint32_t* scratch, int buf) {
  int64_t seg = (n + NT - 1) / NT;
  seg = (seg + 15) & ~(int64_t)15;
  const int64_t beg = (int64_t)threadIdx.x * seg;
  const int64_t end = beg + seg < n ? beg + seg : n;
  // the thresholds (and kept counts) as independent loads
  int tv[8];
  uint32_t kept[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int cc = c < nthr ? c : 0;
    tv[c] = thr[cc];
    kept[c] = kAcc ? (uint32_t)count[cc] : 0u;
  }
  ByteGe ge[8];
  bool on[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    if (c >= nthr) kept[c] = 0u;
    ge[c] = byte_ge_init(c < nthr && kept[c] < (uint32_t)R ? tv[c] : 0);
    on[c] = ge[c].on;
  }
  uint32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t i0 = beg; i0 < end; i0 += 16) {
    uint4 q = *reinterpret_cast<const uint4*>(mb + i0);
    if (i0 + 16 > end) q = clear_from(q, (int)(end - i0));
    if ((q.x | q.y | q.z | q.w) == 0u) continue;  // no match ends here
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (ge[c].on) {
        cnt[c] += __popc(bytes_ge(q.x, ge[c])) + __popc(bytes_ge(q.y, ge[c])) +
                  __popc(bytes_ge(q.z, ge[c])) + __popc(bytes_ge(q.w, ge[c]));
      }
    }
  }
  uint32_t off[8], tot[8];
  SFX_TRACE_POINT(7);
  block_exscan8<NT>(cnt, on, off, tot, scratch + buf * (8 * (NT / kWave)));
  SFX_TRACE_POINT(8);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    off[c] += kept[c];
    tot[c] += kept[c];
  }
  bool more = false;
#pragma unroll
  for (int c = 0; c < 8; ++c) more |= ge[c].on && off[c] < (uint32_t)R;
  for (int64_t i0 = beg; more && i0 < end; i0 += 16) {
    uint4 q = *reinterpret_cast<const uint4*>(mb + i0);
    if (i0 + 16 > end) q = clear_from(q, (int)(end - i0));
    if ((q.x | q.y | q.z | q.w) == 0u) continue;
    const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
    more = false;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (ge[c].on && off[c] < (uint32_t)R) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint32_t m = bytes_ge(w4[k], ge[c]);
          while (m) {
            const int byte = __builtin_ctz(m) >> 3;
            if (off[c] < (uint32_t)R) {
              const int32_t v = out_base + (int32_t)(i0 + 4 * k + byte);
              if (kWsOut)
                ws_store(out + c * R + off[c], v);
              else
                out[c * R + off[c]] = v;
            }
            ++off[c];
            m &= m - 1;
          }
        }
        more |= off[c] < (uint32_t)R;
      }
    }
  }
  if (threadIdx.x < (unsigned)nthr) {
    const int c = threadIdx.x;
    uint32_t total = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k == c) total = tot[k];
    count[c] = total < (uint32_t)R ? (int)total : R;
  }
  SFX_TRACE_POINT(9);
}

// -------------------------------------------------- block-level handover
// Publish this block's global writes, count its arrival on ctr and return
// (to every thread) whether it was the last of `expected` arrivals.  The
// last arriver resets the counter, so the workspace is zero again after
// every call.  Call from uniform control flow.
//
// The fences are device-scope and cost a write-back (release) or an
// invalidation (acquire) of the XCD's whole L2, so each is issued once per
// workgroup, by thread 0, and split into its release and acquire halves:
// the barrier first completes every wave's stores into the L2, thread 0's
// release writes that L2 back before the counter update, and only the last
// arriver's thread 0 invalidates (its CU's L1 and XCD's L2) before the
// barrier that lets the block read the other workgroups' results.
// kAcquire false: no invalidation; the last arriver then reads the other
// workgroups' results only with ws_load (every such load is issued after
// the counter update has returned, behind the barrier).
template <bool kAcquire = true>
__device__ __forceinline__ bool block_arrive(unsigned* ctr,
                                             unsigned expected,
                                             int* lds_flag) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned old = atomicAdd(ctr, 1u);
    const int last = old == expected - 1;
    if (last) {
      atomicExch(ctr, 0u);
      if (kAcquire) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    *lds_flag = last;
  }
  __syncthreads();
  return *lds_flag != 0;
}

}  // namespace sfx
