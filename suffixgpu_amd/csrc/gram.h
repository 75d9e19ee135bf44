// N-gram range table: for every distinct run of the first k tokens
// (k = 1 .. kGramMax) among the sorted suffixes, the ranks [lo, hi) of the
// suffixes that start with it.  An SA interval search for a pattern of l
// tokens starts from the range of its first min(l, kGramMax) tokens: for
// l <= kGramMax that range is the answer, for longer patterns the k-ary
// search runs inside it instead of over the whole suffix array.  On the
// 2^22-token template corpus this cuts the slowest of a row's 32 searches
// from 6 dependent rounds to at most 3 (one lookup plus two rounds).
//
// Layout: a 256-byte header {epoch, ok} and `slots` (a power of two)
// 32-byte slots {t[4], epoch, lo, hi, k}, open addressing with linear
// probing.  A slot belongs to the table built with header epoch e iff its
// own epoch equals e, so a rebuild never clears the table: it bumps the
// epoch and claims slots with a compare-and-swap on their epoch word.  A
// build that runs out of probes sets ok = 0, and searches then ignore the
// table (exact, only slower).
//
// Only runs of real tokens are stored (0 <= t < INT32_MAX): query patterns
// hold real tokens, and the separator, the corpus padding and the -1 read
// past the corpus end never equal one.  A pattern whose first tokens are
// not all real skips the table.
#pragma once

#include "sfx_common.h"

namespace sfx {

constexpr int kGramMax = 4;
constexpr int kGramProbes = 64;  // longest probe sequence of an insert

struct GramSlot {
  int32_t t[4];    // the run's tokens, zero past k
  uint32_t epoch;  // the build that wrote the slot
  uint32_t lo;     // first rank
  uint32_t hi;     // one past the last rank
  uint32_t k;      // run length in tokens
};
static_assert(sizeof(GramSlot) == 32, "one slot is two 16-byte words");

struct GramHeader {
  uint32_t epoch;  // the current build (0: never built)
  uint32_t ok;     // every run of the current build was stored
  uint32_t pad[62];
};
static_assert(sizeof(GramHeader) == 256, "slots start 256-byte aligned");

__host__ __device__ inline size_t gram_table_bytes(int64_t slots) {
  return sizeof(GramHeader) + (size_t)slots * sizeof(GramSlot);
}

__device__ __forceinline__ GramSlot* gram_slots(void* table) {
  return reinterpret_cast<GramSlot*>((char*)table + sizeof(GramHeader));
}

__device__ __forceinline__ const GramSlot* gram_slots(const void* table) {
  return reinterpret_cast<const GramSlot*>((const char*)table +
                                           sizeof(GramHeader));
}

__device__ __forceinline__ bool gram_real(int32_t t) {
  return t >= 0 && t != kPad;
}

// Hash of a run (tokens past k are zero): a multiply-xorshift mix of each
// word (the MurmurHash3 finalizer constants).
__device__ __forceinline__ uint32_t gram_hash(int32_t t0, int32_t t1,
                                              int32_t t2, int32_t t3, int k) {
  uint32_t h = 0x9e3779b9u * (uint32_t)(k + 1);
  const uint32_t w[4] = {(uint32_t)t0, (uint32_t)t1, (uint32_t)t2,
                         (uint32_t)t3};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h ^= w[j] + 0x7f4a7c15u + (h << 6) + (h >> 2);
    h ^= h >> 16;
    h *= 0x85ebca6bu;
    h ^= h >> 13;
    h *= 0xc2b2ae35u;
    h ^= h >> 16;
  }
  return h;
}

// One group of G lanes looks the run (t0..t3, k) up in G consecutive
// slots per step.  Returns 1 (found, [lo, hi) set), 0 (absent) or -1 (no
// answer within the probe limit: search the whole array).  Every lane of
// the group gets the same result.
template <int G>
__device__ __forceinline__ int gram_lookup(const void* table,
                                           uint32_t mask, uint32_t epoch,
                                           int32_t t0, int32_t t1,
                                           int32_t t2, int32_t t3, int k,
                                           uint32_t& lo, uint32_t& hi) {
  const GramSlot* slots = gram_slots(table);
  const int ln = lane_id();
  const int gl = ln % G;
  const int gbase = ln - gl;
  const uint32_t full = G == 32 ? 0xffffffffu : ((1u << G) - 1u);
  const uint32_t h = gram_hash(t0, t1, t2, t3, k);
  for (int base = 0; base < kGramProbes + G; base += G) {
    const uint32_t s = (h + (uint32_t)(base + gl)) & mask;
    const int4 a = *reinterpret_cast<const int4*>(&slots[s].t[0]);
    const uint4 b = *reinterpret_cast<const uint4*>(&slots[s].epoch);
    const bool live = b.x == epoch;
    const bool hit = live && (int)b.w == k && a.x == t0 && a.y == t1 &&
                     a.z == t2 && a.w == t3;
    const uint32_t mh = (uint32_t)(ballot(hit) >> gbase) & full;
    const uint32_t me = (uint32_t)(ballot(!live) >> gbase) & full;
    if (mh && (!me || __builtin_ctz(mh) < __builtin_ctz(me))) {
      const int src = gbase + __builtin_ctz(mh);
      lo = (uint32_t)__shfl((int)b.y, src);
      hi = (uint32_t)__shfl((int)b.z, src);
      return 1;
    }
    if (me) return 0;
  }
  return -1;
}

}  // namespace sfx
