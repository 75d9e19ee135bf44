// N-gram range table: for every distinct run of the first k tokens
// (k = 1 .. kGramMax) among the sorted suffixes, the ranks [lo, hi) of the
// suffixes that start with it.  An SA interval search for a pattern of l
// tokens starts from the range of its first min(l, kGramMax) tokens: for
// l <= kGramMax that range is the answer, for longer patterns the k-ary
// search runs inside it instead of over the whole suffix array.  On the
// 2^22-token template corpus this cuts the slowest of a row's 32 searches
// from 6 dependent rounds to at most 3 (one lookup plus two rounds).
//
// Layout: a 256-byte header {kmax, runs[4]}, then one u32 fill count per bucket
// (padded to 256 bytes), then the buckets, each kGramBucket 16-byte keys
// {t0, t1, t2, t3} (-1 past the run's length, which no real token equals,
// so a key also tells its length) followed by their kGramBucket 8-byte
// rank ranges {lo, hi}: 384 bytes a bucket.  A table has any number of
// buckets; a run hashes to bucket (h * buckets) >> 32, and an insert
// takes position atomicAdd(&count[b], 1) and, when b is full, moves on to
// b + 1, b + 2, ... (wrapping; at most kGramSpill buckets).  The counts
// keep counting past kGramBucket, so count[b] > kGramBucket tells a
// lookup that runs hashed to b (or before) may sit further on.  The
// counts are 4 B a bucket, so the inserts' atomics stay in cache while the
// slot stores stream out; a lookup is one round of loads (the bucket's
// keys, ranges and count together) unless its bucket overflowed.
//
// A build first counts the distinct runs of each length (runs[k - 1]) and
// stores the runs of 1 .. kcap tokens, kcap the longest length whose runs
// together fill at most 3/4 of the slots; an insert that still finds no
// room lowers kmax below its length.  kmax (0 .. kGramMax) is then the
// longest length whose runs are all stored, and a search looks up its
// pattern's first min(l, kmax) tokens: text with about 1.6 distinct runs
// of 1-4 tokens per position keeps all four lengths in 3 slots per
// position, while uniform random tokens over a large vocabulary (about 3
// per position) keep three, and kmax = 0 turns the table off (exact,
// only slower).
//
// Only runs of real tokens are stored (0 <= t < INT32_MAX): query patterns
// hold real tokens, and the separator, the corpus padding and the -1 read
// past the corpus end never equal one.  A pattern whose first tokens are
// not all real skips the table.
#pragma once

#include "sfx_common.h"

namespace sfx {

constexpr int kGramMax = 4;
constexpr int kGramBucket = 16;  // slots per bucket
constexpr int kGramSpill = 16;   // buckets an insert or lookup may visit
// bytes of a bucket: its keys, then their ranges
constexpr int kGramBucketBytes = kGramBucket * (16 + 8);

// Runs of all lengths may fill at most kGramLoadNum / kGramLoadDen of
// the slots.
constexpr int kGramLoadNum = 3;
constexpr int kGramLoadDen = 4;

struct GramHeader {
  uint32_t kmax;  // every run of 1 .. kmax tokens is stored (0: unusable)
  uint32_t pad0;
  unsigned long long runs[kGramMax];  // distinct runs of k + 1 tokens
  uint32_t pad[54];
};
static_assert(sizeof(GramHeader) == 256, "counts start 256-byte aligned");

// Buckets of a table of `slots` slots (a multiple of kGramBucket).
__host__ __device__ inline int64_t gram_buckets(int64_t slots) {
  return slots / kGramBucket;
}

__host__ __device__ inline size_t gram_counts_bytes(int64_t slots) {
  return ((size_t)gram_buckets(slots) * 4 + 255) & ~(size_t)255;
}

__host__ __device__ inline size_t gram_table_bytes(int64_t slots) {
  return sizeof(GramHeader) + gram_counts_bytes(slots) +
         (size_t)gram_buckets(slots) * kGramBucketBytes;
}

__device__ __forceinline__ uint32_t* gram_counts(void* table) {
  return reinterpret_cast<uint32_t*>((char*)table + sizeof(GramHeader));
}

__device__ __forceinline__ const uint32_t* gram_counts(const void* table) {
  return reinterpret_cast<const uint32_t*>((const char*)table +
                                           sizeof(GramHeader));
}

// Bucket b: its keys at the returned address, its ranges 256 bytes on.
__device__ __forceinline__ char* gram_bucket(void* table, int64_t slots,
                                             uint32_t b) {
  return (char*)table + sizeof(GramHeader) + gram_counts_bytes(slots) +
         (size_t)b * kGramBucketBytes;
}

__device__ __forceinline__ const char* gram_bucket(const void* table,
                                                   int64_t slots,
                                                   uint32_t b) {
  return (const char*)table + sizeof(GramHeader) + gram_counts_bytes(slots) +
         (size_t)b * kGramBucketBytes;
}

// The s-th bucket a run of hash h may sit in (its home bucket first).
__device__ __forceinline__ uint32_t gram_probe(uint32_t h, uint32_t nb,
                                               int s) {
  uint32_t b = (uint32_t)(((uint64_t)h * nb) >> 32) + (uint32_t)s;
  while (b >= nb) b -= nb;
  return b;
}

__device__ __forceinline__ bool gram_real(int32_t t) {
  return t >= 0 && t != kPad;
}

// The stored key of a run of k tokens: -1 past k.
__device__ __forceinline__ int4 gram_key(int32_t t0, int32_t t1, int32_t t2,
                                         int32_t t3, int k) {
  return make_int4(t0, k > 1 ? t1 : -1, k > 2 ? t2 : -1, k > 3 ? t3 : -1);
}

// Hash of a run's key: a multiply-xorshift mix of each word (the
// MurmurHash3 finalizer constants).
__device__ __forceinline__ uint32_t gram_hash(const int4& t) {
  uint32_t h = 0x9e3779b9u;
  const uint32_t w[4] = {(uint32_t)t.x, (uint32_t)t.y, (uint32_t)t.z,
                         (uint32_t)t.w};
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

// One group of G lanes looks the run (t0..t3, k) up, kGramBucket / G
// slots of a bucket per lane.  Returns 1 (found, [lo, hi) set), 0 (absent)
// or -1 (no answer within kGramSpill buckets: search the whole array).
// Every lane of the group gets the same result.
template <int G>
__device__ __forceinline__ int gram_lookup(const void* table, int64_t slots,
                                           int32_t t0, int32_t t1,
                                           int32_t t2, int32_t t3, int k,
                                           uint32_t& lo, uint32_t& hi) {
  static_assert(kGramBucket % G == 0, "lanes split a bucket evenly");
  constexpr int PL = kGramBucket / G;  // slots per lane
  const uint32_t* counts = gram_counts(table);
  const uint32_t nb = (uint32_t)gram_buckets(slots);
  const int ln = lane_id();
  const int gl = ln % G;
  const int gbase = ln - gl;
  const uint32_t full = G == 32 ? 0xffffffffu : ((1u << G) - 1u);
  const int4 key = gram_key(t0, t1, t2, t3, k);
  const uint32_t h = gram_hash(key);
  for (int s = 0; s < kGramSpill; ++s) {
    const uint32_t bk = gram_probe(h, nb, s);
    const uint32_t cnt = counts[bk];
    const char* bucket = gram_bucket(table, slots, bk);
    int4 a[PL];
    uint2 w[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int slot = gl * PL + i;
      a[i] = reinterpret_cast<const int4*>(bucket)[slot];
      w[i] = reinterpret_cast<const uint2*>(bucket + 16 * kGramBucket)[slot];
    }
    bool hit = false;
    uint32_t hl = 0, hh = 0;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const uint32_t pos = (uint32_t)(gl * PL + i);
      const bool h1 = pos < cnt && a[i].x == key.x && a[i].y == key.y &&
                      a[i].z == key.z && a[i].w == key.w;
      hl = h1 ? w[i].x : hl;
      hh = h1 ? w[i].y : hh;
      hit = hit || h1;
    }
    const uint32_t mh = (uint32_t)(ballot(hit) >> gbase) & full;
    if (mh) {
      const int src = gbase + __builtin_ctz(mh);
      lo = (uint32_t)__shfl((int)hl, src);
      hi = (uint32_t)__shfl((int)hh, src);
      return 1;
    }
    if (cnt <= (uint32_t)kGramBucket) return 0;
  }
  return -1;
}

}  // namespace sfx
