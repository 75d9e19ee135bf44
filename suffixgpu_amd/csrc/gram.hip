// Building the n-gram range table (gram.h) of a suffix array from its key
// rows, on the caller's stream with no host synchronisation: the bucket
// counts are cleared, one pass counts the distinct runs of each length,
// one pass inserts every run of up to the length that fits at the rank
// that starts it, and one pass stores hi for the runs longer than one
// rank.
// Rank r starts the run of its first k tokens for every k above the common
// prefix (capped at kGramMax) of suffixes r - 1 and r, and ends it for
// every k above that of r and r + 1; all three come from the first 16
// bytes of adjacent key rows.  A run that starts and ends at r (most runs
// of three and four tokens) is stored whole by the insert pass, so the
// second pass looks up only the runs that span several ranks.

#include "gram.h"
#include "launch.h"

namespace sfx {

__global__ __launch_bounds__(256) void k_gram_clear(void* table,
                                                    int64_t buckets) {
  uint32_t* counts = gram_counts(table);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
       i < buckets; i += stride)
    counts[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x < kGramMax) {
    GramHeader* hd = reinterpret_cast<GramHeader*>(table);
    hd->runs[threadIdx.x] = 0;
    if (threadIdx.x == 0) hd->kmax = kGramMax;
  }
}

// Leading tokens two runs share (0 .. kGramMax).
__device__ __forceinline__ int common4(const int4& a, const int4& b) {
  if (a.x != b.x) return 0;
  if (a.y != b.y) return 1;
  if (a.z != b.z) return 2;
  return a.w != b.w ? 3 : 4;
}

// Leading real tokens of a run (0 .. kGramMax).
__device__ __forceinline__ int real4(const int4& a) {
  if (!gram_real(a.x)) return 0;
  if (!gram_real(a.y)) return 1;
  if (!gram_real(a.z)) return 2;
  return gram_real(a.w) ? 4 : 3;
}

// The rank's leading tokens and its common prefixes with both neighbours.
struct RankRuns {
  int4 cur;
  int lcp_prev, lcp_next, nreal;
};

__device__ __forceinline__ RankRuns rank_runs(const int32_t* __restrict__ keys,
                                              int kw, int64_t m, int64_t r) {
  RankRuns q;
  q.cur = *reinterpret_cast<const int4*>(keys + r * kw);
  q.lcp_prev =
      r > 0 ? common4(*reinterpret_cast<const int4*>(keys + (r - 1) * kw),
                      q.cur)
            : 0;
  q.lcp_next =
      r + 1 < m
          ? common4(q.cur, *reinterpret_cast<const int4*>(keys + (r + 1) * kw))
          : 0;
  q.nreal = real4(q.cur);
  return q;
}

// Distinct runs of each length: rank r starts one of k tokens for every
// k in (lcp_prev, nreal].  Each thread counts a strided share of the
// ranks; the counts are summed per wave, then per block, then added with
// one atomic per length and block (at most kGramCountBlocks blocks, so
// the few global atomics on the header do not serialise the pass).
constexpr int kGramCountBlocks = 512;

__global__ __launch_bounds__(256) void k_gram_count(
    const int32_t* __restrict__ keys, int kw, int64_t m, void* table) {
  __shared__ uint32_t c[kGramMax];
  if (threadIdx.x < kGramMax) c[threadIdx.x] = 0;
  __syncthreads();
  uint32_t n[kGramMax] = {0, 0, 0, 0};
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < m;
       r += stride) {
    const RankRuns q = rank_runs(keys, kw, m, r);
#pragma unroll
    for (int k = 1; k <= kGramMax; ++k)
      n[k - 1] += (k > q.lcp_prev && k <= q.nreal) ? 1u : 0u;
  }
#pragma unroll
  for (int k = 0; k < kGramMax; ++k) {
    const uint32_t t = (uint32_t)__shfl((int)wave_incl_scan(n[k]), kWave - 1);
    if (lane_id() == 0 && t) atomicAdd(&c[k], t);
  }
  __syncthreads();
  if (threadIdx.x < kGramMax && c[threadIdx.x])
    atomicAdd(&reinterpret_cast<GramHeader*>(table)->runs[threadIdx.x],
              (unsigned long long)c[threadIdx.x]);
}

// The longest run length whose runs of 1 .. k tokens fit the load limit.
__device__ __forceinline__ int gram_kcap(const GramHeader* hd,
                                         int64_t slots) {
  const unsigned long long lim =
      (unsigned long long)slots * kGramLoadNum / kGramLoadDen;
  unsigned long long n = 0;
  int k = 0;
  while (k < kGramMax) {
    n += hd->runs[k];
    if (n > lim) break;
    ++k;
  }
  return k;
}

__global__ __launch_bounds__(256) void k_gram_insert(
    const int32_t* __restrict__ keys, int kw, int64_t m, void* table,
    int64_t slots) {
  GramHeader* hd = reinterpret_cast<GramHeader*>(table);
  const int kcap = gram_kcap(hd, slots);
  if (blockIdx.x == 0 && threadIdx.x == 0) atomicMin(&hd->kmax, (uint32_t)kcap);
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= m) return;
  const RankRuns q = rank_runs(keys, kw, m, r);
  const int kend = q.nreal < kcap ? q.nreal : kcap;
  if (kend <= q.lcp_prev) return;  // every run here started earlier
  uint32_t* counts = gram_counts(table);
  const uint32_t nb = (uint32_t)gram_buckets(slots);
  for (int k = q.lcp_prev + 1; k <= kend; ++k) {
    const int4 t = gram_key(q.cur.x, q.cur.y, q.cur.z, q.cur.w, k);
    const uint32_t h = gram_hash(t);
    // hi is known now when the run ends here; else the close pass sets it
    const uint32_t hi = k > q.lcp_next ? (uint32_t)r + 1 : 0u;
    bool placed = false;
    for (int s = 0; s < kGramSpill && !placed; ++s) {
      const uint32_t bk = gram_probe(h, nb, s);
      const uint32_t pos = atomicAdd(&counts[bk], 1u);
      if (pos < (uint32_t)kGramBucket) {
        char* bucket = gram_bucket(table, slots, bk);
        reinterpret_cast<int4*>(bucket)[pos] = t;
        reinterpret_cast<uint2*>(bucket + 16 * kGramBucket)[pos] =
            make_uint2((uint32_t)r, hi);
        placed = true;
      }
    }
    if (!placed) atomicMin(&hd->kmax, (uint32_t)(k - 1));
  }
}

__global__ __launch_bounds__(256) void k_gram_close(
    const int32_t* __restrict__ keys, int kw, int64_t m, void* table,
    int64_t slots) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= m) return;
  const RankRuns q = rank_runs(keys, kw, m, r);
  // runs ending at r that started before r: lcp_next < k <= lcp_prev,
  // of the lengths the table holds
  const int kt = (int)reinterpret_cast<const GramHeader*>(table)->kmax;
  int kmax = q.lcp_prev < q.nreal ? q.lcp_prev : q.nreal;
  kmax = kmax < kt ? kmax : kt;
  if (kmax <= q.lcp_next) return;
  const uint32_t* counts = gram_counts(table);
  const uint32_t nb = (uint32_t)gram_buckets(slots);
  for (int k = q.lcp_next + 1; k <= kmax; ++k) {
    const int4 t = gram_key(q.cur.x, q.cur.y, q.cur.z, q.cur.w, k);
    const uint32_t h = gram_hash(t);
    bool done = false;
    for (int s = 0; s < kGramSpill && !done; ++s) {
      const uint32_t bk = gram_probe(h, nb, s);
      const uint32_t cnt = counts[bk];
      const uint32_t n = cnt < (uint32_t)kGramBucket ? cnt : kGramBucket;
      char* bucket = gram_bucket(table, slots, bk);
      const int4* bkeys = reinterpret_cast<const int4*>(bucket);
      uint2* ranges = reinterpret_cast<uint2*>(bucket + 16 * kGramBucket);
      for (uint32_t i = 0; i < n; ++i) {
        const int4 a = bkeys[i];
        if (a.x == t.x && a.y == t.y && a.z == t.z && a.w == t.w) {
          ranges[i].y = (uint32_t)r + 1;
          done = true;
          break;
        }
      }
      if (cnt <= (uint32_t)kGramBucket) break;  // absent: the insert failed
    }
  }
}

}  // namespace sfx

using namespace sfx;

static bool gram_slots_ok(int64_t slots) {
  return slots >= kGramBucket && slots % kGramBucket == 0 &&
         slots <= (1ll << 31);
}

extern "C" size_t sfx_gram_table_bytes(int64_t slots) {
  if (!gram_slots_ok(slots)) return 0;
  return gram_table_bytes(slots);
}

extern "C" int sfx_gram_build(const int32_t* keys, int64_t key_width,
                              int64_t m, void* table, int64_t slots,
                              hipStream_t stream) {
  if (!table || !gram_slots_ok(slots) || m < 0 || m > 0x7fffffffLL ||
      key_width < 4 || key_width > 32 || (key_width & 3) ||
      (m > 0 && !keys) || ((uintptr_t)table & 255) ||
      ((uintptr_t)keys & 15))
    return SFX_EINVAL;
  const int64_t nb = gram_buckets(slots);
  const unsigned cblocks =
      (unsigned)(nb / 256 < 1024 ? (nb + 255) / 256 : 1024);
  hipLaunchKernelGGL(k_gram_clear, dim3(cblocks), dim3(256), 0, stream,
                     table, nb);
  if (m > 0) {
    const unsigned blocks = (unsigned)((m + 255) / 256);
    hipLaunchKernelGGL(k_gram_count,
                       dim3(blocks < (unsigned)kGramCountBlocks
                                ? blocks
                                : (unsigned)kGramCountBlocks),
                       dim3(256), 0, stream, keys, (int)key_width, m, table);
    hipLaunchKernelGGL(k_gram_insert, dim3(blocks), dim3(256), 0, stream,
                       keys, (int)key_width, m, table, slots);
    hipLaunchKernelGGL(k_gram_close, dim3(blocks), dim3(256), 0, stream,
                       keys, (int)key_width, m, table, slots);
  }
  return (int)hipGetLastError();
}
