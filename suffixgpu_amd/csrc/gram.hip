// Building the n-gram range table (gram.h) of a suffix array from its key
// rows, on the caller's stream with no host synchronisation: a new epoch,
// then one pass in which every rank that starts a run inserts it with
// hi = lo + 1, then one pass in which every rank that ends a run stores
// hi.  Rank r starts the run of its first k tokens for every k above the
// common prefix (capped at kGramMax) of suffixes r - 1 and r, and ends it
// for every k above that of r and r + 1; both come from the first 16 bytes
// of adjacent key rows.

#include "gram.h"
#include "launch.h"

namespace sfx {

__global__ void k_gram_epoch(GramHeader* h) {
  if (threadIdx.x == 0) {
    const uint32_t e = h->epoch + 1;
    h->epoch = e == 0 ? 1 : e;  // 0 marks a table never built
    h->ok = 1;
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

__device__ __forceinline__ int4 first4(const int4& a, int k) {
  return make_int4(a.x, k > 1 ? a.y : 0, k > 2 ? a.z : 0, k > 3 ? a.w : 0);
}

__global__ __launch_bounds__(256) void k_gram_insert(
    const int32_t* __restrict__ keys, int kw, int64_t m, void* table,
    uint32_t mask) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= m) return;
  GramHeader* hdr = reinterpret_cast<GramHeader*>(table);
  GramSlot* slots = gram_slots(table);
  const uint32_t ep = hdr->epoch;
  const int4 cur = *reinterpret_cast<const int4*>(keys + r * kw);
  const int lcp =
      r > 0 ? common4(*reinterpret_cast<const int4*>(keys + (r - 1) * kw),
                      cur)
            : 0;
  const int nreal = real4(cur);
  for (int k = lcp + 1; k <= nreal; ++k) {
    const int4 t = first4(cur, k);
    const uint32_t h = gram_hash(t.x, t.y, t.z, t.w, k);
    bool placed = false;
    for (int p = 0; p < kGramProbes && !placed; ++p) {
      GramSlot& s = slots[(h + (uint32_t)p) & mask];
      const uint32_t e = s.epoch;
      if (e == ep) continue;
      if (atomicCAS(&s.epoch, e, ep) != e) continue;  // taken meanwhile
      *reinterpret_cast<int4*>(&s.t[0]) = t;
      s.lo = (uint32_t)r;
      s.hi = (uint32_t)r + 1;
      s.k = (uint32_t)k;
      placed = true;
    }
    if (!placed) hdr->ok = 0;
  }
}

__global__ __launch_bounds__(256) void k_gram_close(
    const int32_t* __restrict__ keys, int kw, int64_t m, void* table,
    uint32_t mask) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= m) return;
  GramHeader* hdr = reinterpret_cast<GramHeader*>(table);
  GramSlot* slots = gram_slots(table);
  const uint32_t ep = hdr->epoch;
  const int4 cur = *reinterpret_cast<const int4*>(keys + r * kw);
  const int lcp =
      r + 1 < m
          ? common4(cur, *reinterpret_cast<const int4*>(keys + (r + 1) * kw))
          : 0;
  const int nreal = real4(cur);
  for (int k = lcp + 1; k <= nreal; ++k) {
    const int4 t = first4(cur, k);
    const uint32_t h = gram_hash(t.x, t.y, t.z, t.w, k);
    for (int p = 0; p < kGramProbes; ++p) {
      GramSlot& s = slots[(h + (uint32_t)p) & mask];
      if (s.epoch != ep) break;  // not stored: the insert pass failed
      if ((int)s.k == k && s.t[0] == t.x && s.t[1] == t.y &&
          s.t[2] == t.z && s.t[3] == t.w) {
        s.hi = (uint32_t)r + 1;
        break;
      }
    }
  }
}

}  // namespace sfx

using namespace sfx;

extern "C" size_t sfx_gram_table_bytes(int64_t slots) {
  if (slots < 1 || (slots & (slots - 1))) return 0;
  return gram_table_bytes(slots);
}

extern "C" int sfx_gram_build(const int32_t* keys, int64_t key_width,
                              int64_t m, void* table, int64_t slots,
                              hipStream_t stream) {
  if (!table || slots < 1 || (slots & (slots - 1)) || slots > (1ll << 31) ||
      m < 0 || m > 0x7fffffffLL || key_width < 4 || key_width > 32 ||
      (key_width & 3) || (m > 0 && !keys) ||
      ((uintptr_t)table & 255) || ((uintptr_t)keys & 15))
    return SFX_EINVAL;
  hipLaunchKernelGGL(k_gram_epoch, dim3(1), dim3(64), 0, stream,
                     reinterpret_cast<GramHeader*>(table));
  if (m > 0) {
    const unsigned blocks = (unsigned)((m + 255) / 256);
    const uint32_t mask = (uint32_t)(slots - 1);
    hipLaunchKernelGGL(k_gram_insert, dim3(blocks), dim3(256), 0, stream,
                       keys, (int)key_width, m, table, mask);
    hipLaunchKernelGGL(k_gram_close, dim3(blocks), dim3(256), 0, stream,
                       keys, (int)key_width, m, table, mask);
  }
  return (int)hipGetLastError();
}
