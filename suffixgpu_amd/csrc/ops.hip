// Standalone operators at the reference's kernel boundary
// (suffix_gpu/triton_kernels.py): scatter_append, match_back,
// first_occurrences, sa_search and expand_chain.  The fused decode step
// uses the same device building blocks; these entry points expose them one
// at a time for the index-level API and for parity checks.

#include <algorithm>

#include "launch.h"
#include "pick.h"
#include "sa_search.h"
#include "sfx_common.h"

namespace sfx {

// ---------------------------------------------------------- scatter_append
__global__ __launch_bounds__(64) void k_scatter(sfx_batch bt,
                                                int32_t* new_counts) {
  const int b = blockIdx.x;
  const RowState st = row_state(bt, b);
  const int64_t S = bt.seq;
  const int32_t* sp = bt.sampled + (int64_t)b * bt.num_sampled;
  for (int64_t j = threadIdx.x; j < bt.num_sampled; j += blockDim.x) {
    const int64_t pos = st.base + j;
    const int32_t v = sp[j];
    if (j < st.cnt && v != -1 && pos < S && pos >= 0)
      bt.tokens[(int64_t)b * S + pos] = v;
  }
  if (new_counts && threadIdx.x == 0) new_counts[b] = (int32_t)st.q;
}

// ---------------------------------------------------------- index swap
// Up to three buffer copies in one grid-stride launch: 16-byte words where
// both sides are 16-byte aligned, single words for the rest.
struct CopySpan {
  int32_t* dst;
  const int32_t* src;
  int64_t n;
};

__device__ __forceinline__ void copy_span(const CopySpan& c, int64_t tid,
                                          int64_t nthreads) {
  if (c.n <= 0) return;
  const bool vec = ((reinterpret_cast<uintptr_t>(c.dst) |
                     reinterpret_cast<uintptr_t>(c.src)) & 15u) == 0;
  const int64_t n4 = vec ? c.n / 4 : 0;
  const int4* s4 = reinterpret_cast<const int4*>(c.src);
  int4* d4 = reinterpret_cast<int4*>(c.dst);
  for (int64_t i = tid; i < n4; i += nthreads) d4[i] = s4[i];
  for (int64_t i = 4 * n4 + tid; i < c.n; i += nthreads) c.dst[i] = c.src[i];
}

// The swap's in-place copies of corpus and SA; block 0 also stores the
// key-row selector word (a vector store from one lane).
__global__ __launch_bounds__(256) void k_swap(CopySpan a, CopySpan b,
                                              int32_t* key_select,
                                              int32_t key_select_value) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nth = (int64_t)gridDim.x * blockDim.x;
  copy_span(a, tid, nth);
  copy_span(b, tid, nth);
  if (key_select && tid == 0) *key_select = key_select_value;
}

// ------------------------------------------------------------ delta writes
// Appends up to SFX_APPEND_MAX_DOCS documents: block (x, d) copies a
// grid-stride share of document d, block (0, d) also writes its SEP and
// block (0, 0) the new delta length.
struct AppendDocs {
  sfx_append_doc doc[SFX_APPEND_MAX_DOCS];
};

__global__ __launch_bounds__(256) void k_delta_append(AppendDocs docs,
                                                      int32_t* delta,
                                                      int64_t* delta_len,
                                                      int64_t new_len) {
  const sfx_append_doc& d = docs.doc[blockIdx.y];
  int32_t* out = delta + d.dst;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nth = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = tid; i < d.n; i += nth) out[i] = d.src[i];
  if (tid == 0) out[d.n] = kSep;
  if (tid == 0 && blockIdx.y == 0 && delta_len) *delta_len = new_len;
}

// delta[0 .. n) = delta[from .. from + n) in place (from > 0), by one
// block in ascending windows: a window's sources are all read before the
// barrier, and its writes only land on sources of outputs at or below the
// window, which are read already.
constexpr int kShiftThreads = 1024;
constexpr int kShiftPer = 8;

__global__ __launch_bounds__(kShiftThreads) void k_delta_shift(
    int32_t* delta, int64_t from, int64_t n, int64_t* delta_len,
    int64_t new_len) {
  constexpr int64_t W = (int64_t)kShiftThreads * kShiftPer;
  for (int64_t k = 0; k < n; k += W) {
    int32_t v[kShiftPer];
#pragma unroll
    for (int u = 0; u < kShiftPer; ++u) {
      const int64_t o = k + u * kShiftThreads + threadIdx.x;
      v[u] = o < n ? delta[from + o] : 0;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kShiftPer; ++u) {
      const int64_t o = k + u * kShiftThreads + threadIdx.x;
      if (o < n) delta[o] = v[u];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && delta_len) *delta_len = new_len;
}

// -------------------------------------------------------------- match_back
__global__ __launch_bounds__(256) void k_match_back(
    const int32_t* __restrict__ src, int64_t row_stride,
    const int32_t* __restrict__ pat, int P, int64_t n_out, int32_t* out) {
  const int b = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_out) return;
  const int32_t* base = src + (int64_t)b * row_stride;
  const int32_t* pb = pat + (int64_t)b * P;
  int m = 0;
  for (int t = 0; t < P; ++t) {
    const int64_t j = i - 1 - t;
    const int32_t x = j >= 0 ? base[j] : -1;
    if (x != pb[t]) break;
    ++m;
  }
  out[(int64_t)b * n_out + i] = m;
}

// ------------------------------------------------------- first_occurrences
constexpr int kOccThreads = 256;

__global__ __launch_bounds__(kOccThreads) void k_first_occ(
    const int32_t* __restrict__ mb, int64_t n_cols,
    const int64_t* __restrict__ thr, int64_t per_row, int R, int64_t* pos,
    int64_t* count) {
  __shared__ int wcnt[kOccThreads / kWave];
  __shared__ int sfound;
  const int64_t row = blockIdx.x;
  const int64_t b = row / per_row;
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int64_t t = thr[row];
  const int32_t* src = mb + b * n_cols;
  int64_t* out = pos + row * R;
  if (tid == 0) sfound = 0;
  __syncthreads();
  if (t > 0) {
    for (int64_t base = 0; base < n_cols; base += kOccThreads) {
      const int64_t i = base + tid;
      const bool hit = i < n_cols && (int64_t)src[i] >= t;
      const uint64_t bm = ballot(hit);
      if (lane_id() == 0) wcnt[wv] = popc(bm);
      __syncthreads();
      int off = sfound;
      int tot = 0;
      for (int w = 0; w < kOccThreads / kWave; ++w) {
        if (w < wv) off += wcnt[w];
        tot += wcnt[w];
      }
      if (hit) {
        const int slot = off + rank_lt(bm);
        if (slot < R) out[slot] = i;
      }
      __syncthreads();
      if (tid == 0) sfound += tot;
      __syncthreads();
      if (sfound >= R) break;
    }
  }
  const int f = sfound < R ? sfound : R;
  for (int r = tid; r < R; r += kOccThreads)
    if (r >= f) out[r] = 0;
  if (tid == 0) count[row] = f;
}

// --------------------------------------------------------------- sa_search
constexpr int kSearchThreads = 256;
constexpr int kOpGroup = 8;

__global__ __launch_bounds__(kSearchThreads) void k_sa_search(
    const int32_t* __restrict__ sa, const int32_t* __restrict__ corpus,
    int64_t n, const int32_t* __restrict__ pattern, int64_t batch,
    int64_t width, const int64_t* __restrict__ plen, int64_t* lower,
    int64_t* upper) {
  const int64_t row =
      (int64_t)blockIdx.x * (kSearchThreads / kOpGroup) +
      threadIdx.x / kOpGroup;
  if (row >= batch) return;  // whole groups exit together
  const int32_t* pr = pattern + row * width;
  int64_t pl = plen[row];
  pl = pl < 0 ? 0 : (pl > width ? width : pl);
  auto pat_at = [&](int j) -> int32_t { return pr[j]; };
  int64_t lo, hi;
  kary_bounds<kOpGroup>(sa, corpus, n, nullptr, 0, pat_at, (int)pl, lo, hi,
                        0u, (uint32_t)n);
  if (threadIdx.x % kOpGroup == 0) {
    lower[row] = lo;
    upper[row] = hi;
  }
}

// ------------------------------------------------------------ expand_chain
struct ExpandArgs {
  const int32_t* cont;
  int64_t rows;
  int R;
  int K;
  const int64_t* num_occ;
  const int64_t* cap;
  const float* weights;
  float min_prob;
  float alpha;
  int32_t* chain;
  int64_t* num_valid;
  int64_t* num_emit;
  float* score;
  int waves_per_block;
};

__host__ __device__ inline int round16(int x) { return (x + 15) & ~15; }

// Per-wave LDS: continuation cache [R, K + 1], vote buffer A [R],
// weights W [R],
// chain [K]; every region 16-byte aligned.
__host__ __device__ inline int expand_wave_bytes(int R, int K) {
  return round16(R * (K + 1) * 4) + 2 * round16(R * 4) + round16(K * 4) +
         2 * kHashSlots * 4;
}

template <bool kWeighted>
__global__ __launch_bounds__(256) void k_expand(ExpandArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int wv = threadIdx.x / kWave;
  const int ln = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * a.waves_per_block + wv;
  if (wv >= a.waves_per_block || row >= a.rows) return;
  const int R = a.R;
  const int K = a.K;
  unsigned char* base = smem + (size_t)wv * expand_wave_bytes(R, K);
  const int cb = round16(R * (K + 1) * 4);
  int32_t* cache = (int32_t*)base;
  int32_t* A = (int32_t*)(base + cb);
  float* W = (float*)(base + cb + round16(R * 4));
  int32_t* chain = (int32_t*)(base + cb + 2 * round16(R * 4));
  int32_t* H = (int32_t*)(base + cb + 2 * round16(R * 4) + round16(K * 4));
  const int32_t* src = a.cont + row * R * K;
  // rows K + 1 words apart (an odd stride): one depth's rows fall in
  // distinct LDS banks for the expansion's per-lane reads
  for (int e = ln; e < R * K; e += kWave)
    cache[(e / K) * (K + 1) + e % K] = src[e];
  wave_lds_sync();
  const int64_t occ = a.num_occ[row];
  const int64_t cap = a.cap ? a.cap[row] : K;
  auto cont_at = [&](int r, int d) -> int32_t { return cache[r * (K + 1) + d]; };
  const float* wrow = a.weights ? a.weights + row * R : nullptr;
  auto w_at = [&](int r) -> float { return wrow[r]; };
  ExpandResult er;
  if (kWeighted)
    er = expand_wave<true>(cont_at, w_at, R, occ, K, cap, a.min_prob,
                           a.alpha, A, W, H, chain);
  else
    er = expand_wave<false>(cont_at, NoWeight(), R, occ, K, cap, a.min_prob,
                            a.alpha, A, W, H, chain);
  wave_lds_sync();
  for (int d = ln; d < K; d += kWave) a.chain[row * K + d] = chain[d];
  if (ln == 0) {
    const int64_t cap0 = cap > 0 ? cap : 0;
    a.num_valid[row] = er.nv;
    a.num_emit[row] = er.nv < cap0 ? er.nv : cap0;
    a.score[row] = er.score;
  }
}

}  // namespace sfx

using namespace sfx;

#ifdef SFX_TRACE
__constant__ uint64_t* sfx_trace_buf = nullptr;
__constant__ uint64_t* sfx_trace_stats = nullptr;

// Profiling builds only: per-wave expansion counters (8 u64 per wave).
extern "C" int sfx_trace_stats_set(uint64_t* buf) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(sfx_trace_stats), &buf,
                                sizeof(buf));
}

// Profiling builds only: point the phase-timestamp buffer (device memory,
// 16 u64 per block) at `buf`, or disable with NULL.
extern "C" int sfx_trace_set(uint64_t* buf) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(sfx_trace_buf), &buf,
                                sizeof(buf));
}
#endif

extern "C" int sfx_abi_version(void) { return SFX_ABI_VERSION; }

extern "C" int sfx_index_swap(int32_t* corpus, int32_t* sa,
                              const int32_t* new_corpus,
                              const int32_t* new_sa, int64_t capacity,
                              int32_t* key_select, int32_t key_select_value,
                              hipStream_t stream) {
  if (capacity < 0) return SFX_EINVAL;
  if (capacity == 0 && !key_select) return 0;
  if (capacity > 0 && (!corpus || !sa || !new_corpus || !new_sa))
    return SFX_EINVAL;
  const CopySpan a{corpus, new_corpus, capacity};
  const CopySpan b{sa, new_sa, capacity};
  // Up to eight 256-thread blocks per CU keep every CU streaming (32 MiB
  // of copies at N = 2^22).
  const int64_t want = (capacity / 4 + 255) / 256;
  const unsigned blocks =
      (unsigned)(want < 1 ? 1 : (want > 2048 ? 2048 : want));
  hipLaunchKernelGGL(k_swap, dim3(blocks), dim3(256), 0, stream, a, b,
                     key_select, key_select_value);
  return (int)hipGetLastError();
}

extern "C" int sfx_delta_append(const sfx_append_doc* docs, int32_t ndocs,
                                int32_t* delta, int64_t delta_capacity,
                                int64_t* delta_len, int64_t new_len,
                                hipStream_t stream) {
  if (ndocs < 0 || delta_capacity < 0 || new_len < 0 ||
      new_len > delta_capacity || (ndocs > 0 && (!docs || !delta)))
    return SFX_EINVAL;
  int64_t longest = 0;
  for (int32_t i = 0; i < ndocs; ++i) {
    const sfx_append_doc& d = docs[i];
    if (d.n < 0 || d.dst < 0 || d.dst + d.n + 1 > delta_capacity ||
        (d.n > 0 && !d.src))
      return SFX_EINVAL;
    longest = d.n > longest ? d.n : longest;
  }
  if (ndocs == 0) {
    if (!delta_len) return 0;
    hipLaunchKernelGGL(k_delta_shift, dim3(1), dim3(kShiftThreads), 0,
                       stream, delta, (int64_t)0, (int64_t)0, delta_len,
                       new_len);
    return (int)hipGetLastError();
  }
  const unsigned bx = (unsigned)std::min<int64_t>(
      std::max<int64_t>((longest + 1023) / 1024, 1), 64);
  for (int32_t g = 0; g < ndocs; g += SFX_APPEND_MAX_DOCS) {
    const int32_t cnt = std::min<int32_t>(ndocs - g, SFX_APPEND_MAX_DOCS);
    AppendDocs a = {};
    for (int32_t i = 0; i < cnt; ++i) a.doc[i] = docs[g + i];
    hipLaunchKernelGGL(k_delta_append, dim3(bx, (unsigned)cnt), dim3(256), 0,
                       stream, a, delta, delta_len, new_len);
    const int rc = (int)hipGetLastError();
    if (rc) return rc;
  }
  return 0;
}

extern "C" int sfx_delta_shift(int32_t* delta, int64_t delta_capacity,
                               int64_t from, int64_t n, int64_t* delta_len,
                               hipStream_t stream) {
  if (!delta || from < 0 || n < 0 || from + n > delta_capacity)
    return SFX_EINVAL;
  if (from == 0 && !delta_len) return 0;
  hipLaunchKernelGGL(k_delta_shift, dim3(1), dim3(kShiftThreads), 0, stream,
                     delta, from, from > 0 ? n : 0, delta_len, n);
  return (int)hipGetLastError();
}

extern "C" int sfx_scatter_append(const sfx_batch* bt, int32_t* new_counts,
                                  hipStream_t stream) {
  if (!bt || bt->batch < 0 || bt->seq < 1 || !bt->tokens ||
      !bt->num_tokens || !bt->sampled || bt->num_sampled < 0)
    return SFX_EINVAL;
  if (bt->batch == 0) return 0;
  hipLaunchKernelGGL(k_scatter, dim3((unsigned)bt->batch), dim3(64), 0,
                     stream, *bt, new_counts);
  return (int)hipGetLastError();
}

extern "C" int sfx_match_back(const int32_t* src, int64_t row_stride,
                              const int32_t* pat, int64_t batch,
                              int64_t pattern_len, int64_t n_out,
                              int32_t* out, hipStream_t stream) {
  if (batch < 0 || pattern_len < 0 || n_out < 0 || row_stride < 0)
    return SFX_EINVAL;
  if (batch == 0 || n_out == 0) return 0;
  if (!src || !out || (pattern_len > 0 && !pat)) return SFX_EINVAL;
  if (batch > 65535) return SFX_EINVAL;
  dim3 grid((unsigned)((n_out + 255) / 256), (unsigned)batch);
  hipLaunchKernelGGL(k_match_back, grid, dim3(256), 0, stream, src,
                     row_stride, pat, (int)pattern_len, n_out, out);
  return (int)hipGetLastError();
}

extern "C" int sfx_first_occurrences(const int32_t* mb, int64_t n_cols,
                                     const int64_t* thr, int64_t rows,
                                     int64_t per_row, int64_t max_occ,
                                     int64_t* pos, int64_t* count,
                                     hipStream_t stream) {
  if (rows < 0 || n_cols < 0 || per_row < 1 || max_occ < 1) return SFX_EINVAL;
  if (rows == 0) return 0;
  if (!mb || !thr || !pos || !count) return SFX_EINVAL;
  if (max_occ > 0x7fffffff) return SFX_EINVAL;
  hipLaunchKernelGGL(k_first_occ, dim3((unsigned)rows), dim3(kOccThreads), 0,
                     stream, mb, n_cols, thr, per_row, (int)max_occ, pos,
                     count);
  return (int)hipGetLastError();
}

extern "C" int sfx_sa_search(const int32_t* sa, const int32_t* corpus,
                             int64_t n, const int32_t* pattern,
                             int64_t batch, int64_t width,
                             const int64_t* plen, int64_t* lower,
                             int64_t* upper, hipStream_t stream) {
  if (batch < 0 || n < 1 || n > 0x7fffffffLL || width < 0) return SFX_EINVAL;
  if (batch == 0) return 0;
  if (!sa || !corpus || !plen || !lower || !upper ||
      (width > 0 && !pattern))
    return SFX_EINVAL;
  const int64_t per_block = kSearchThreads / kOpGroup;
  const int64_t blocks = (batch + per_block - 1) / per_block;
  hipLaunchKernelGGL(k_sa_search, dim3((unsigned)blocks),
                     dim3(kSearchThreads), 0, stream, sa, corpus, n, pattern,
                     batch, width, plen, lower, upper);
  return (int)hipGetLastError();
}

extern "C" int sfx_expand_chain(const int32_t* cont, int64_t rows,
                                int64_t max_occ, int64_t k,
                                const int64_t* num_occ, const int64_t* cap,
                                const float* weights, float min_token_prob,
                                float alpha, int32_t* chain,
                                int64_t* num_valid, int64_t* num_emit,
                                float* score, hipStream_t stream) {
  if (rows < 0 || max_occ < 1 || max_occ > 2048 || k < 1 || k > 4096)
    return SFX_EINVAL;
  if (rows == 0) return 0;
  if (!cont || !num_occ || !chain || !num_valid || !num_emit || !score)
    return SFX_EINVAL;
  ExpandArgs a;
  a.cont = cont;
  a.rows = rows;
  a.R = (int)max_occ;
  a.K = (int)k;
  a.num_occ = num_occ;
  a.cap = cap;
  a.weights = weights;
  a.min_prob = min_token_prob;
  a.alpha = alpha;
  a.chain = chain;
  a.num_valid = num_valid;
  a.num_emit = num_emit;
  a.score = score;
  const size_t per_wave = (size_t)expand_wave_bytes(a.R, a.K);
  if (per_wave > kMaxLds) return SFX_EINVAL;
  int wpb = (int)(kMaxLds / per_wave);
  wpb = wpb > 4 ? 4 : wpb;
  a.waves_per_block = wpb;
  const int64_t blocks = (rows + wpb - 1) / wpb;
  const size_t lds = per_wave * (size_t)wpb;
  static std::atomic<uint64_t> lds_opt_w{0};
  allow_max_lds((const void*)k_expand<true>, lds_opt_w);
  static std::atomic<uint64_t> lds_opt_u{0};
  allow_max_lds((const void*)k_expand<false>, lds_opt_u);
  if (weights)
    hipLaunchKernelGGL(k_expand<true>, dim3((unsigned)blocks), dim3(256),
                       lds, stream, a);
  else
    hipLaunchKernelGGL(k_expand<false>, dim3((unsigned)blocks), dim3(256),
                       lds, stream, a);
  return (int)hipGetLastError();
}
