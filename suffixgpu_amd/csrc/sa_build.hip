// Suffix-array construction on the GPU: prefix doubling over LSD radix
// sorts, with no host synchronisation.
//
// Round 0 sorts positions by token (signed order, 4 passes of 8 bits).
// Round h sorts them by (rank[i], rank[i+h]+1 or 0), rank = SA position of
// the first suffix of the same h-prefix group; a proper prefix sorts first,
// as in suffix_gpu/suffix_array.py:15-63.  After each sort a device-wide
// max-scan of group-start flags yields the new ranks and a device flag
// records whether every rank is distinct; all later rounds then return at
// their first instruction, so the fixed launch sequence (capturable, no
// host reads) costs only empty launches once the array is final.
//
// Each LSD pass is histogram -> single-block exclusive scan -> stable
// scatter; the scatter ranks equal digits inside a wave with eight ballots
// (wave64 match) and across waves through LDS, keeping tile order.

#include "launch.h"
#include "sfx_common.h"

namespace sfx {

constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kTile = kSortThreads * kSortItems;  // 4096
constexpr int kRadix = 256;

struct SaWs {
  uint64_t* keyA;
  uint64_t* keyB;
  uint32_t* valA;
  uint32_t* valB;
  uint32_t* rank;
  uint32_t* sa;
  uint32_t* hist;    // [256 * NB]
  uint32_t* blkmax;  // [NB]
  uint32_t* blkcnt;  // [NB]
  uint32_t* carry;   // [NB]
  uint32_t* state;   // [0] done, [1] pending
};

static size_t sa_ws_layout(int64_t n, void* base, SaWs* w) {
  const size_t N = (size_t)(n > 0 ? n : 1);
  const size_t NB = (N + kTile - 1) / kTile;
  size_t off = 0;
  char* c = (char*)base;
  auto take = [&](size_t bytes) -> void* {
    void* ptr = c ? (void*)(c + off) : nullptr;
    off += ws_align(bytes);
    return ptr;
  };
  SaWs s;
  s.keyA = (uint64_t*)take(N * 8);
  s.keyB = (uint64_t*)take(N * 8);
  s.valA = (uint32_t*)take(N * 4);
  s.valB = (uint32_t*)take(N * 4);
  s.rank = (uint32_t*)take(N * 4);
  s.sa = (uint32_t*)take(N * 4);
  s.hist = (uint32_t*)take((size_t)kRadix * NB * 4);
  s.blkmax = (uint32_t*)take(NB * 4);
  s.blkcnt = (uint32_t*)take(NB * 4);
  s.carry = (uint32_t*)take(NB * 4);
  s.state = (uint32_t*)take(256);
  if (w) *w = s;
  return off;
}

__global__ void k_sa_reset(uint32_t* state) {
  if (threadIdx.x == 0) {
    state[0] = 0;
    state[1] = 0;
  }
}

__global__ void k_sa_commit(uint32_t* state) {
  if (threadIdx.x == 0 && state[0] == 0) state[0] = state[1];
}

__global__ __launch_bounds__(256) void k_sa_init(const int32_t* text,
                                                 int64_t n, uint64_t* key,
                                                 uint32_t* val) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  key[i] = (uint64_t)((uint32_t)text[i] ^ 0x80000000u);
  val[i] = (uint32_t)i;
}

__global__ __launch_bounds__(256) void k_sa_keys(const uint32_t* sa,
                                                 const uint32_t* rank,
                                                 int64_t n, int64_t h,
                                                 uint64_t* key, uint32_t* val,
                                                 const uint32_t* state) {
  if (state[0]) return;
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const uint32_t i = sa[j];
  const uint64_t k1 = rank[i];
  const uint64_t k2 = (int64_t)i + h < n ? (uint64_t)rank[i + h] + 1 : 0;
  key[j] = k1 * (uint64_t)(n + 1) + k2;
  val[j] = i;
}

// Lanes of the wave holding the same 8-bit digit as the calling lane.
__device__ __forceinline__ uint64_t match_digit(bool act, uint32_t d) {
  uint64_t peers = ballot(act);
#pragma unroll
  for (int bit = 0; bit < 8; ++bit) {
    const bool set = (d >> bit) & 1u;
    const uint64_t m = ballot(act && set);
    peers &= set ? m : ~m;
  }
  return peers;
}

__global__ __launch_bounds__(kSortThreads) void k_rs_hist(
    const uint64_t* __restrict__ key, int64_t n, int sh, uint32_t* hist,
    int64_t nb, const uint32_t* state) {
  if (state[0]) return;
  __shared__ uint32_t h[kRadix];
  const int tid = threadIdx.x;
  h[tid] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kTile;
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t idx = base + (int64_t)r * kSortThreads + tid;
    const bool act = idx < n;
    const uint32_t d = act ? (uint32_t)(key[idx] >> sh) & 255u : 0u;
    const uint64_t peers = match_digit(act, d);
    if (act && rank_lt(peers) == 0) atomicAdd(&h[d], (uint32_t)popc(peers));
  }
  __syncthreads();
  hist[(int64_t)tid * nb + blockIdx.x] = h[tid];
}

// In-place exclusive scan of `total` u32 by one 1024-thread block.
__global__ __launch_bounds__(1024) void k_scan_excl(uint32_t* a,
                                                    int64_t total,
                                                    const uint32_t* state) {
  if (state && state[0]) return;
  __shared__ uint32_t part[1024];
  const int tid = threadIdx.x;
  const int64_t per = (total + 1023) / 1024;
  const int64_t lo = (int64_t)tid * per;
  const int64_t hi = lo + per < total ? lo + per : total;
  uint32_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += a[i];
  part[tid] = s;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const uint32_t v = tid >= o ? part[tid - o] : 0u;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  uint32_t run = part[tid] - s;
  for (int64_t i = lo; i < hi; ++i) {
    const uint32_t v = a[i];
    a[i] = run;
    run += v;
  }
}

__global__ __launch_bounds__(kSortThreads) void k_rs_scatter(
    const uint64_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint64_t* __restrict__ kout, uint32_t* __restrict__ vout, int64_t n,
    int sh, const uint32_t* __restrict__ offs, int64_t nb,
    const uint32_t* state) {
  if (state[0]) return;
  constexpr int NW = kSortThreads / kWave;
  __shared__ uint32_t gofs[kRadix];
  __shared__ uint32_t whist[NW][kRadix];
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  gofs[tid] = offs[(int64_t)tid * nb + blockIdx.x];
  for (int w = 0; w < NW; ++w) whist[w][tid] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kTile;
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t idx = base + (int64_t)r * kSortThreads + tid;
    const bool act = idx < n;
    const uint64_t k = act ? kin[idx] : 0;
    const uint32_t v = act ? vin[idx] : 0;
    const uint32_t d = (uint32_t)(k >> sh) & 255u;
    const uint64_t peers = match_digit(act, d);
    const int rk = rank_lt(peers);
    if (act && rk == 0) whist[wv][d] = (uint32_t)popc(peers);
    __syncthreads();
    if (act) {
      uint32_t pos = gofs[d] + (uint32_t)rk;
      for (int w = 0; w < wv; ++w) pos += whist[w][d];
      kout[pos] = k;
      vout[pos] = v;
    }
    __syncthreads();
    uint32_t add = 0;
    for (int w = 0; w < NW; ++w) {
      add += whist[w][tid];
      whist[w][tid] = 0;
    }
    gofs[tid] += add;
    __syncthreads();
  }
}

// Group starts: flag[j] = j == 0 || key[j] != key[j-1].
__global__ __launch_bounds__(kSortThreads) void k_grp_reduce(
    const uint64_t* __restrict__ key, int64_t n, uint32_t* blkmax,
    uint32_t* blkcnt, const uint32_t* state) {
  if (state[0]) return;
  __shared__ uint32_t smax[kSortThreads / kWave];
  __shared__ uint32_t scnt[kSortThreads / kWave];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kTile;
  uint32_t mx = 0, cnt = 0;
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t j = base + (int64_t)r * kSortThreads + tid;
    if (j < n && (j == 0 || key[j] != key[j - 1])) {
      mx = (uint32_t)j;
      ++cnt;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
    cnt += (uint32_t)__shfl_xor((int)cnt, o);
  }
  if (lane_id() == 0) {
    smax[tid / kWave] = mx;
    scnt[tid / kWave] = cnt;
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t m = 0, c = 0;
    for (int w = 0; w < kSortThreads / kWave; ++w) {
      m = max(m, smax[w]);
      c += scnt[w];
    }
    blkmax[blockIdx.x] = m;
    blkcnt[blockIdx.x] = c;
  }
}

// Carry-in of the max-scan per block and the all-distinct flag.
__global__ __launch_bounds__(1024) void k_grp_carry(const uint32_t* blkmax,
                                                    const uint32_t* blkcnt,
                                                    uint32_t* carry,
                                                    int64_t nb, int64_t n,
                                                    uint32_t* state) {
  if (state[0]) return;
  __shared__ uint32_t pm[1024];
  __shared__ uint64_t pc[1024];
  const int tid = threadIdx.x;
  const int64_t per = (nb + 1023) / 1024;
  const int64_t lo = (int64_t)tid * per;
  const int64_t hi = lo + per < nb ? lo + per : nb;
  uint32_t m = 0;
  uint64_t c = 0;
  for (int64_t i = lo; i < hi; ++i) {
    m = max(m, blkmax[i]);
    c += blkcnt[i];
  }
  pm[tid] = m;
  pc[tid] = c;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const uint32_t vm = tid >= o ? pm[tid - o] : 0u;
    const uint64_t vc = tid >= o ? pc[tid - o] : 0u;
    __syncthreads();
    pm[tid] = max(pm[tid], vm);
    pc[tid] += vc;
    __syncthreads();
  }
  uint32_t run = tid > 0 ? pm[tid - 1] : 0u;
  for (int64_t i = lo; i < hi; ++i) {
    carry[i] = run;
    run = max(run, blkmax[i]);
  }
  if (tid == 1023) state[1] = pc[1023] == (uint64_t)n ? 1u : 0u;
}

// head[j] = last group start <= j; rank[sa[j]] = head[j].
__global__ __launch_bounds__(kSortThreads) void k_grp_rank(
    const uint64_t* __restrict__ key, const uint32_t* __restrict__ val,
    int64_t n, const uint32_t* __restrict__ carry, uint32_t* rank,
    uint32_t* sa, const uint32_t* state) {
  if (state[0]) return;
  __shared__ uint32_t part[kSortThreads];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kTile + (int64_t)tid * kSortItems;
  uint32_t mx = 0;
  for (int u = 0; u < kSortItems; ++u) {
    const int64_t j = base + u;
    if (j < n && (j == 0 || key[j] != key[j - 1])) mx = (uint32_t)j;
  }
  part[tid] = mx;
  __syncthreads();
  for (int o = 1; o < kSortThreads; o <<= 1) {
    const uint32_t v = tid >= o ? part[tid - o] : 0u;
    __syncthreads();
    part[tid] = max(part[tid], v);
    __syncthreads();
  }
  uint32_t run = max(carry[blockIdx.x], tid > 0 ? part[tid - 1] : 0u);
  for (int u = 0; u < kSortItems; ++u) {
    const int64_t j = base + u;
    if (j >= n) break;
    if (j == 0 || key[j] != key[j - 1]) run = (uint32_t)j;
    const uint32_t i = val[j];
    rank[i] = run;
    sa[j] = i;
  }
}

// keys[r * W + j] = corpus[sa[r] + j] (-1 at or past n).
__global__ __launch_bounds__(256) void k_rank_keys(const int32_t* corpus,
                                                 const int32_t* sa, int64_t n,
                                                 int W, int32_t* keys) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n * W) return;
  const int64_t r = e / W;
  const int j = (int)(e - r * W);
  const int64_t pos = (int64_t)sa[r] + j;
  keys[e] = pos < n && pos >= 0 ? corpus[pos] : -1;
}

template <typename T>
__global__ __launch_bounds__(256) void k_sa_out(const uint32_t* sa, int64_t m,
                                                int64_t n_total, T* out) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n_total) return;
  out[j] = j < m ? (T)sa[j] : (T)j;
}

static int bits_for(uint64_t maxval) {
  int b = 0;
  while (b < 64 && (maxval >> b) != 0) ++b;
  return b;
}

}  // namespace sfx

using namespace sfx;

extern "C" int sfx_sa_keys(const int32_t* corpus, const int32_t* sa,
                           int64_t n, int64_t width, int32_t* keys,
                           hipStream_t stream) {
  if (n < 0 || width < 4 || width > 32 || (width & 3)) return SFX_EINVAL;
  if (n == 0) return 0;
  if (!corpus || !sa || !keys) return SFX_EINVAL;
  const int64_t total = n * width;
  hipLaunchKernelGGL(k_rank_keys, dim3((unsigned)((total + 255) / 256)),
                     dim3(256), 0, stream, corpus, sa, n, (int)width, keys);
  return (int)hipGetLastError();
}

extern "C" size_t sfx_sa_build_workspace_size(int64_t m) {
  if (m < 0) return 0;
  return sa_ws_layout(m, nullptr, nullptr);
}

extern "C" int sfx_sa_build(const int32_t* text, int64_t m, int64_t n_total,
                            void* sa_out, int32_t sa_is64, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
  if (m < 0 || n_total < m || m > 0x7fffffffLL || n_total > 0x7fffffffLL)
    return SFX_EINVAL;
  if (n_total == 0) return 0;
  if (!sa_out || (m > 0 && !text)) return SFX_EINVAL;
  const size_t need = sa_ws_layout(m, nullptr, nullptr);
  if (m > 1 && (!workspace || workspace_bytes < need)) return SFX_EINVAL;
  const unsigned out_blocks = (unsigned)((n_total + 255) / 256);
  if (m <= 1) {
    // SA of zero or one symbol is the identity.
    if (sa_is64)
      hipLaunchKernelGGL(k_sa_out<int64_t>, dim3(out_blocks), dim3(256), 0,
                         stream, (const uint32_t*)nullptr, (int64_t)0,
                         n_total, (int64_t*)sa_out);
    else
      hipLaunchKernelGGL(k_sa_out<int32_t>, dim3(out_blocks), dim3(256), 0,
                         stream, (const uint32_t*)nullptr, (int64_t)0,
                         n_total, (int32_t*)sa_out);
    return (int)hipGetLastError();
  }
  SaWs w;
  sa_ws_layout(m, workspace, &w);
  const int64_t nb = (m + kTile - 1) / kTile;
  const unsigned eb = (unsigned)((m + 255) / 256);
  hipLaunchKernelGGL(k_sa_reset, dim3(1), dim3(64), 0, stream, w.state);
  hipLaunchKernelGGL(k_sa_init, dim3(eb), dim3(256), 0, stream, text, m,
                     w.keyA, w.valA);
  int rounds = 0;
  while ((1LL << rounds) < m) ++rounds;  // ceil(log2 m)
  for (int round = 0; round <= rounds; ++round) {
    int nbits;
    if (round == 0) {
      nbits = 32;
    } else {
      const int64_t h = 1LL << (round - 1);
      hipLaunchKernelGGL(k_sa_keys, dim3(eb), dim3(256), 0, stream, w.sa,
                         w.rank, m, h, w.keyA, w.valA, w.state);
      const uint64_t maxkey =
          (uint64_t)(m - 1) * (uint64_t)(m + 1) + (uint64_t)m;
      nbits = bits_for(maxkey);
    }
    uint64_t* kin = w.keyA;
    uint32_t* vin = w.valA;
    uint64_t* kout = w.keyB;
    uint32_t* vout = w.valB;
    for (int sh = 0; sh < nbits; sh += 8) {
      hipLaunchKernelGGL(k_rs_hist, dim3((unsigned)nb), dim3(kSortThreads), 0,
                         stream, kin, m, sh, w.hist, nb, w.state);
      hipLaunchKernelGGL(k_scan_excl, dim3(1), dim3(1024), 0, stream, w.hist,
                         (int64_t)kRadix * nb, (const uint32_t*)w.state);
      hipLaunchKernelGGL(k_rs_scatter, dim3((unsigned)nb),
                         dim3(kSortThreads), 0, stream, kin, vin, kout, vout,
                         m, sh, w.hist, nb, w.state);
      uint64_t* tk = kin;
      kin = kout;
      kout = tk;
      uint32_t* tv = vin;
      vin = vout;
      vout = tv;
    }
    hipLaunchKernelGGL(k_grp_reduce, dim3((unsigned)nb), dim3(kSortThreads),
                       0, stream, kin, m, w.blkmax, w.blkcnt, w.state);
    hipLaunchKernelGGL(k_grp_carry, dim3(1), dim3(1024), 0, stream, w.blkmax,
                       w.blkcnt, w.carry, nb, m, w.state);
    hipLaunchKernelGGL(k_grp_rank, dim3((unsigned)nb), dim3(kSortThreads), 0,
                       stream, kin, vin, m, w.carry, w.rank, w.sa, w.state);
    hipLaunchKernelGGL(k_sa_commit, dim3(1), dim3(64), 0, stream, w.state);
    int rc = (int)hipGetLastError();
    if (rc) return rc;
  }
  if (sa_is64)
    hipLaunchKernelGGL(k_sa_out<int64_t>, dim3(out_blocks), dim3(256), 0,
                       stream, (const uint32_t*)w.sa, m, n_total,
                       (int64_t*)sa_out);
  else
    hipLaunchKernelGGL(k_sa_out<int32_t>, dim3(out_blocks), dim3(256), 0,
                       stream, (const uint32_t*)w.sa, m, n_total,
                       (int32_t*)sa_out);
  return (int)hipGetLastError();
}
