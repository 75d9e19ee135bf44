// Suffix-array construction on the GPU: prefix doubling over LSD radix
// sorts of the still-unsorted suffixes only, with no host synchronisation.
//
// Round 0 sorts all positions by their first two tokens when the text's
// tokens span fewer than 2^18 values (every LLM vocabulary; found on the
// device, so the doubling then starts at h = 2), else by their first token
// (signed order) -- 4 passes of 9 bits either way.  Every later round
// h = h0, 2 h0, 4 h0, ... re-sorts only the suffixes whose group still has
// more than one member, by the key
// (group head, rank[i+h]+1 or 0) -- a proper prefix sorts first, as in
// suffix_gpu/suffix_array.py:15-63 -- and writes them back into the SA
// positions their groups occupy, in order.  rank[i] is the SA position of
// the first suffix of i's group (for a finished suffix, its final
// position).  When no group of two or more is left the device sets a done
// flag and every later launch returns at its first instruction, so the
// fixed launch sequence (capturable, no host reads) is safe for any input.
//
// Each LSD pass is histogram (per 4096-element tile) -> per-digit row scan
// across tiles -> stable scatter.  The scatter ranks equal digits inside a
// wave with eight ballots (wave64 match) and across waves by per-wave digit
// counts, so tile order and element order are kept.

#include "launch.h"
#include "sfx_common.h"

namespace sfx {

constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kTile = kSortThreads * kSortItems;  // 4096
constexpr int kDigitBits = 9;
constexpr int kRadix = 1 << kDigitBits;                 // 512
constexpr int kDigitsPerThread = kRadix / kSortThreads;  // 2
constexpr int kSortWaves = kSortThreads / kWave;  // 4
constexpr int kWaveSpan = kTile / kSortWaves;     // 1024 per wave

struct SaWs {
  uint64_t* keyA;
  uint64_t* keyB;
  uint32_t* valA;
  uint32_t* valB;
  uint32_t* pos;     // SA positions of the active suffixes, ascending
  uint32_t* rank;    // [m] group head of text position i
  uint32_t* sa;      // [m] current suffix order
  uint32_t* grp;     // [m] group head of SA position j
  uint32_t* hist;    // [256][NB] digit counts per tile, then offsets
  uint32_t* rowsum;  // [256] digit totals
  uint32_t* tcnt;    // [NB] active suffixes per tile
  uint32_t* blkmax;  // [NB] last group start per tile
  uint32_t* state;   // [0] done, [1] active count, [2] round that found
                     // none left, [3] / [4] least / largest token other
                     // than PAD (INT32_MAX), [5] h of round 1
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
  s.pos = (uint32_t*)take(N * 4);
  s.rank = (uint32_t*)take(N * 4);
  s.sa = (uint32_t*)take(N * 4);
  s.grp = (uint32_t*)take(N * 4);
  s.hist = (uint32_t*)take((size_t)kRadix * NB * 4);
  s.rowsum = (uint32_t*)take(kRadix * 4);
  s.tcnt = (uint32_t*)take(NB * 4);
  s.blkmax = (uint32_t*)take(NB * 4);
  s.state = (uint32_t*)take(256);
  if (w) *w = s;
  return off;
}

__device__ __forceinline__ int64_t tiles_of(int64_t a) {
  return (a + kTile - 1) / kTile;
}

// Block-wide exclusive scan of one u32 per thread (NT threads); `red`
// holds NT/64 u32 in LDS.  Returns the prefix; *total gets the sum.
template <int NT>
__device__ __forceinline__ uint32_t block_exscan1(uint32_t v, uint32_t* red,
                                                  uint32_t* total) {
  constexpr int NW = NT / kWave;
  const int wv = threadIdx.x / kWave;
  const uint32_t inc = wave_incl_scan(v);
  if (lane_id() == kWave - 1) red[wv] = inc;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const uint32_t t = red[w];
    if (w < wv) before += t;
    all += t;
  }
  __syncthreads();
  *total = all;
  return before + inc - v;
}

// Block-wide least and largest of one int32 per thread (all threads).
__device__ __forceinline__ void block_minmax(int32_t& lo, int32_t& hi,
                                             int32_t (*red)[256 / kWave]) {
  lo = ~wave_max_i32(~lo);  // ~ reverses the signed order, no overflow
  hi = wave_max_i32(hi);
  const int wv = threadIdx.x / kWave;
  if (lane_id() == 0) {
    red[0][wv] = lo;
    red[1][wv] = hi;
  }
  __syncthreads();
  for (int w = 0; w < 256 / kWave; ++w) {
    lo = red[0][w] < lo ? red[0][w] : lo;
    hi = red[1][w] > hi ? red[1][w] : hi;
  }
}

// Least and largest token of the text, PAD (INT32_MAX) left out, per
// block (part_lo / part_hi, gridDim.x <= 256 entries each).
__global__ __launch_bounds__(256) void k_sa_range(const int32_t* text,
                                                  int64_t n,
                                                  int32_t* part_lo,
                                                  int32_t* part_hi) {
  __shared__ int32_t red[2][256 / kWave];
  int32_t lo = INT32_MAX, hi = INT32_MIN;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t t = text[i];
    if (t != INT32_MAX) {
      lo = t < lo ? t : lo;
      hi = t > hi ? t : hi;
    }
  }
  block_minmax(lo, hi, red);
  if (threadIdx.x == 0) {
    part_lo[blockIdx.x] = lo;
    part_hi[blockIdx.x] = hi;
  }
}

// Tokens of the pair keys: 1 + t - least, PAD after every other token, 0
// past the end; pair keys need span + 2 < 2^kPairBits.
constexpr int kPairBits = 18;

__global__ __launch_bounds__(256) void k_sa_init(const int32_t* text,
                                                 int64_t n, uint64_t* key,
                                                 uint32_t* val, uint32_t* pos,
                                                 const int32_t* part_lo,
                                                 const int32_t* part_hi,
                                                 int nparts,
                                                 uint32_t* state) {
  __shared__ int32_t red[2][256 / kWave];
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int32_t tlo = (int)threadIdx.x < nparts ? part_lo[threadIdx.x] : INT32_MAX;
  int32_t thi = (int)threadIdx.x < nparts ? part_hi[threadIdx.x] : INT32_MIN;
  block_minmax(tlo, thi, red);
  // thi < tlo: the text is all PAD
  const int64_t span = thi < tlo ? 0 : (int64_t)thi - (int64_t)tlo + 1;
  const bool pairs = span + 2 < ((int64_t)1 << kPairBits);
  if (i == 0) {
    state[0] = 0;
    state[1] = (uint32_t)n;
    state[3] = (uint32_t)tlo;
    state[4] = (uint32_t)thi;
    state[5] = pairs ? 2u : 1u;
  }
  if (i >= n) return;
  if (pairs) {
    auto code = [&](int64_t j) -> uint64_t {
      if (j >= n) return 0;
      const int32_t t = text[j];
      return t == INT32_MAX ? (uint64_t)span + 1
                            : (uint64_t)((int64_t)t - tlo + 1);
    };
    key[i] = (code(i) << kPairBits) | code(i + 1);
  } else {
    key[i] = (uint64_t)((uint32_t)text[i] ^ 0x80000000u);
  }
  val[i] = (uint32_t)i;
  pos[i] = (uint32_t)i;
}

// Lanes of the wave holding the same digit as the calling lane.
__device__ __forceinline__ uint64_t match_digit(bool act, uint32_t d) {
  uint64_t peers = ballot(act);
#pragma unroll
  for (int bit = 0; bit < kDigitBits; ++bit) {
    const bool set = (d >> bit) & 1u;
    const uint64_t m = ballot(act && set);
    peers &= set ? m : ~m;
  }
  return peers;
}

__device__ __forceinline__ uint32_t digit_of(uint64_t k, int sh) {
  return (uint32_t)(k >> sh) & (kRadix - 1u);
}

// Block-wide exclusive scan of the kRadix digit counts held
// kDigitsPerThread per thread (digits tid * kDigitsPerThread + j).
__device__ __forceinline__ void digit_exscan(const uint32_t (&c)[kDigitsPerThread],
                                             uint32_t (&ex)[kDigitsPerThread],
                                             uint32_t* red) {
  uint32_t sum = 0;
#pragma unroll
  for (int j = 0; j < kDigitsPerThread; ++j) sum += c[j];
  uint32_t tot;
  uint32_t run = block_exscan1<kSortThreads>(sum, red, &tot);
#pragma unroll
  for (int j = 0; j < kDigitsPerThread; ++j) {
    ex[j] = run;
    run += c[j];
  }
}

// ---------------------------------------------------------------- radix

__global__ __launch_bounds__(kSortThreads) void k_rs_hist(
    const uint64_t* __restrict__ key, int sh, uint32_t* hist, int64_t nb,
    const uint32_t* state) {
  if (state[0]) return;
  const int64_t A = state[1];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  // One histogram per wave (LDS atomics of a wave only collide on equal
  // digits), summed at the end.
  __shared__ uint32_t h[kSortWaves][kRadix];
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
#pragma unroll
  for (int w = 0; w < kSortWaves; ++w)
#pragma unroll
    for (int j = 0; j < kDigitsPerThread; ++j)
      h[w][tid * kDigitsPerThread + j] = 0;
  uint32_t d[kSortItems];
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t idx = base + (int64_t)r * kSortThreads + tid;
    d[r] = idx < A ? digit_of(key[idx], sh) : kRadix;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kSortItems; ++r)
    if (d[r] < kRadix) atomicAdd(&h[wv][d[r]], 1u);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kDigitsPerThread; ++j) {
    const int dg = tid * kDigitsPerThread + j;
    uint32_t sum = 0;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) sum += h[w][dg];
    hist[(int64_t)dg * nb + blockIdx.x] = sum;
  }
}

// Row d of the histogram (tiles 0 .. ceil(A/4096)) becomes its exclusive
// prefix; rowsum[d] the digit total.  One block per digit.
__global__ __launch_bounds__(kSortThreads) void k_rs_rowscan(
    uint32_t* hist, int64_t nb, uint32_t* rowsum, const uint32_t* state) {
  if (state[0]) return;
  __shared__ uint32_t red[kSortWaves];
  const int64_t nbA = tiles_of(state[1]);
  uint32_t* row = hist + (int64_t)blockIdx.x * nb;
  uint32_t carry = 0;
  for (int64_t c0 = 0; c0 < nbA; c0 += kSortThreads) {
    const int64_t t = c0 + threadIdx.x;
    const uint32_t v = t < nbA ? row[t] : 0u;
    uint32_t tot;
    const uint32_t ex = block_exscan1<kSortThreads>(v, red, &tot);
    if (t < nbA) row[t] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) rowsum[blockIdx.x] = carry;
}

// Stable scatter of one tile.  Wave w owns the tile's elements
// base + w*1024 + s*64 + lane (s < 16), i.e. a contiguous quarter, so the
// element order is (wave, step, lane).  The waves first count their digits
// (LDS atomics), one scan gives every (wave, digit) its output offset, and
// then each wave places its elements step by step with an eight-ballot
// digit match, advancing only its own offsets: three barriers per tile.
__global__ __launch_bounds__(kSortThreads) void k_rs_scatter(
    const uint64_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint64_t* __restrict__ kout, uint32_t* __restrict__ vout, int sh,
    const uint32_t* __restrict__ hist, int64_t nb,
    const uint32_t* __restrict__ rowsum, const uint32_t* state) {
  if (state[0]) return;
  const int64_t A = state[1];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  __shared__ uint32_t woff[kSortWaves][kRadix];
  __shared__ uint32_t red[kSortWaves];
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int ln = lane_id();
  constexpr int kSteps = kWaveSpan / kWave;  // 16
  const int64_t wbase = base + (int64_t)wv * kWaveSpan;
  uint64_t k[kSteps];
  uint32_t v[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t idx = wbase + s * kWave + ln;
    k[s] = idx < A ? kin[idx] : 0;
    v[s] = idx < A ? vin[idx] : 0;
  }
#pragma unroll
  for (int w = 0; w < kSortWaves; ++w)
#pragma unroll
    for (int j = 0; j < kDigitsPerThread; ++j)
      woff[w][tid * kDigitsPerThread + j] = 0;
  uint32_t rs[kDigitsPerThread], dbase[kDigitsPerThread];
#pragma unroll
  for (int j = 0; j < kDigitsPerThread; ++j)
    rs[j] = rowsum[tid * kDigitsPerThread + j];
  digit_exscan(rs, dbase, red);  // ends with a barrier: counters zeroed
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    if (wbase + s * kWave + ln < A)
      atomicAdd(&woff[wv][digit_of(k[s], sh)], 1u);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kDigitsPerThread; ++j) {
    const int dg = tid * kDigitsPerThread + j;
    uint32_t run = dbase[j] + hist[(int64_t)dg * nb + blockIdx.x];
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) {
      const uint32_t c = woff[w][dg];
      woff[w][dg] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const bool act = wbase + s * kWave + ln < A;
    const uint32_t d = digit_of(k[s], sh);
    const uint64_t peers = match_digit(act, d);
    const int rk = rank_lt(peers);
    if (act) {
      const uint32_t p = woff[wv][d] + (uint32_t)rk;
      kout[p] = k[s];
      vout[p] = v[s];
    }
    wave_lds_sync();  // every lane has read its offset
    if (act && rk == 0) woff[wv][d] += (uint32_t)popc(peers);
    wave_lds_sync();
  }
}

// ----------------------------------------------------------- group heads
// Over the sorted active list: slot t starts a group when its key differs
// from slot t-1's; the group's head is pos[start] (pos ascends with t, so
// the head of slot t is the largest start position at or before t).  Wave
// w of a tile owns slots base + w*1024 .. +1024, 64 consecutive per step.

__device__ __forceinline__ bool starts_group(const uint64_t* key, int64_t t,
                                             uint64_t kt) {
  return t == 0 || key[t - 1] != kt;
}

__global__ __launch_bounds__(kSortThreads) void k_grp_reduce(
    const uint64_t* __restrict__ key, const uint32_t* __restrict__ pos,
    uint32_t* blkmax, const uint32_t* state) {
  if (state[0]) return;
  const int64_t A = state[1];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  __shared__ uint32_t smax[kSortWaves];
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  const int64_t wbase = base + (int64_t)wv * kWaveSpan;
  uint32_t mx = 0;
#pragma unroll 4
  for (int s = 0; s < kWaveSpan / kWave; ++s) {
    const int64_t t = wbase + s * kWave + ln;
    if (t < A) {
      const uint64_t kt = key[t];
      if (starts_group(key, t, kt)) mx = max(mx, pos[t]);
    }
  }
  mx = (uint32_t)wave_max_i32((int)mx);
  if (ln == 0) smax[wv] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t m = 0;
    for (int w = 0; w < kSortWaves; ++w) m = max(m, smax[w]);
    blkmax[blockIdx.x] = m;
  }
}

// rank[val[t]] = head, sa[pos[t]] = val[t], grp[pos[t]] = head.
// The group start carried into a tile is the largest start of all earlier
// tiles: each block reduces blkmax[0 .. tile) itself.
__global__ __launch_bounds__(kSortThreads) void k_grp_rank(
    const uint64_t* __restrict__ key, const uint32_t* __restrict__ val,
    const uint32_t* __restrict__ pos, const uint32_t* __restrict__ blkmax,
    uint32_t* rank, uint32_t* sa, uint32_t* grp, const uint32_t* state) {
  if (state[0]) return;
  const int64_t A = state[1];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  __shared__ uint32_t smax[kSortWaves];
  __shared__ uint32_t cred[kSortWaves];
  uint32_t cm = 0;
  for (int t = threadIdx.x; t < (int)blockIdx.x; t += kSortThreads)
    cm = max(cm, blkmax[t]);
  cm = (uint32_t)wave_max_i32((int)cm);
  if (lane_id() == 0) cred[threadIdx.x / kWave] = cm;
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  const int64_t wbase = base + (int64_t)wv * kWaveSpan;
  constexpr int kSteps = kWaveSpan / kWave;  // 16
  uint32_t st[kSteps];  // start position of a group beginning here, or 0
  uint32_t mx = 0;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t t = wbase + s * kWave + ln;
    st[s] = 0;
    if (t < A) {
      const uint64_t kt = key[t];
      if (starts_group(key, t, kt)) st[s] = pos[t];
    }
    mx = max(mx, st[s]);
  }
  mx = (uint32_t)wave_max_i32((int)mx);
  if (ln == 0) smax[wv] = mx;
  __syncthreads();
  uint32_t run = 0;
  for (int w = 0; w < kSortWaves; ++w) run = max(run, cred[w]);
  for (int w = 0; w < wv; ++w) run = max(run, smax[w]);
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t t = wbase + s * kWave + ln;
    const uint32_t head = max(run, wave_incl_max(st[s]));
    run = max(run, (uint32_t)__builtin_amdgcn_readlane((int)head, kWave - 1));
    if (t < A) {
      const uint32_t i = val[t];
      const uint32_t j = pos[t];
      rank[i] = head;
      sa[j] = i;
      grp[j] = head;
    }
  }
}

// ------------------------------------------------------ active suffixes
// SA position j is finished when its group is the singleton {j}.
__device__ __forceinline__ bool unfinished(const uint32_t* grp, int64_t j,
                                           int64_t m) {
  const bool single =
      grp[j] == (uint32_t)j && (j + 1 == m || grp[j + 1] == (uint32_t)(j + 1));
  return !single;
}

__global__ __launch_bounds__(kSortThreads) void k_sa_mark(
    const uint32_t* __restrict__ grp, int64_t m, uint32_t* tcnt,
    const uint32_t* state) {
  if (state[0]) return;
  __shared__ uint32_t scnt[kSortWaves];
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  const int64_t wbase = (int64_t)blockIdx.x * kTile + (int64_t)wv * kWaveSpan;
  uint32_t cnt = 0;
#pragma unroll 4
  for (int s = 0; s < kWaveSpan / kWave; ++s) {
    const int64_t j = wbase + s * kWave + ln;
    cnt += (uint32_t)popc(ballot(j < m && unfinished(grp, j, m)));
  }
  if (ln == 0) scnt[wv] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t c = 0;
    for (int w = 0; w < kSortWaves; ++w) c += scnt[w];
    tcnt[blockIdx.x] = c;
  }
}

// Active suffixes of the tile, in SA order, with their sort keys:
// key = head * (m + 1) + (rank[i + h] + 1, or 0 past the end), where round
// r doubles h = state[5] << (r - 1).
// Each block sums the earlier tiles' counts for its output offset; block 0
// also sums them all: that is the round's active count, and none left
// means the array is final (the done flag).
__global__ __launch_bounds__(kSortThreads) void k_sa_gather(
    const uint32_t* __restrict__ sa, const uint32_t* __restrict__ rank,
    const uint32_t* __restrict__ grp, int64_t m, int round, int64_t nb,
    const uint32_t* __restrict__ tcnt, uint64_t* key, uint32_t* val,
    uint32_t* pos, uint32_t* state) {
  if (state[0]) return;
  const int64_t h = (int64_t)state[5] << (round - 1);
  __shared__ uint32_t scnt[kSortWaves];
  __shared__ uint32_t ored[kSortWaves];
  {
    const int64_t upto = blockIdx.x == 0 ? nb : (int64_t)blockIdx.x;
    uint32_t c = 0;
    for (int64_t t = threadIdx.x; t < upto; t += kSortThreads) c += tcnt[t];
    uint32_t tot;
    block_exscan1<kSortThreads>(c, ored, &tot);
    if (blockIdx.x == 0) {
      if (threadIdx.x == 0) {
        state[1] = tot;
        if (tot == 0) {
          state[0] = 1;
          state[2] = (uint32_t)round;  // the round that found none
        }
      }
      if (tot == 0) return;
      ored[0] = 0;  // block 0's own offset (the barrier below publishes it)
    } else if (threadIdx.x == 0) {
      ored[0] = tot;
    }
  }
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  const int64_t wbase = (int64_t)blockIdx.x * kTile + (int64_t)wv * kWaveSpan;
  constexpr int kSteps = kWaveSpan / kWave;
  uint32_t flags = 0;
  uint32_t cnt = 0;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t j = wbase + s * kWave + ln;
    const bool a = j < m && unfinished(grp, j, m);
    flags |= (uint32_t)a << s;
    cnt += (uint32_t)popc(ballot(a));
  }
  if (ln == 0) scnt[wv] = cnt;
  __syncthreads();
  uint32_t out = ored[0];
  for (int w = 0; w < wv; ++w) out += scnt[w];
  const uint64_t M1 = (uint64_t)m + 1;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t j = wbase + s * kWave + ln;
    const bool a = (flags >> s) & 1u;
    const uint64_t bm = ballot(a);
    if (a) {
      const uint32_t o = out + (uint32_t)rank_lt(bm);
      const uint32_t i = sa[j];
      const uint64_t k2 =
          (int64_t)i + h < m ? (uint64_t)rank[i + h] + 1 : 0;
      key[o] = (uint64_t)grp[j] * M1 + k2;
      val[o] = i;
      pos[o] = (uint32_t)j;
    }
    out += (uint32_t)popc(bm);
  }
}

// ------------------------------------------------------------ outputs
// keys[r * W + j] = corpus[sa[r] + j] (-1 at or past n).
__global__ __launch_bounds__(256) void k_rank_keys(const int32_t* corpus,
                                                 const int32_t* sa, int64_t n,
                                                 int W, int32_t* keys) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n * W) return;
  const int64_t r = e / W;
  const int j = (int)(e - r * W);
  const int64_t p = (int64_t)sa[r] + j;
  keys[e] = p < n && p >= 0 ? corpus[p] : -1;
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

// LSD radix sort of the active (key, val) pairs by the low `nbits` bits,
// then the group heads of the sorted order.
static int sort_and_rank(SaWs& w, int64_t nb, int nbits, hipStream_t stream) {
  uint64_t* kin = w.keyA;
  uint32_t* vin = w.valA;
  uint64_t* kout = w.keyB;
  uint32_t* vout = w.valB;
  for (int sh = 0; sh < nbits; sh += kDigitBits) {
    hipLaunchKernelGGL(k_rs_hist, dim3((unsigned)nb), dim3(kSortThreads), 0,
                       stream, kin, sh, w.hist, nb, w.state);
    hipLaunchKernelGGL(k_rs_rowscan, dim3(kRadix), dim3(kSortThreads), 0,
                       stream, w.hist, nb, w.rowsum, w.state);
    hipLaunchKernelGGL(k_rs_scatter, dim3((unsigned)nb), dim3(kSortThreads),
                       0, stream, kin, vin, kout, vout, sh, w.hist, nb,
                       w.rowsum, w.state);
    uint64_t* tk = kin;
    kin = kout;
    kout = tk;
    uint32_t* tv = vin;
    vin = vout;
    vout = tv;
  }
  hipLaunchKernelGGL(k_grp_reduce, dim3((unsigned)nb), dim3(kSortThreads), 0,
                     stream, kin, w.pos, w.blkmax, w.state);
  hipLaunchKernelGGL(k_grp_rank, dim3((unsigned)nb), dim3(kSortThreads), 0,
                     stream, kin, vin, w.pos, w.blkmax, w.rank, w.sa, w.grp,
                     w.state);
  return (int)hipGetLastError();
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

namespace {

int launch_out(const uint32_t* sa, int64_t m, int64_t n_total, void* sa_out,
               int32_t sa_is64, hipStream_t stream) {
  const unsigned out_blocks = (unsigned)((n_total + 255) / 256);
  if (sa_is64)
    hipLaunchKernelGGL(k_sa_out<int64_t>, dim3(out_blocks), dim3(256), 0,
                       stream, sa, m, n_total, (int64_t*)sa_out);
  else
    hipLaunchKernelGGL(k_sa_out<int32_t>, dim3(out_blocks), dim3(256), 0,
                       stream, sa, m, n_total, (int32_t*)sa_out);
  return (int)hipGetLastError();
}

bool ws_ok(int64_t m, const void* workspace, size_t bytes) {
  return m <= 1 || (workspace && bytes >= sa_ws_layout(m, nullptr, nullptr));
}

// Doubling rounds after the token round: one per h = 1, 2, 4, ... < m.
int total_rounds(int64_t m) {
  int r = 0;
  for (int64_t h = 1; h < m; h <<= 1) ++r;
  return r;
}

int build_begin(const int32_t* text, int64_t m, void* workspace,
                hipStream_t stream) {
  if (m <= 1) return 0;
  SaWs w;
  sa_ws_layout(m, workspace, &w);
  const int64_t nb = (m + kTile - 1) / kTile;
  const unsigned eb = (unsigned)((m + 255) / 256);
  // per-block token ranges in the per-tile arrays, unused until round 1
  const int parts = (int)(nb < 256 ? nb : 256);
  int32_t* plo = reinterpret_cast<int32_t*>(w.tcnt);
  int32_t* phi = reinterpret_cast<int32_t*>(w.blkmax);
  hipLaunchKernelGGL(k_sa_range, dim3((unsigned)parts), dim3(256), 0, stream,
                     text, m, plo, phi);
  hipLaunchKernelGGL(k_sa_init, dim3(eb), dim3(256), 0, stream, text, m,
                     w.keyA, w.valA, w.pos, plo, phi, parts, w.state);
  return sort_and_rank(w, nb, 2 * kPairBits, stream);
}

// Rounds first .. first + count - 1 (round r doubles h = h0 * 2^(r-1),
// h0 = 1 or 2 as round 0 decided; with h0 = 2 the last round finds none).
int build_rounds(int64_t m, int first, int count, void* workspace,
                 hipStream_t stream) {
  if (m <= 1) return 0;
  SaWs w;
  sa_ws_layout(m, workspace, &w);
  const int64_t nb = (m + kTile - 1) / kTile;
  const uint64_t maxkey = (uint64_t)(m - 1) * (uint64_t)(m + 1) + (uint64_t)m;
  const int nbits = bits_for(maxkey);
  const int last = total_rounds(m);
  for (int r = first < 1 ? 1 : first; r < first + count && r <= last; ++r) {
    hipLaunchKernelGGL(k_sa_mark, dim3((unsigned)nb), dim3(kSortThreads), 0,
                       stream, w.grp, m, w.tcnt, w.state);
    hipLaunchKernelGGL(k_sa_gather, dim3((unsigned)nb), dim3(kSortThreads), 0,
                       stream, w.sa, w.rank, w.grp, m, r, nb, w.tcnt, w.keyA,
                       w.valA, w.pos, w.state);
    const int rc = sort_and_rank(w, nb, nbits, stream);
    if (rc) return rc;
  }
  return (int)hipGetLastError();
}

int build_finish(int64_t m, int64_t n_total, void* sa_out, int32_t sa_is64,
                 void* workspace, hipStream_t stream) {
  if (m <= 1) return launch_out(nullptr, 0, n_total, sa_out, sa_is64, stream);
  SaWs w;
  sa_ws_layout(m, workspace, &w);
  return launch_out(w.sa, m, n_total, sa_out, sa_is64, stream);
}

}  // namespace

extern "C" int sfx_sa_build(const int32_t* text, int64_t m, int64_t n_total,
                            void* sa_out, int32_t sa_is64, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
  if (m < 0 || n_total < m || m > 0x7fffffffLL || n_total > 0x7fffffffLL)
    return SFX_EINVAL;
  if (n_total == 0) return 0;
  if (!sa_out || (m > 0 && !text)) return SFX_EINVAL;
  if (!ws_ok(m, workspace, workspace_bytes)) return SFX_EINVAL;
  int rc = build_begin(text, m, workspace, stream);
  if (rc) return rc;
  rc = build_rounds(m, 1, total_rounds(m), workspace, stream);
  if (rc) return rc;
  return build_finish(m, n_total, sa_out, sa_is64, workspace, stream);
}

extern "C" int sfx_sa_build_rounds_total(int64_t m) {
  return m < 0 ? SFX_EINVAL : total_rounds(m);
}

extern "C" int64_t sfx_sa_build_flag_offset(int64_t m) {
  if (m < 0) return SFX_EINVAL;
  // Lay the workspace out over a stand-in base address to read the state
  // block's offset; nothing is dereferenced.
  char* const base = reinterpret_cast<char*>(uintptr_t{1} << 20);
  SaWs w;
  sa_ws_layout(m, base, &w);
  return (int64_t)(reinterpret_cast<char*>(w.state) - base);
}

extern "C" int sfx_sa_build_begin(const int32_t* text, int64_t m,
                                  void* workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  if (m < 0 || m > 0x7fffffffLL || (m > 0 && !text)) return SFX_EINVAL;
  if (!ws_ok(m, workspace, workspace_bytes)) return SFX_EINVAL;
  return build_begin(text, m, workspace, stream);
}

extern "C" int sfx_sa_build_rounds(int64_t m, int32_t first, int32_t count,
                                   void* workspace, size_t workspace_bytes,
                                   hipStream_t stream) {
  if (m < 0 || m > 0x7fffffffLL || first < 1 || count < 0) return SFX_EINVAL;
  if (!ws_ok(m, workspace, workspace_bytes)) return SFX_EINVAL;
  return build_rounds(m, first, count, workspace, stream);
}

extern "C" int sfx_sa_build_finish(int64_t m, int64_t n_total, void* sa_out,
                                   int32_t sa_is64, void* workspace,
                                   size_t workspace_bytes,
                                   hipStream_t stream) {
  if (m < 0 || n_total < m || m > 0x7fffffffLL || n_total > 0x7fffffffLL)
    return SFX_EINVAL;
  if (n_total == 0) return 0;
  if (!sa_out) return SFX_EINVAL;
  if (!ws_ok(m, workspace, workspace_bytes)) return SFX_EINVAL;
  return build_finish(m, n_total, sa_out, sa_is64, workspace, stream);
}
