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
// A round works on its active list: the still-unsorted suffixes in SA
// order, (key, suffix, SA position) per entry.  The round's last kernel
// marks every entry whose new group is a singleton and counts the others
// per tile; the next round's gather compacts the rest of the list into the
// next list, so no round rescans the m SA positions.
//
// Each LSD pass is histogram (per 4096-element tile) -> per-digit row scan
// across tiles -> stable scatter.  The scatter ranks equal digits inside a
// wave with nine ballots (wave64 match) and across waves by per-wave digit
// counts, so tile order and element order are kept.

#include "launch.h"
#include "sfx_common.h"

namespace sfx {

constexpr int kTile = 4096;  // list entries per tile (one block per tile)
constexpr int kDigitBits = 9;
constexpr int kRadix = 1 << kDigitBits;                 // 512
constexpr uint32_t kFinished = 0xffffffffu;  // hd[] of a singleton entry
// state[] words: [0] done, [1] / [6] list length of even / odd rounds,
// [2] round that found none left, [3] / [4] least / largest token other
// than PAD (INT32_MAX), [5] h of round 1.
constexpr int kDone = 0, kLenEven = 1, kFoundNone = 2, kTokLo = 3,
              kTokHi = 4, kH0 = 5, kLenOdd = 6;
__host__ __device__ constexpr int len_slot(int round) {
  return (round & 1) ? kLenOdd : kLenEven;
}

struct SaWs {
  uint64_t* keyA;
  uint64_t* keyB;
  uint32_t* valA;
  uint32_t* valB;
  uint32_t* pos[2];  // SA positions of the list entries (ascending) of
                     // even / odd rounds
  uint32_t* rank;    // [m] group head of text position i
  uint32_t* sa;      // [m] current suffix order
  uint32_t* hd;      // [list] group head of a sorted entry, kFinished for a
                     // singleton
  uint32_t* hist;    // [512][NB] digit counts per tile, then offsets
  uint32_t* rowsum;  // [512] digit totals
  uint32_t* tcnt;    // [NB] unfinished entries per tile of the sorted list
  uint32_t* blkmax;  // [NB] last group start per tile
  uint32_t* state;   // the state[] words above
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
  s.pos[0] = (uint32_t*)take(N * 4);
  s.pos[1] = (uint32_t*)take(N * 4);
  s.rank = (uint32_t*)take(N * 4);
  s.sa = (uint32_t*)take(N * 4);
  s.hd = (uint32_t*)take(N * 4);
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
  constexpr int kUnroll = 8;
  int32_t lo = INT32_MAX, hi = INT32_MIN;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < n;
       i0 += kUnroll * stride) {
    int32_t t[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i0 + u * stride;
      t[u] = i < n ? text[i] : INT32_MAX;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (t[u] != INT32_MAX) {
        lo = t[u] < lo ? t[u] : lo;
        hi = t[u] > hi ? t[u] : hi;
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
    state[kDone] = 0;
    state[len_slot(0)] = (uint32_t)n;
    state[kTokLo] = (uint32_t)tlo;
    state[kTokHi] = (uint32_t)thi;
    state[kH0] = pairs ? 2u : 1u;
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

// ---------------------------------------------------------------- radix
// The passes run NT threads per 4096-element tile.  With about one active
// tile per CU, 1024 threads (16 waves) keep four times more loads and LDS
// operations in flight per CU than 256 threads would.

constexpr int kRsThreads = 1024;
constexpr int kRsHists = 4;  // LDS sub-histograms of the histogram pass

template <int NT>
__global__ __launch_bounds__(NT) void k_rs_hist(
    const uint64_t* __restrict__ key, int sh, uint32_t* hist, int64_t nb,
    const uint32_t* state, int slot) {
  static_assert(kTile % NT == 0 && NT >= kRadix, "tile shape");
  constexpr int kItems = kTile / NT;
  if (state[kDone]) return;
  const int64_t A = state[slot];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  // Waves w, w + kRsHists, ... share a histogram; the sub-histograms are
  // summed at the end.  A wave's lanes hold consecutive entries, and equal
  // keys sit next to each other in every pass (suffixes inside repeated
  // text share their key until h outgrows the repeat), so each run of
  // equal digits adds its length with one atomic from its first lane:
  // same-address LDS atomics within a wave would serialise.
  __shared__ uint32_t h[kRsHists][kRadix];
  const int tid = threadIdx.x;
  const int ln = lane_id();
  const int hw = (tid / kWave) % kRsHists;
  for (int e = tid; e < kRsHists * kRadix; e += NT) (&h[0][0])[e] = 0;
  uint32_t d[kItems];
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    const int64_t idx = base + (int64_t)r * NT + tid;
    d[r] = idx < A ? digit_of(key[idx], sh) : kRadix;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    const uint32_t prev = __shfl_up(d[r], 1);
    const bool start = ln == 0 || prev != d[r];
    const uint64_t starts = ballot(start);
    const uint64_t after = ln == kWave - 1 ? 0ull : starts >> (ln + 1);
    const uint32_t len =
        after ? (uint32_t)__builtin_ctzll(after) + 1u : (uint32_t)(kWave - ln);
    if (start && d[r] < kRadix) atomicAdd(&h[hw][d[r]], len);
  }
  __syncthreads();
  if (tid < kRadix) {
    uint32_t sum = 0;
#pragma unroll
    for (int w = 0; w < kRsHists; ++w) sum += h[w][tid];
    hist[(int64_t)tid * nb + blockIdx.x] = sum;
  }
}

// Row d of the histogram (tiles 0 .. ceil(A/4096)) becomes its exclusive
// prefix; rowsum[d] the digit total.  One block per digit.
template <int NT>
__global__ __launch_bounds__(NT) void k_rs_rowscan(
    uint32_t* hist, int64_t nb, uint32_t* rowsum, const uint32_t* state,
    int slot) {
  if (state[kDone]) return;
  __shared__ uint32_t red[NT / kWave];
  const int64_t nbA = tiles_of(state[slot]);
  uint32_t* row = hist + (int64_t)blockIdx.x * nb;
  uint32_t carry = 0;
  for (int64_t c0 = 0; c0 < nbA; c0 += NT) {
    const int64_t t = c0 + threadIdx.x;
    const uint32_t v = t < nbA ? row[t] : 0u;
    uint32_t tot;
    const uint32_t ex = block_exscan1<NT>(v, red, &tot);
    if (t < nbA) row[t] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) rowsum[blockIdx.x] = carry;
}

// Stable scatter of one tile.  Wave w owns the tile's contiguous span
// base + w * kTile / NW .. + kTile / NW, 64 consecutive elements per step,
// so the element order is (wave, step, lane).  The waves first count their
// digits (LDS atomics), one scan gives every (wave, digit) its output
// offset, and then each wave places its elements step by step with a
// nine-ballot digit match, advancing only its own offsets: three barriers
// per tile.
template <int NT>
__global__ __launch_bounds__(NT) void k_rs_scatter(
    const uint64_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint64_t* __restrict__ kout, uint32_t* __restrict__ vout, int sh,
    const uint32_t* __restrict__ hist, int64_t nb,
    const uint32_t* __restrict__ rowsum, const uint32_t* state, int slot) {
  constexpr int NW = NT / kWave;
  constexpr int kSpan = kTile / NW;
  constexpr int kSteps = kSpan / kWave;
  static_assert(kTile % NT == 0 && NT >= kRadix, "tile shape");
  if (state[kDone]) return;
  const int64_t A = state[slot];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  __shared__ uint32_t woff[NW][kRadix];
  __shared__ uint32_t red[NW];
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int ln = lane_id();
  const int64_t wbase = base + (int64_t)wv * kSpan;
  uint64_t k[kSteps];
  uint32_t v[kSteps];
  uint64_t peers[kSteps];  // lanes of the same step holding the same digit
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t idx = wbase + s * kWave + ln;
    k[s] = idx < A ? kin[idx] : 0;
    v[s] = idx < A ? vin[idx] : 0;
  }
  for (int e = tid; e < NW * kRadix; e += NT) (&woff[0][0])[e] = 0;
  // Digit d's first output slot: the totals of the digits below it.
  uint32_t tot;
  const uint32_t dbase =
      block_exscan1<NT>(tid < kRadix ? rowsum[tid] : 0u, red, &tot);
  // block_exscan1 ends with a barrier: the counters are zeroed.  Each
  // digit's count of a step is added once, by its lowest lane (equal
  // digits would otherwise serialise on one LDS address).
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const bool act = wbase + s * kWave + ln < A;
    const uint32_t d = digit_of(k[s], sh);
    peers[s] = match_digit(act, d);
    if (act && rank_lt(peers[s]) == 0)
      atomicAdd(&woff[wv][d], (uint32_t)popc(peers[s]));
  }
  __syncthreads();
  if (tid < kRadix) {
    uint32_t run = dbase + hist[(int64_t)tid * nb + blockIdx.x];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t c = woff[w][tid];
      woff[w][tid] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const bool act = wbase + s * kWave + ln < A;
    const uint32_t d = digit_of(k[s], sh);
    const int rk = rank_lt(peers[s]);
    if (act) {
      const uint32_t p = woff[wv][d] + (uint32_t)rk;
      kout[p] = k[s];
      vout[p] = v[s];
    }
    wave_lds_sync();  // every lane has read its offset
    if (act && rk == 0) woff[wv][d] += (uint32_t)popc(peers[s]);
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

template <int NT>
__global__ __launch_bounds__(NT) void k_grp_reduce(
    const uint64_t* __restrict__ key, const uint32_t* __restrict__ pos,
    uint32_t* blkmax, const uint32_t* state, int slot) {
  constexpr int NW = NT / kWave;
  constexpr int kSpan = kTile / NW;
  if (state[kDone]) return;
  const int64_t A = state[slot];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  __shared__ uint32_t smax[NW];
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  const int64_t wbase = base + (int64_t)wv * kSpan;
  uint32_t mx = 0;
#pragma unroll
  for (int s = 0; s < kSpan / kWave; ++s) {
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
    for (int w = 0; w < NW; ++w) m = max(m, smax[w]);
    blkmax[blockIdx.x] = m;
  }
}

// rank[val[t]] = head, sa[pos[t]] = val[t]; hd[t] = head, or kFinished
// when t's group is the singleton {t}; tcnt[tile] = the tile's entries
// that are not finished.  The group start carried into a tile is the
// largest start of all earlier tiles: each block reduces blkmax[0 .. tile)
// itself.
template <int NT>
__global__ __launch_bounds__(NT) void k_grp_rank(
    const uint64_t* __restrict__ key, const uint32_t* __restrict__ val,
    const uint32_t* __restrict__ pos, const uint32_t* __restrict__ blkmax,
    uint32_t* __restrict__ rank, uint32_t* __restrict__ sa,
    uint32_t* __restrict__ hd, uint32_t* __restrict__ tcnt,
    const uint32_t* state, int slot) {
  constexpr int NW = NT / kWave;
  constexpr int kSpan = kTile / NW;
  constexpr int kSteps = kSpan / kWave;
  if (state[kDone]) return;
  const int64_t A = state[slot];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  __shared__ uint32_t smax[NW];
  __shared__ uint32_t cred[NW];
  __shared__ uint32_t ucnt[NW];
  uint32_t cm = 0;
  for (int t = threadIdx.x; t < (int)blockIdx.x; t += NT)
    cm = max(cm, blkmax[t]);
  cm = (uint32_t)wave_max_i32((int)cm);
  if (lane_id() == 0) cred[threadIdx.x / kWave] = cm;
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  const int64_t wbase = base + (int64_t)wv * kSpan;
  uint32_t st[kSteps];  // start position of a group beginning here, or 0
  uint32_t single = 0;  // bit s: entry s is a group of its own
  uint32_t mx = 0;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t t = wbase + s * kWave + ln;
    st[s] = 0;
    if (t < A) {
      const uint64_t kt = key[t];
      const bool first = starts_group(key, t, kt);
      const bool last = t + 1 == A || key[t + 1] != kt;
      if (first) st[s] = pos[t];
      single |= (uint32_t)(first && last) << s;
    }
    mx = max(mx, st[s]);
  }
  mx = (uint32_t)wave_max_i32((int)mx);
  if (ln == 0) smax[wv] = mx;
  __syncthreads();
  uint32_t run = 0;
  for (int w = 0; w < NW; ++w) run = max(run, cred[w]);
  for (int w = 0; w < wv; ++w) run = max(run, smax[w]);
  uint32_t open = 0;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t t = wbase + s * kWave + ln;
    const uint32_t head = max(run, wave_incl_max(st[s]));
    run = max(run, (uint32_t)__builtin_amdgcn_readlane((int)head, kWave - 1));
    const bool fin = (single >> s) & 1u;
    open += (uint32_t)popc(ballot(t < A && !fin));
    if (t < A) {
      const uint32_t i = val[t];
      rank[i] = head;
      sa[pos[t]] = i;
      hd[t] = fin ? kFinished : head;
    }
  }
  if (ln == 0) ucnt[wv] = open;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t c = 0;
    for (int w = 0; w < NW; ++w) c += ucnt[w];
    tcnt[blockIdx.x] = c;
  }
}

// ------------------------------------------------------ active suffixes
// Round r's list: the unfinished entries of round r-1's sorted list (hd,
// vold, pold; length in state[cin]) in the same SA order, keyed
// head * (m + 1) + (rank[i + h] + 1, or 0 past the end), where round r
// doubles h = state[kH0] << (r - 1).  Each block sums the earlier tiles'
// counts for its output offset; block 0 also sums them all: that is the
// new length (state[cout]), and none left means the array is final (the
// done flag).
template <int NT>
__global__ __launch_bounds__(NT) void k_sa_gather(
    const uint32_t* __restrict__ hd, const uint32_t* __restrict__ vold,
    const uint32_t* __restrict__ pold, const uint32_t* __restrict__ rank,
    const uint32_t* __restrict__ tcnt, int64_t m, int round,
    uint64_t* __restrict__ key, uint32_t* __restrict__ val,
    uint32_t* __restrict__ pos, uint32_t* state, int cin, int cout) {
  constexpr int NW = NT / kWave;
  constexpr int kSpan = kTile / NW;
  constexpr int kSteps = kSpan / kWave;
  if (state[kDone]) return;
  const int64_t Aold = state[cin];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (blockIdx.x > 0 && base >= Aold) return;  // block 0 writes the length
  const int64_t h = (int64_t)state[kH0] << (round - 1);
  __shared__ uint32_t scnt[NW];
  __shared__ uint32_t ored[NW];
  {
    const int64_t upto = blockIdx.x == 0 ? tiles_of(Aold) : (int64_t)blockIdx.x;
    uint32_t c = 0;
    for (int64_t t = threadIdx.x; t < upto; t += NT) c += tcnt[t];
    uint32_t tot;
    block_exscan1<NT>(c, ored, &tot);
    if (blockIdx.x == 0) {
      if (threadIdx.x == 0) {
        state[cout] = tot;
        if (tot == 0) {
          state[kDone] = 1;
          state[kFoundNone] = (uint32_t)round;
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
  const int64_t wbase = base + (int64_t)wv * kSpan;
  uint32_t hv[kSteps];
  uint32_t cnt = 0;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t t = wbase + s * kWave + ln;
    hv[s] = t < Aold ? hd[t] : kFinished;
    cnt += (uint32_t)popc(ballot(hv[s] != kFinished));
  }
  if (ln == 0) scnt[wv] = cnt;
  __syncthreads();
  uint32_t out = ored[0];
  for (int w = 0; w < wv; ++w) out += scnt[w];
  const uint64_t M1 = (uint64_t)m + 1;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t t = wbase + s * kWave + ln;
    const bool a = hv[s] != kFinished;
    const uint64_t bm = ballot(a);
    if (a) {
      const uint32_t o = out + (uint32_t)rank_lt(bm);
      const uint32_t i = vold[t];
      const uint64_t k2 =
          (int64_t)i + h < m ? (uint64_t)rank[i + h] + 1 : 0;
      key[o] = (uint64_t)hv[s] * M1 + k2;
      val[o] = i;
      pos[o] = pold[t];
    }
    out += (uint32_t)popc(bm);
  }
}

// ------------------------------------------------------------ outputs
// keys[r * W + j] = corpus[sa[r] + j] (-1 at or past n), ranks r < rows.
__global__ __launch_bounds__(256) void k_rank_keys(const int32_t* corpus,
                                                 const int32_t* sa, int64_t n,
                                                 int64_t rows, int W,
                                                 int32_t* keys) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * W) return;
  const int64_t r = e / W;
  const int j = (int)(e - r * W);
  const int64_t p = (int64_t)sa[r] + j;
  keys[e] = p < n && p >= 0 ? corpus[p] : -1;
}

// The same rows four tokens per thread with one 16-byte store (keys
// 16-byte aligned, W % 4 == 0): a quarter of the threads and store
// instructions for the 128 B-per-rank write that bounds the kernel.
__global__ __launch_bounds__(256) void k_rank_keys4(const int32_t* corpus,
                                                  const int32_t* sa, int64_t n,
                                                  int64_t rows, int W,
                                                  int32_t* keys) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int W4 = W >> 2;
  if (e >= rows * W4) return;
  const int64_t r = e / W4;
  const int64_t p = (int64_t)sa[r] + 4 * (e - r * W4);
  int4 v;
  v.x = p < n && p >= 0 ? corpus[p] : -1;
  v.y = p + 1 < n && p + 1 >= 0 ? corpus[p + 1] : -1;
  v.z = p + 2 < n && p + 2 >= 0 ? corpus[p + 2] : -1;
  v.w = p + 3 < n && p + 3 >= 0 ? corpus[p + 3] : -1;
  reinterpret_cast<int4*>(keys)[e] = v;
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

static int passes_of(int nbits) {
  return (nbits + kDigitBits - 1) / kDigitBits;
}

// Key bits of a doubling round: head * (m + 1) + k2 with head < m, k2 <= m.
static int round_bits(int64_t m) {
  return bits_for((uint64_t)(m - 1) * (uint64_t)(m + 1) + (uint64_t)m);
}

// Key buffer (0: A, 1: B) holding round r's list before its sort: round 0
// starts in A, and each round's gather writes the buffer its predecessor's
// sorted list is not in.
static int list_buf(int64_t m, int round) {
  const int p0 = passes_of(2 * kPairBits);
  const int p = passes_of(round_bits(m));
  int x = 0;
  for (int q = 0; q < round; ++q) x = (x ^ ((q == 0 ? p0 : p) & 1)) ^ 1;
  return x;
}

// Buffer holding round r's sorted list.
static int sorted_buf(int64_t m, int round) {
  const int p = round == 0 ? passes_of(2 * kPairBits)
                           : passes_of(round_bits(m));
  return list_buf(m, round) ^ (p & 1);
}

// LSD radix sort of round r's list by the low `nbits` bits of its keys,
// then the group heads of the sorted order.
static int sort_and_rank(SaWs& w, int64_t nb, int64_t m, int round,
                         hipStream_t stream) {
  const int nbits = round == 0 ? 2 * kPairBits : round_bits(m);
  const int slot = len_slot(round);
  uint64_t* keys[2] = {w.keyA, w.keyB};
  uint32_t* vals[2] = {w.valA, w.valB};
  int x = list_buf(m, round);
  for (int sh = 0; sh < nbits; sh += kDigitBits) {
    hipLaunchKernelGGL(k_rs_hist<kRsThreads>, dim3((unsigned)nb),
                       dim3(kRsThreads), 0, stream, keys[x], sh, w.hist, nb,
                       w.state, slot);
    hipLaunchKernelGGL(k_rs_rowscan<kRsThreads>, dim3(kRadix),
                       dim3(kRsThreads), 0, stream, w.hist, nb, w.rowsum,
                       w.state, slot);
    hipLaunchKernelGGL(k_rs_scatter<kRsThreads>, dim3((unsigned)nb),
                       dim3(kRsThreads), 0, stream, keys[x], vals[x],
                       keys[x ^ 1], vals[x ^ 1], sh, w.hist, nb, w.rowsum,
                       w.state, slot);
    x ^= 1;
  }
  uint32_t* pos = w.pos[round & 1];
  hipLaunchKernelGGL(k_grp_reduce<kRsThreads>, dim3((unsigned)nb),
                     dim3(kRsThreads), 0, stream, keys[x], pos, w.blkmax,
                     w.state, slot);
  hipLaunchKernelGGL(k_grp_rank<kRsThreads>, dim3((unsigned)nb),
                     dim3(kRsThreads), 0, stream, keys[x], vals[x], pos,
                     w.blkmax, w.rank, w.sa, w.hd, w.tcnt, w.state, slot);
  return (int)hipGetLastError();
}

}  // namespace sfx

using namespace sfx;

extern "C" int sfx_sa_keys(const int32_t* corpus, const int32_t* sa,
                           int64_t n, int64_t rows, int64_t width,
                           int32_t* keys, hipStream_t stream) {
  if (n < 0 || rows < 0 || rows > n || n > 0x7fffffffLL || width < 4 ||
      width > 32 || (width & 3))
    return SFX_EINVAL;
  if (rows == 0) return 0;
  if (!corpus || !sa || !keys) return SFX_EINVAL;
  const int64_t total = rows * width;
  if ((((uintptr_t)keys) & 15) == 0) {
    const int64_t total4 = total / 4;
    hipLaunchKernelGGL(k_rank_keys4, dim3((unsigned)((total4 + 255) / 256)),
                       dim3(256), 0, stream, corpus, sa, n, rows, (int)width,
                       keys);
  } else {
    hipLaunchKernelGGL(k_rank_keys, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, stream, corpus, sa, n, rows, (int)width,
                       keys);
  }
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
                     w.keyA, w.valA, w.pos[0], plo, phi, parts, w.state);
  return sort_and_rank(w, nb, m, 0, stream);
}

// Rounds first .. first + count - 1 (round r doubles h = h0 * 2^(r-1),
// h0 = 1 or 2 as round 0 decided; with h0 = 2 the last round finds none).
int build_rounds(int64_t m, int first, int count, void* workspace,
                 hipStream_t stream) {
  if (m <= 1) return 0;
  SaWs w;
  sa_ws_layout(m, workspace, &w);
  const int64_t nb = (m + kTile - 1) / kTile;
  const int last = total_rounds(m);
  uint64_t* keys[2] = {w.keyA, w.keyB};
  uint32_t* vals[2] = {w.valA, w.valB};
  for (int r = first < 1 ? 1 : first; r < first + count && r <= last; ++r) {
    const int src = sorted_buf(m, r - 1);
    const int dst = list_buf(m, r);
    hipLaunchKernelGGL(k_sa_gather<kRsThreads>, dim3((unsigned)nb),
                       dim3(kRsThreads), 0, stream, w.hd, vals[src],
                       w.pos[(r - 1) & 1], w.rank, w.tcnt, m, r, keys[dst],
                       vals[dst], w.pos[r & 1], w.state, len_slot(r - 1),
                       len_slot(r));
    const int rc = sort_and_rank(w, nb, m, r, stream);
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
