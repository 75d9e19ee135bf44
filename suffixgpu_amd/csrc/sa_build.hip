// Suffix-array construction on the GPU: prefix doubling with no host
// synchronisation, as suffix_gpu/suffix_array.py:15-63 specifies it (a
// proper prefix sorts first), on state kept per SA position.
//
// Round 0 sorts all positions by their first two tokens when the text's
// tokens span fewer than 2^18 values (every LLM vocabulary; found on the
// device, so the doubling then starts at h = 2), else by their first token
// (signed order) -- 4 LSD radix passes of 9 bits either way.  Round
// r = 1, 2, ... doubles h = h0 << (r - 1): every group of two or more
// suffixes that agree on their first h tokens (a run of SA positions) is
// re-sorted by rank[i + h] + 1 (0 past the end), where rank[i] is the SA
// position of the first suffix of i's group (for a finished suffix, its
// final position).  Per SA position p the state holds sa[p], gp[p] (the
// head position of p's group, or a finished mark) and, at a head, gsz[]
// (the group's size); rank[] has two buffers, read and written by
// alternate rounds, so that no round reads a rank the same round changes.
//
// A round sorts each group by one of two means, chosen per group on the
// device from its size:
//  * groups of at most kCap suffixes: one launch for the round.  A
//    workgroup owns the groups whose head lies in its 4096-position tile
//    (a group that started in the tile before is skipped, skip[] holding
//    its length; one that runs on into the next tile is followed), sorts
//    each of them by its keys in LDS (a 64-lane bitonic sort per
//    64-position window, then a binary search in every other window of the
//    group) and writes the new order, heads and sizes back;
//  * groups above kCap (the radix part): their positions are compacted
//    into a list keyed (head, rank[i + h] + 1) in SA order, LSD radix
//    sorted, and the group heads of the sorted list are written back.
// A round with a group above kCap whose radix launches the caller did not
// enqueue only marks itself stalled: every later launch returns at once,
// and a caller that enqueues the round again with the radix part resumes
// it.  When no group of two or more is left the device sets a done flag
// and every later launch returns at its first instruction, so a fixed
// launch sequence (capturable, no host reads) is safe for any input.
//
// Each LSD pass is histogram (per 4096-element tile) -> per-digit row scan
// across tiles -> stable scatter.  The scatter ranks equal digits inside a
// wave with nine ballots (wave64 match) and across waves by per-wave digit
// counts, so tile order and element order are kept.

#include "launch.h"
#include "sfx_common.h"

namespace sfx {

constexpr int kTile = 4096;     // list entries / SA positions per radix tile
constexpr int kPosTile = 4096;  // SA positions per local-round tile
constexpr int kCap = 2048;      // largest group the local part sorts
constexpr int kSlots = kPosTile + kCap;  // positions a local workgroup reads
// One 1024-thread workgroup per CU measured faster than 2 x 512 threads or
// 2048-position tiles: fewer windows per wave, and one barrier pair per
// 4096 positions.
constexpr int kSaLocalThreads = 1024;
constexpr int kDigitBits = 9;
constexpr int kRadix = 1 << kDigitBits;                 // 512
constexpr uint32_t kFinished = 0xffffffffu;  // gp[] of a finished position
// gp[] of a position finished by the previous round: its final rank is in
// that round's rank buffer only, and the next round copies it to the other
constexpr uint32_t kJustFinished = 0xfffffffeu;
// state[] words: [0] done, [1] global list length, [2] round that found no
// group left, [3] / [4] least / largest token other than PAD (INT32_MAX),
// [5] h of round 1, [7] round that stalled (0: none), [8] bit r set when
// round r took the global path, [16 + r] largest group entering round r,
// [64 + r] h of round r (the prefix length its groups share).
constexpr int kDone = 0, kLen = 1, kFoundNone = 2, kTokLo = 3, kTokHi = 4,
              kH0 = 5, kStalled = 7, kGlobalMask = 8, kMaxGrp = 16,
              kHRound = 64;
constexpr int kStateWords = 128;
// Group sizes above this are recorded per local tile (tmax) to order the
// next round's tiles; kOrderClasses size classes (see k_sa_order).
constexpr uint32_t kOrderMin = 32;
constexpr int kOrderClasses = 33;
static_assert(kMaxGrp + 33 <= kHRound, "a round word per doubling");
static_assert(kHRound + 33 <= kStateWords, "an h word per doubling");
// A round whose groups all fit the local part sorts them by the ranks at
// i + h and i + 2h (h -> 3h) when both fit one 64-bit key beside the
// bitonic sort's chunk and lane fields: ranks + 1 below 2^26.
constexpr int kTripleBits = 26;
constexpr int64_t kTripleMaxM = (1ll << kTripleBits) - 2;
static_assert(kCap <= kPosTile, "a group spans at most two tiles");

struct SaWs {
  uint64_t* keyA;
  uint64_t* keyB;
  uint32_t* valA;
  uint32_t* valB;
  uint32_t* pos;      // SA positions of the global list (ascending)
  uint32_t* rank[2];  // [m] group head of text position i; round r reads
                      // rank[r & 1] and writes rank[(r + 1) & 1]
  uint32_t* sa;       // [m] current suffix order
  uint32_t* gp;       // [m] group head of SA position p, or a finished mark
  uint32_t* gsz;      // [m] size of the group headed at p
  uint32_t* hist;     // [NB][512] digit counts per tile, then offsets
  uint32_t* rowsum;   // [512] digit totals
  uint32_t* tcnt;     // [NB] unfinished positions per tile
  uint32_t* blkmax;   // [NB] last group start per tile
  uint32_t* skip[2];  // [NL + 1] leading positions of a local tile owned
                      // by the tile before; round r reads skip[r & 1]
  uint32_t* tmax[2];  // [NL + 1] largest group (above kOrderMin) headed in
                      // a local tile, as the token round's and the radix
                      // parts' group-head passes record them; round r's
                      // tile order reads tmax[r & 1]
  uint32_t* order;    // [NL] the local tiles, largest groups first
  uint32_t* state;    // the state[] words above
};

static size_t sa_ws_layout(int64_t n, void* base, SaWs* w) {
  const size_t N = (size_t)(n > 0 ? n : 1);
  const size_t NB = (N + kTile - 1) / kTile;
  const size_t NL = (N + kPosTile - 1) / kPosTile;
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
  s.rank[0] = (uint32_t*)take(N * 4);
  s.rank[1] = (uint32_t*)take(N * 4);
  s.sa = (uint32_t*)take(N * 4);
  s.gp = (uint32_t*)take(N * 4);
  s.gsz = (uint32_t*)take(N * 4);
  s.hist = (uint32_t*)take((size_t)kRadix * NB * 4);
  s.rowsum = (uint32_t*)take(kRadix * 4);
  s.tcnt = (uint32_t*)take(NB * 4);
  s.blkmax = (uint32_t*)take(NB * 4);
  s.skip[0] = (uint32_t*)take((NL + 1) * 4);
  s.skip[1] = (uint32_t*)take((NL + 1) * 4);
  s.tmax[0] = (uint32_t*)take((NL + 1) * 4);
  s.tmax[1] = (uint32_t*)take((NL + 1) * 4);
  s.order = (uint32_t*)take(NL * 4);
  s.state = (uint32_t*)take(kStateWords * 4);
  if (w) *w = s;
  return off;
}

__device__ __forceinline__ int64_t tiles_of(int64_t a) {
  return (a + kTile - 1) / kTile;
}

// True when round r's radix launches have nothing to do: the array is
// final, the build stalled, or the round is a local one (round 0 is
// always a radix round).
__device__ __forceinline__ bool radix_idle(const uint32_t* state, int round) {
  return state[kDone] || state[kStalled] ||
         (round > 0 && state[kMaxGrp + round] <= (uint32_t)kCap);
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

// Block-wide least and largest of one int32 per thread (all NT threads).
template <int NT>
__device__ __forceinline__ void block_minmax(int32_t& lo, int32_t& hi,
                                             int32_t (*red)[NT / kWave]) {
  lo = ~wave_max_i32(~lo);  // ~ reverses the signed order, no overflow
  hi = wave_max_i32(hi);
  const int wv = threadIdx.x / kWave;
  if (lane_id() == 0) {
    red[0][wv] = lo;
    red[1][wv] = hi;
  }
  __syncthreads();
  for (int w = 0; w < NT / kWave; ++w) {
    lo = red[0][w] < lo ? red[0][w] : lo;
    hi = red[1][w] > hi ? red[1][w] : hi;
  }
}

// Least and largest token of the text, PAD (INT32_MAX) left out, per
// block (part_lo / part_hi, gridDim.x <= kInitParts entries each).
constexpr int kRangeThreads = 1024;
constexpr int kInitThreads = 1024;
constexpr int kInitParts = 256;  // partials k_sa_init reduces

__global__ __launch_bounds__(kRangeThreads) void k_sa_range(
    const int32_t* text, int64_t n, int32_t* part_lo, int32_t* part_hi) {
  __shared__ int32_t red[2][kRangeThreads / kWave];
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
  block_minmax<kRangeThreads>(lo, hi, red);
  if (threadIdx.x == 0) {
    part_lo[blockIdx.x] = lo;
    part_hi[blockIdx.x] = hi;
  }
}

__device__ __forceinline__ uint32_t digit_of(uint64_t k, int sh) {
  return (uint32_t)(k >> sh) & (kRadix - 1u);
}

// Tokens of the pair keys: 1 + t - least, PAD after every other token, 0
// past the end; pair keys need span + 2 < 2^kPairBits.
constexpr int kPairBits = 18;

// The token round's sort key of position i (below the vb position bits):
// with `pairs`, code(t[i]) << kPairBits | code(t[i + 1]), code(t) = 1 +
// t - lo, span + 1 for PAD, 0 past the end; else t[i] in signed order.
struct TokenCoding {
  int32_t lo;
  int64_t span;
  bool pairs;
};

__device__ __forceinline__ TokenCoding token_coding(int32_t lo, int32_t hi) {
  TokenCoding c;
  c.lo = lo;
  // hi < lo: the text is all PAD
  c.span = hi < lo ? 0 : (int64_t)hi - (int64_t)lo + 1;
  c.pairs = c.span + 2 < ((int64_t)1 << kPairBits);
  return c;
}

__device__ __forceinline__ uint64_t token_code(const TokenCoding& c,
                                               int32_t t, bool in_text) {
  if (!in_text) return 0;
  return t == INT32_MAX ? (uint64_t)c.span + 1
                        : (uint64_t)((int64_t)t - c.lo + 1);
}

__device__ __forceinline__ uint64_t token_key(const TokenCoding& c,
                                              int32_t t0, int32_t t1,
                                              bool t1_in_text) {
  return c.pairs ? (token_code(c, t0, true) << kPairBits) |
                       token_code(c, t1, t1_in_text)
                 : (uint64_t)((uint32_t)t0 ^ 0x80000000u);
}

// vb > 0: the key carries the position in its low vb bits (no value or
// position arrays), and the token round's first scatter computes the keys
// from the text itself, so none are written here; vb = 0: key, value and
// position arrays.  Each thread keys kInitItems consecutive positions, so
// a block keys one radix tile, and the block also writes that tile's
// digit counts for the first radix pass (digit at bit vb) to
// hist[tile * 512 + d].
constexpr int kInitItems = 4;
static_assert(kInitThreads * kInitItems == kTile, "a block per radix tile");

__global__ __launch_bounds__(kInitThreads) void k_sa_init(
    const int32_t* text, int64_t n, uint64_t* key, uint32_t* val,
    uint32_t* pos, int vb, const int32_t* part_lo, const int32_t* part_hi,
    int nparts, uint32_t* skip0, uint32_t* skip1, uint32_t* tmax0,
    uint32_t* tmax1, int64_t nl, uint32_t* hist, int64_t nb,
    uint32_t* state) {
  __shared__ int32_t red[2][kInitThreads / kWave];
  __shared__ uint32_t hcnt[kRadix];
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int d = threadIdx.x; d < kRadix; d += kInitThreads) hcnt[d] = 0;
  int32_t tlo = (int)threadIdx.x < nparts ? part_lo[threadIdx.x] : INT32_MAX;
  int32_t thi = (int)threadIdx.x < nparts ? part_hi[threadIdx.x] : INT32_MIN;
  block_minmax<kInitThreads>(tlo, thi, red);
  const TokenCoding tc = token_coding(tlo, thi);
  const bool pairs = tc.pairs;
  if (tid < kStateWords) {
    uint32_t v = 0;
    if (tid == kLen) v = (uint32_t)n;
    if (tid == kTokLo) v = (uint32_t)tlo;
    if (tid == kTokHi) v = (uint32_t)thi;
    if (tid == kH0 || tid == kHRound + 1) v = pairs ? 2u : 1u;
    if (tid == kGlobalMask) v = 1u;  // round 0 is a radix round
    state[tid] = v;
  }
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = tid; e <= nl; e += stride) {
    skip0[e] = 0;
    skip1[e] = 0;
    tmax0[e] = 0;
    tmax1[e] = 0;
  }
  // Every thread passes both barriers below (a thread past n keys
  // nothing): a barrier in divergent code would pair up wrongly.
  const int64_t i0 = tid * kInitItems;
  // tokens i0 .. i0 + kInitItems (the last one: the pair partner)
  int32_t t[kInitItems + 1];
#pragma unroll
  for (int j = 0; j <= kInitItems; ++j)
    t[j] = i0 + j < n ? text[i0 + j] : 0;
  uint64_t k[kInitItems];
#pragma unroll
  for (int j = 0; j < kInitItems; ++j) {
    k[j] = token_key(tc, t[j], t[j + 1], i0 + j + 1 < n);
    if (vb > 0) k[j] = (k[j] << vb) | (uint64_t)(i0 + j);
  }
  __syncthreads();  // the counters are cleared
#pragma unroll
  for (int j = 0; j < kInitItems; ++j)
    if (i0 + j < n) atomicAdd(&hcnt[digit_of(k[j], vb)], 1u);
  __syncthreads();
  if (threadIdx.x < kRadix)
    hist[(int64_t)blockIdx.x * kRadix + threadIdx.x] = hcnt[threadIdx.x];
  if (i0 >= n || vb > 0) return;
  if (i0 + kInitItems <= n) {
    // key, val and pos are 256-byte aligned workspace arrays
    static_assert(kInitItems == 4, "two 16-byte key stores");
    reinterpret_cast<ulonglong2*>(key + i0)[0] = make_ulonglong2(k[0], k[1]);
    reinterpret_cast<ulonglong2*>(key + i0)[1] = make_ulonglong2(k[2], k[3]);
    const uint32_t p = (uint32_t)i0;
    const uint4 ix = make_uint4(p, p + 1, p + 2, p + 3);
    *reinterpret_cast<uint4*>(val + i0) = ix;
    *reinterpret_cast<uint4*>(pos + i0) = ix;
  } else {
#pragma unroll
    for (int j = 0; j < kInitItems; ++j) {
      if (i0 + j < n) {
        key[i0 + j] = k[j];
        val[i0 + j] = (uint32_t)(i0 + j);
        pos[i0 + j] = (uint32_t)(i0 + j);
      }
    }
  }
}

__device__ __forceinline__ uint64_t lanes_le(int ln) {
  return ln == kWave - 1 ? ~0ull : (2ull << ln) - 1;
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


// ---------------------------------------------------------------- radix
// The passes run NT threads per 4096-element tile.  With about one active
// tile per CU, 1024 threads (16 waves) keep four times more loads and LDS
// operations in flight per CU than 256 threads would.

constexpr int kRsThreads = 1024;
constexpr int kRsHists = 4;  // LDS sub-histograms of the histogram pass

template <int NT>
__global__ __launch_bounds__(NT) void k_rs_hist(
    const uint64_t* __restrict__ key, int sh, uint32_t* hist, int64_t nb,
    const uint32_t* state, int round) {
  static_assert(kTile % NT == 0 && NT >= kRadix, "tile shape");
  constexpr int kItems = kTile / NT;
  if (radix_idle(state, round)) return;
  const int64_t A = state[kLen];
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
    hist[(int64_t)blockIdx.x * kRadix + tid] = sum;
  }
}

// The histogram is stored by tile, hist[t * 512 + d]: a tile's counts are
// one contiguous 2 KB row, written and read back by its own tile's
// workgroups with whole-sector accesses (a column-major layout costs a
// 32-byte sector per 4-byte count on both sides).  Column d (tiles
// 0 .. ceil(A/4096)) becomes its exclusive prefix; rowsum[d] the digit
// total.  Block j scans the kScanDigits digits from j * kScanDigits: lane
// (part, d) = (tid / kScanDigits, tid % kScanDigits) sums kScanRun
// consecutive tiles, so the kScanDigits lanes of a part read and write one
// 128-byte line per tile.  The parts of a wave (the lanes kScanDigits
// apart) are scanned by shuffles, the waves through LDS.
constexpr int kScanDigits = 32;
constexpr int kScanRun = 32;
static_assert(kRadix % kScanDigits == 0 && kWave % kScanDigits == 0,
              "digit blocks");
constexpr int kScanBlocks = kRadix / kScanDigits;

template <int NT>
__global__ __launch_bounds__(NT) void k_rs_rowscan(
    uint32_t* hist, int64_t nb, uint32_t* rowsum, const uint32_t* state,
    int round) {
  constexpr int NW = NT / kWave;
  constexpr int kChunk = NT / kScanDigits * kScanRun;  // tiles per pass
  if (radix_idle(state, round)) return;
  __shared__ uint32_t wtot[NW][kScanDigits];
  const int ln = lane_id();
  const int wv = threadIdx.x / kWave;
  const int dl = threadIdx.x % kScanDigits;
  const int part = threadIdx.x / kScanDigits;
  uint32_t* col = hist + (int64_t)blockIdx.x * kScanDigits + dl;
  const int64_t nbA = tiles_of(state[kLen]);
  uint32_t carry = 0;
  for (int64_t c0 = 0; c0 < nbA; c0 += kChunk) {
    const int64_t t0 = c0 + (int64_t)part * kScanRun;
    uint32_t v[kScanRun];
#pragma unroll
    for (int r = 0; r < kScanRun; ++r)
      v[r] = t0 + r < nbA ? col[(t0 + r) * kRadix] : 0u;
    uint32_t sum = 0;
#pragma unroll
    for (int r = 0; r < kScanRun; ++r) {
      const uint32_t x = v[r];
      v[r] = sum;
      sum += x;
    }
    // inclusive over the wave's parts of digit dl
    uint32_t inc = sum;
#pragma unroll
    for (int off = kScanDigits; off < kWave; off <<= 1) {
      const uint32_t o = __shfl_up(inc, off);
      if (ln >= off) inc += o;
    }
    if (ln >= kWave - kScanDigits) wtot[wv][dl] = inc;
    __syncthreads();
    uint32_t before = inc - sum, all = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t x = wtot[w][dl];
      if (w < wv) before += x;
      all += x;
    }
    __syncthreads();  // wtot is rewritten by the next pass
#pragma unroll
    for (int r = 0; r < kScanRun; ++r)
      if (t0 + r < nbA) col[(t0 + r) * kRadix] = carry + before + v[r];
    carry += all;
  }
  if (part == 0) rowsum[(int64_t)blockIdx.x * kScanDigits + dl] = carry;
}

// Stable scatter of one tile.  Wave w owns the tile's contiguous span
// base + w * kTile / NW .. + kTile / NW, 64 consecutive elements per step,
// so the element order is (wave, step, lane).  The waves first count their
// digits (LDS atomics); one scan over the digits gives each digit's first
// slot in the tile and each (wave, digit) its slot, and each wave places
// its elements into LDS step by step (a nine-ballot digit match) in digit
// order.  The tile is then written out from LDS by consecutive threads, so
// each store instruction writes the runs of a few digits contiguously
// instead of up to 64 scattered words.  Four barriers per tile.
// kText: the token round's first pass (packed keys, sh = vb), which keys
// position idx from text[idx], text[idx + 1] as k_sa_init does instead of
// reading keys (kin unused).
template <int NT, bool kVal = true, bool kText = false>
__global__ __launch_bounds__(NT) void k_rs_scatter(
    const uint64_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint64_t* __restrict__ kout, uint32_t* __restrict__ vout, int sh,
    const uint32_t* __restrict__ hist, int64_t nb,
    const uint32_t* __restrict__ rowsum, const uint32_t* state, int round,
    const int32_t* __restrict__ text) {
  static_assert(!(kText && kVal), "the text pass packs the position");
  constexpr int NW = NT / kWave;
  constexpr int kSpan = kTile / NW;
  constexpr int kSteps = kSpan / kWave;
  static_assert(kTile % NT == 0 && NT >= kRadix, "tile shape");
  if (radix_idle(state, round)) return;
  const int64_t A = state[kLen];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  __shared__ uint32_t woff[NW][kRadix];
  __shared__ uint32_t gdelta[kRadix];  // global slot - tile slot, per digit
  __shared__ uint64_t sk[kTile];
  __shared__ uint32_t sv[kVal ? kTile : 1];
  __shared__ uint32_t red[NW];
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int ln = lane_id();
  const int64_t wbase = base + (int64_t)wv * kSpan;
  const int nvalid = (int)(A - base < kTile ? A - base : kTile);
  uint64_t k[kSteps];
  uint32_t v[kSteps];
  uint64_t peers[kSteps];  // lanes of the same step holding the same digit
  if (kText) {
    const TokenCoding tc =
        token_coding((int32_t)state[kTokLo], (int32_t)state[kTokHi]);
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const int64_t idx = wbase + s * kWave + ln;
      const int32_t t0 = idx < A ? text[idx] : 0;
      const int32_t t1 = idx + 1 < A ? text[idx + 1] : 0;
      k[s] = idx < A ? (token_key(tc, t0, t1, idx + 1 < A) << sh) |
                           (uint64_t)idx
                     : 0;
      v[s] = 0;
    }
  } else {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const int64_t idx = wbase + s * kWave + ln;
      k[s] = idx < A ? kin[idx] : 0;
      v[s] = kVal && idx < A ? vin[idx] : 0;
    }
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
  // thread d: the tile's count of digit d, then its first tile slot
  uint32_t cnt = 0;
  if (tid < kRadix) {
#pragma unroll
    for (int w = 0; w < NW; ++w) cnt += woff[w][tid];
  }
  uint32_t ttot;
  const uint32_t ls = block_exscan1<NT>(cnt, red, &ttot);
  if (tid < kRadix) {
    gdelta[tid] = dbase + hist[(int64_t)blockIdx.x * kRadix + tid] - ls;
    uint32_t run = ls;
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
      sk[p] = k[s];
      if (kVal) sv[p] = v[s];
    }
    wave_lds_sync();  // every lane has read its offset
    if (act && rk == 0) woff[wv][d] += (uint32_t)popc(peers[s]);
    wave_lds_sync();
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTile / NT; ++i) {
    const int j = tid + i * NT;
    if (j < nvalid) {
      const uint64_t kk = sk[j];
      const uint32_t p = gdelta[digit_of(kk, sh)] + (uint32_t)j;
      kout[p] = kk;
      if (kVal) vout[p] = sv[j];
    }
  }
}

// ----------------------------------------------------------- group heads
// Over the sorted active list: slot t starts a group when its key differs
// from slot t-1's; the group's head is pos[start] (pos ascends with t, so
// the head of slot t is the largest start position at or before t).  Wave
// w of a tile owns slots base + w*1024 .. +1024, 64 consecutive per step.
// vb > 0 (the token round's packed keys): the key above its low vb bits is
// the sort key, the low bits the value, and pos[t] = t.

__device__ __forceinline__ bool starts_group(const uint64_t* key, int64_t t,
                                             uint64_t kt, int vb) {
  return t == 0 || (key[t - 1] >> vb) != kt;
}

template <int NT>
__global__ __launch_bounds__(NT) void k_grp_reduce(
    const uint64_t* __restrict__ key, const uint32_t* __restrict__ pos,
    int vb, uint32_t* blkmax, const uint32_t* state, int round) {
  constexpr int NW = NT / kWave;
  constexpr int kSpan = kTile / NW;
  if (radix_idle(state, round)) return;
  const int64_t A = state[kLen];
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
      const uint64_t kt = key[t] >> vb;
      if (starts_group(key, t, kt, vb))
        mx = max(mx, vb ? (uint32_t)t : pos[t]);
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

// Over the sorted list of round r: rank_next[val[t]] = head,
// sa[pos[t]] = val[t], gp[pos[t]] = head, or kJustFinished when t's group
// is the singleton {t}; at the last entry of a larger group its size goes
// to gsz[head] and to the round's largest-group word, and a group that
// runs from one local tile into the next sets the skip_next[] word of the
// tile its last entry lies in (the round's local launch, which precedes
// this one, cleared it).  The group start carried into a tile is the
// largest start of all earlier tiles: each block reduces
// blkmax[0 .. tile) itself.
template <int NT>
__global__ __launch_bounds__(NT) void k_grp_rank(
    const uint64_t* __restrict__ key, const uint32_t* __restrict__ val,
    const uint32_t* __restrict__ pos, int vb,
    const uint32_t* __restrict__ blkmax,
    uint32_t* __restrict__ rank_next, uint32_t* __restrict__ sa,
    uint32_t* __restrict__ gp, uint32_t* __restrict__ gsz,
    uint32_t* __restrict__ skip_next, uint32_t* __restrict__ tmax_next,
    uint32_t* state, int round) {
  constexpr int NW = NT / kWave;
  constexpr int kSpan = kTile / NW;
  constexpr int kSteps = kSpan / kWave;
  static_assert(kSteps <= 32, "per-entry bits in one word");
  if (radix_idle(state, round)) return;
  const int64_t A = state[kLen];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  if (base >= A) return;
  __shared__ uint32_t smax[NW];
  __shared__ uint32_t cred[NW];
  __shared__ uint32_t gmax[NW];
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
  uint32_t lastb = 0;   // bit s: entry s ends its group
  uint32_t mx = 0;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t t = wbase + s * kWave + ln;
    st[s] = 0;
    if (t < A) {
      const uint64_t kt = key[t] >> vb;
      const bool first = starts_group(key, t, kt, vb);
      const bool last = t + 1 == A || (key[t + 1] >> vb) != kt;
      if (first) st[s] = vb ? (uint32_t)t : pos[t];
      single |= (uint32_t)(first && last) << s;
      lastb |= (uint32_t)last << s;
    }
    mx = max(mx, st[s]);
  }
  mx = (uint32_t)wave_max_i32((int)mx);
  if (ln == 0) smax[wv] = mx;
  __syncthreads();
  uint32_t run = 0;
  for (int w = 0; w < NW; ++w) run = max(run, cred[w]);
  for (int w = 0; w < wv; ++w) run = max(run, smax[w]);
  uint32_t big = 0;  // largest group ending in this lane's entries
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t t = wbase + s * kWave + ln;
    const uint32_t head = max(run, wave_incl_max(st[s]));
    run = max(run, (uint32_t)__builtin_amdgcn_readlane((int)head, kWave - 1));
    const bool fin = (single >> s) & 1u;
    if (t < A) {
      const uint32_t i =
          vb ? (uint32_t)(key[t] & ((1ull << vb) - 1)) : val[t];
      const uint32_t p = vb ? (uint32_t)t : pos[t];
      rank_next[i] = head;
      sa[p] = i;
      gp[p] = fin ? kJustFinished : head;
      if (((lastb >> s) & 1u) && !fin) {
        const uint32_t size = p - head + 1;
        gsz[head] = size;
        big = max(big, size);
        const uint32_t c = p / kPosTile;
        if (head / kPosTile < c) skip_next[c] = p + 1 - c * kPosTile;
        if (size > kOrderMin) atomicMax(&tmax_next[head / kPosTile], size);
      }
    }
  }
  big = (uint32_t)wave_max_i32((int)big);
  if (ln == 0) gmax[wv] = big;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t g = 0;
    for (int w = 0; w < NW; ++w) g = max(g, gmax[w]);
    if (g) atomicMax(&state[kMaxGrp + round + 1], g);
  }
}

// ------------------------------------------------------- radix part
// The suffixes of a round's groups of more than kCap.  k_pos_count: per
// tile of SA positions, how many lie in such a group (tcnt[]) and how many
// of them are a group's head (hcnt[]).  It runs after the round's local
// launch, which changed only groups of at most kCap.
__device__ __forceinline__ bool in_big_group(const uint32_t* gsz, uint32_t g) {
  return g < kJustFinished && gsz[g] > (uint32_t)kCap;
}

// Groups of more than kCap among m suffixes, at most (and at least 1).
__host__ __device__ inline int64_t big_groups_max(int64_t m) {
  const int64_t n = m / (kCap + 1);
  return n > 1 ? n : 1;
}

template <int NT>
__global__ __launch_bounds__(NT) void k_pos_count(
    const uint32_t* __restrict__ gp, const uint32_t* __restrict__ gsz,
    uint32_t* __restrict__ tcnt, uint32_t* __restrict__ hcnt, int64_t m,
    const uint32_t* state, int round) {
  if (radix_idle(state, round)) return;
  __shared__ uint32_t red[NT / kWave];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  uint32_t c = 0, hc = 0;
#pragma unroll
  for (int s = 0; s < kTile / NT; ++s) {
    const int64_t p = base + s * NT + threadIdx.x;
    if (p < m) {
      const uint32_t g = gp[p];
      const bool big = in_big_group(gsz, g);
      c += big;
      hc += big && g == (uint32_t)p;
    }
  }
  uint32_t tot, htot;
  block_exscan1<NT>(c, red, &tot);
  block_exscan1<NT>(hc, red, &htot);
  if (threadIdx.x == 0) {
    tcnt[blockIdx.x] = tot;
    hcnt[blockIdx.x] = htot;
  }
}

// The round's list: the SA positions of its groups of more than kCap in
// order, keyed q * (m + 1) + (rank[i + h] + 1, or 0 past the end) with
// i = sa[p] and q the group's ordinal among those groups (its head's: the
// list is in SA order, so q + 1 counts the heads at or before p; below
// big_groups_max(m), so the key takes fewer bits than the head would).
// Each block sums the earlier tiles' counts for its output offset and
// ordinal base; block 0 also sums them all: the list length (state[kLen]).
template <int NT>
__global__ __launch_bounds__(NT) void k_pos_gather(
    const uint32_t* __restrict__ gp, const uint32_t* __restrict__ gsz,
    const uint32_t* __restrict__ sa,
    const uint32_t* __restrict__ rank_cur, const uint32_t* __restrict__ tcnt,
    const uint32_t* __restrict__ hcnt, int64_t m, int64_t nb, int round,
    uint64_t* __restrict__ key, uint32_t* __restrict__ val,
    uint32_t* __restrict__ pos, uint32_t* state) {
  constexpr int NW = NT / kWave;
  constexpr int kSpan = kTile / NW;
  constexpr int kSteps = kSpan / kWave;
  if (radix_idle(state, round)) return;
  const int64_t h = state[kHRound + round];
  const int64_t base = (int64_t)blockIdx.x * kTile;
  __shared__ uint32_t scnt[NW];
  __shared__ uint32_t shcnt[NW];
  __shared__ uint32_t ored[NW];
  __shared__ uint32_t hbase;
  {
    const int64_t upto = blockIdx.x == 0 ? nb : (int64_t)blockIdx.x;
    uint32_t c = 0, hc = 0;
    for (int64_t t = threadIdx.x; t < upto; t += NT) {
      c += tcnt[t];
      hc += (int64_t)t < (int64_t)blockIdx.x ? hcnt[t] : 0u;
    }
    uint32_t tot, htot;
    block_exscan1<NT>(hc, ored, &htot);
    if (threadIdx.x == 0) hbase = htot;
    block_exscan1<NT>(c, ored, &tot);
    if (blockIdx.x == 0) {
      if (threadIdx.x == 0) {
        state[kLen] = tot;
        state[kGlobalMask] |= 1u << round;
      }
      ored[0] = 0;  // block 0's own offset (the barrier below publishes it)
    } else if (threadIdx.x == 0) {
      ored[0] = tot;
    }
  }
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  const int64_t wbase = base + (int64_t)wv * kSpan;
  uint32_t gv[kSteps];
  uint32_t cnt = 0, hcn = 0;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t p = wbase + s * kWave + ln;
    gv[s] = p < m ? gp[p] : kFinished;
    if (!in_big_group(gsz, gv[s])) gv[s] = kFinished;
    cnt += (uint32_t)popc(ballot(gv[s] != kFinished));
    hcn += (uint32_t)popc(ballot(gv[s] == (uint32_t)p));
  }
  if (ln == 0) {
    scnt[wv] = cnt;
    shcnt[wv] = hcn;
  }
  __syncthreads();
  uint32_t out = ored[0];
  uint32_t hrun = hbase;
  for (int w = 0; w < wv; ++w) {
    out += scnt[w];
    hrun += shcnt[w];
  }
  const uint64_t M1 = (uint64_t)m + 1;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t p = wbase + s * kWave + ln;
    const bool a = gv[s] != kFinished;
    const uint64_t bm = ballot(a);
    const uint64_t hm = ballot(a && gv[s] == (uint32_t)p);
    if (a) {
      const uint32_t o = out + (uint32_t)rank_lt(bm);
      // heads at or before p in this step, then the group's ordinal
      const uint32_t q = hrun + (uint32_t)popc(hm & lanes_le(ln)) - 1u;
      const uint32_t i = sa[p];
      const uint64_t k2 =
          (int64_t)i + h < m ? (uint64_t)rank_cur[i + h] + 1 : 0;
      key[o] = (uint64_t)q * M1 + k2;
      val[o] = i;
      pos[o] = (uint32_t)p;
    }
    out += (uint32_t)popc(bm);
    hrun += (uint32_t)popc(hm);
  }
}

// ------------------------------------------------------------ tile order
// A local round's workgroups take its tiles largest group first: a tile
// with a group of hundreds of suffixes takes several times as long as one
// of small groups, and when the large ones start last they set the
// round's end.  order[] lists the tiles by the size class of their
// largest group (tmax, recorded by the previous round for groups above
// kOrderMin), largest first; within a class in any order (every tile's
// result is the same whichever workgroup takes it and when).  Only rounds
// with a radix part are ordered: the groups above the cap that make the
// radix part are recorded by the group-head pass of the round before (the
// token round for round 1), and the order kernel clears the other tmax
// buffer for this round's radix part.

__device__ __forceinline__ int order_class(uint32_t t) {
  // 0 for tmax <= kOrderMin, else 1 + floor(log2(t)) - 5
  return t <= kOrderMin ? 0 : 32 - __builtin_clz(t) - 5;
}

// Workgroups are handed to the 8 XCDs in turn (workgroup b to XCD b % 8),
// and a tile stays with its XCD from round to round when workgroup b takes
// tile b, so the XCD's L2 still holds what the round before wrote of it.
// The order keeps that: workgroup b takes a tile t = b mod 8, the largest
// group first among those tiles.
constexpr int kXcds = 8;

template <int NT>
__global__ __launch_bounds__(NT) void k_sa_order(
    const uint32_t* __restrict__ tmax, uint32_t* __restrict__ tmax_next,
    uint32_t* __restrict__ order, int64_t nl, const uint32_t* state) {
  if (state[kDone]) return;
  // cleared for the round's radix part, which records its groups there
  for (int64_t t = threadIdx.x; t <= nl; t += NT) tmax_next[t] = 0;
  __shared__ uint32_t cnt[kXcds][kOrderClasses];
  __shared__ uint32_t cur[kXcds][kOrderClasses];
  for (int c = threadIdx.x; c < kXcds * kOrderClasses; c += NT)
    (&cnt[0][0])[c] = 0;
  __syncthreads();
  for (int64_t t = threadIdx.x; t < nl; t += NT)
    atomicAdd(&cnt[t % kXcds][order_class(tmax[t])], 1u);
  __syncthreads();
  if (threadIdx.x < kXcds) {
    const int x = threadIdx.x;
    uint32_t run = 0;
    for (int c = kOrderClasses - 1; c >= 0; --c) {
      cur[x][c] = run;
      run += cnt[x][c];
    }
  }
  __syncthreads();
  for (int64_t t = threadIdx.x; t < nl; t += NT) {
    const int x = (int)(t % kXcds);
    const uint32_t r = atomicAdd(&cur[x][order_class(tmax[t])], 1u);
    order[(int64_t)r * kXcds + x] = (uint32_t)t;
  }
}

// -------------------------------------------------------- local rounds
// Ascending sort of one u64 per lane across the wave (bitonic network).
__device__ __forceinline__ uint64_t wave_sort_u64(uint64_t v) {
  const int ln = lane_id();
#pragma unroll
  for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint32_t ol = (uint32_t)__shfl_xor((int)(uint32_t)v, j);
      const uint32_t oh = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), j);
      const uint64_t o = ((uint64_t)oh << 32) | ol;
      const bool take_min = ((ln & j) == 0) == ((ln & k) == 0);
      const bool less = v < o;
      v = (take_min == less) ? v : o;
    }
  }
  return v;
}

// The value of lane ln - 1 (lane 0: its own) and of lane ln + 1 (lane 63:
// its own), by DPP wave shifts (wave_shr:1 / wave_shl:1).
__device__ __forceinline__ uint32_t lane_prev(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x138, 0xf,
                                               0xf, false);
}
__device__ __forceinline__ uint32_t lane_next(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x130, 0xf,
                                               0xf, false);
}

__device__ __forceinline__ uint64_t lane_prev64(uint64_t v) {
  return ((uint64_t)lane_prev((uint32_t)(v >> 32)) << 32) |
         lane_prev((uint32_t)v);
}
__device__ __forceinline__ uint64_t lane_next64(uint64_t v) {
  return ((uint64_t)lane_next((uint32_t)(v >> 32)) << 32) |
         lane_next((uint32_t)v);
}


// Entries of c[0 .. len) (ascending, len <= 64) below key, or at most key
// when `incl`.
__device__ __forceinline__ int count_below(const uint64_t* c, int len,
                                           uint64_t key, bool incl) {
  int at = 0;
#pragma unroll
  for (int step = kWave; step >= 1; step >>= 1) {
    const int q = at + step;
    if (q <= len) {
      const uint64_t v = c[q - 1];
      if (incl ? v <= key : v < key) at = q;
    }
  }
  return at;
}

// The local part of a round: the groups of at most kCap suffixes.
// Workgroup b owns those whose head lies in its kPosTile-position tile b.
// It reads the tile and the tail of a group running on into the next
// tile (at most kCap - 1 positions) as slots s = p - ts; window
// w = slots 64w .. 64w + 63, held by wave w mod NW, lane = slot mod 64.
// The first skip_cur[b] positions belong to the group that runs in from
// the tile before; that tile's workgroup rewrites them meanwhile, so they
// are never read as owned.
//  1. per slot: gp, then sa where unfinished, then for an owned one its
//     group size and key rank_cur[i + h] + 1; positions of the tile the
//     previous round finished get their final rank in rank_next;
//  2. per window: the lanes of one group form a chunk; one bitonic sort by
//     (chunk, key, lane) sorts every chunk in place; the sorted keys go to
//     LDS, and equal-key runs inside the chunk are found by lane masks;
//  3. per element: counts of keys below / at most its own in every other
//     chunk of its group (binary search in LDS) give its new position
//     (ties by old position), its new group's head and its size; it writes
//     sa, gp, rank_next, and the head writes gsz; skip_next[b + 1] gets
//     the length of the group running into the next tile, or 0 (the
//     round's radix part then sets it for a group it sorted).
// Groups above kCap are left to the round's radix launches; when the
// caller enqueued none (global_follows == 0) this launch marks the round
// stalled and does nothing.  A round with no group left sets the done
// flag.  kExpectDone: the caller expects the array to be final by this
// round (a rebuild's margin rounds), so the launch reads the state words
// before the tile's group marks, which it then reads only if the round
// has work after all.  (A separate instantiation: a run-time switch
// changed the load schedule of every round.)
template <int NT, bool kExpectDone>
__global__ __launch_bounds__(NT) void k_sa_local(
    uint32_t* __restrict__ gp, uint32_t* __restrict__ gsz,
    uint32_t* __restrict__ sa, const uint32_t* __restrict__ rank_cur,
    uint32_t* __restrict__ rank_next, const uint32_t* __restrict__ skip_cur,
    uint32_t* __restrict__ skip_next, const uint32_t* __restrict__ order,
    int64_t m, int64_t nl, int round, int global_follows, uint32_t* state) {
  constexpr int NW = NT / kWave;
  constexpr int kW = kSlots / kWave / NW;  // windows per wave
  static_assert(kSlots % (kWave * NW) == 0, "windows per wave");
  static_assert(kPosTile % (kWave * NW) == 0, "tile windows per wave");
  // this workgroup's tile (order: NULL for tile = workgroup)
  const int64_t b = order ? (int64_t)order[blockIdx.x] : (int64_t)blockIdx.x;
  const int64_t ts = b * kPosTile;
  const int wv = threadIdx.x / kWave;
  const int ln = lane_id();
  // The tile's group marks are read before the state and skip words are
  // known, so they share one round trip; the slots the skip words exclude
  // are dropped below.  (The suffixes are read only where a mark says
  // unfinished: reading them with the marks cost 16 MB more per round at
  // 2^22 tokens, and a round after the array is final reads the marks
  // alone.)  Slot (wv + k * NW) * 64 + ln lies in the tile for k < kWT.
  constexpr int kWT = kPosTile / kWave / NW;
  uint32_t gt[kWT];
#pragma unroll
  for (int k = 0; k < kWT; ++k) {
    const int64_t p = ts + (wv + k * NW) * kWave + ln;
    gt[k] = !kExpectDone && p < m ? gp[p] : kFinished;
  }
  // every word the launch decides on, loaded at once
  const uint32_t done = state[kDone];
  const uint32_t stalled = state[kStalled];
  const uint32_t mg = state[kMaxGrp + round];
  const int64_t h = state[kHRound + round];
  const int skip = (int)skip_cur[b];
  const uint32_t sn = b + 1 < nl ? skip_cur[b + 1] : 0u;
  // (kept together: the compiler would otherwise sink each load to its
  // first use past the early returns, one round trip each)
  asm volatile("" ::"s"(done), "s"(stalled), "s"(mg), "s"((uint32_t)h),
               "s"(skip), "s"(sn));
  if (done) return;
  if (stalled != 0 && stalled < (uint32_t)round) return;
  if (mg == 0) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      state[kDone] = 1;
      state[kFoundNone] = (uint32_t)round;
    }
    return;
  }
  if (mg > (uint32_t)kCap && !global_follows) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
      state[kStalled] = (uint32_t)round;
    return;
  }
  // a resumed round clears its stall mark before its radix launches
  if (stalled != 0 && blockIdx.x == 0 && threadIdx.x == 0)
    state[kStalled] = 0;
  if (kExpectDone) {
#pragma unroll
    for (int k = 0; k < kWT; ++k) {
      const int64_t p = ts + (wv + k * NW) * kWave + ln;
      gt[k] = p < m ? gp[p] : kFinished;
    }
  }
  // Every group fits this launch: sort by (rank[i + h], rank[i + 2h]) and
  // the round triples h; a round with a radix part doubles it.
  const bool triple = mg <= (uint32_t)kCap && m <= kTripleMaxM;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const int64_t hn = triple ? 3 * h : 2 * h;
    state[kHRound + round + 1] = (uint32_t)(hn < 0x7fffffff ? hn : 0x7fffffff);
  }
  __shared__ uint64_t sk[kSlots];  // sorted keys, chunk by chunk
  __shared__ uint32_t gmax[NW];
  __shared__ uint32_t skip_out;
  const int64_t te = min(ts + (int64_t)kPosTile, m);
  if (threadIdx.x == 0) skip_out = 0;
  // slots cover [ts, ts + n): the tile and the tail of the group that
  // runs on into the next tile (its skip word; a run of kCap or more
  // belongs to a group above kCap, not sorted here)
  const uint32_t ext = sn < (uint32_t)kCap ? sn : 0u;
  const int n = (int)(min(m, te + (int64_t)ext) - ts);

  // 1. loads: gp (the tile's above, the extension's here), then sa where
  // unfinished, then the group's size and key.  The first `skip` positions
  // belong to a group the tile before owns (its workgroup rewrites them
  // meanwhile): what was read of them is dropped.
  uint32_t g[kW], iv[kW], sz[kW];
  uint64_t kv[kW];
#pragma unroll
  for (int k = 0; k < kW; ++k) {
    const int slot = (wv + k * NW) * kWave + ln;
    if (k < kWT)
      g[k] = slot < n && slot >= skip ? gt[k] : kFinished;
    else
      g[k] = slot < n && slot >= skip ? gp[ts + slot] : kFinished;
  }
#pragma unroll
  for (int k = 0; k < kW; ++k) {
    const int slot = (wv + k * NW) * kWave + ln;
    iv[k] = g[k] != kFinished ? sa[ts + slot] : 0u;
  }
#pragma unroll
  for (int k = 0; k < kW; ++k) {
    const int slot = (wv + k * NW) * kWave + ln;
    sz[k] = 0;
    kv[k] = 0;
    if (g[k] == kJustFinished && slot < kPosTile) {
      rank_next[iv[k]] = (uint32_t)(ts + slot);
      gp[ts + slot] = kFinished;
    }
    // owned: a group whose head lies in the tile
    if (g[k] < kJustFinished && g[k] >= (uint32_t)ts && g[k] < (uint32_t)te) {
      sz[k] = gsz[g[k]];
      const int64_t i1 = (int64_t)iv[k] + h;
      uint64_t k2 = i1 < m ? (uint64_t)rank_cur[i1] + 1 : 0;
      if (triple) {
        const int64_t i2 = i1 + h;
        const uint64_t k3 = i2 < m ? (uint64_t)rank_cur[i2] + 1 : 0;
        k2 = (k2 << kTripleBits) | k3;
      }
      kv[k] = k2;
    } else {
      g[k] = kFinished;
    }
  }
#pragma unroll
  for (int k = 0; k < kW; ++k)  // a group above kCap is the radix part's
    if (sz[k] > (uint32_t)kCap) g[k] = kFinished;

  // 2. per window: sort each chunk; kept for step 3: the suffix now at
  // the lane (iv), the group's first slot and size (gs: slot | size << 16,
  // 0xffffffff for no group), the own-chunk counts and the lane the
  // element came from (own, a byte each)
  uint32_t gs[kW], own[kW];
#pragma unroll
  for (int k = 0; k < kW; ++k) {
    own[k] = 0;
    const bool act = g[k] != kFinished;
    gs[k] = act ? (g[k] - (uint32_t)ts) | (sz[k] << 16) : 0xffffffffu;
    const int base = (wv + k * NW) * kWave;
    if (base >= n || ballot(act) == 0) continue;
    const uint32_t gprev = lane_prev(g[k]);
    const bool start = ln == 0 || !act || gprev != g[k];
    const uint64_t starts = ballot(start);
    const uint64_t le = starts & lanes_le(ln);
    const int c0 = kWave - 1 - __builtin_clzll(le);
    const uint64_t after = starts & ~lanes_le(ln);
    const int c1 = after ? __builtin_ctzll(after) : kWave;
    uint64_t ke = act ? kv[k] : 0ull;
    int from = ln;  // the lane this lane's element came from
    // Most groups keep their order (keys equal or already ascending):
    // the sort runs only for a window with a descent inside a chunk.
    // (chunk index: 6 bits, key: at most 52, lane: 6)
    const uint64_t kin = lane_prev64(ke);
    if (ballot(ln > c0 && kin > ke)) {
      const uint64_t key64 = ((uint64_t)(popc(le) - 1) << 58) | (ke << 6) |
                             (uint64_t)ln;
      const uint64_t sorted = wave_sort_u64(key64);
      ke = (sorted >> 6) & ((1ull << 52) - 1);
      from = (int)(sorted & (kWave - 1));
      iv[k] = (uint32_t)__shfl((int)iv[k], from);
    }
    sk[base + ln] = ke;
    const uint64_t kprev = lane_prev64(ke);
    const uint64_t knext = lane_next64(ke);
    const bool eqprev = ln > c0 && kprev == ke;
    const bool eqnext = ln + 1 < c1 && knext == ke;
    const uint64_t rs = ballot(!eqprev) & lanes_le(ln);
    const int js = kWave - 1 - __builtin_clzll(rs);
    const uint64_t re = ballot(!eqnext) & ~(lanes_le(ln) >> 1);
    const int je = __builtin_ctzll(re);
    own[k] = (uint32_t)(ln - c0) | ((uint32_t)(js - c0) << 8) |
             ((uint32_t)(je - c0 + 1) << 16) | ((uint32_t)from << 24);
  }
  __syncthreads();

  // 3. counts in the group's other chunks, then the writes
  uint32_t big = 0;
#pragma unroll
  for (int k = 0; k < kW; ++k) {
    const int w = wv + k * NW;
    const int base = w * kWave;
    if (base >= n || gs[k] == 0xffffffffu) continue;
    const int g0 = (int)(gs[k] & 0xffffu);
    const uint32_t osz = gs[k] >> 16;  // the old group's size
    const uint32_t oh = (uint32_t)(ts + g0);  // and head
    const int g1 = min(g0 + (int)osz, n);
    const uint64_t ke = sk[base + ln];
    int stable = (int)(own[k] & 0xff);
    int lt = (int)((own[k] >> 8) & 0xff);
    int leq = (int)((own[k] >> 16) & 0xff);
    const int64_t p_old = ts + base + (int)(own[k] >> 24);
    for (int w2 = g0 / kWave; w2 <= (g1 - 1) / kWave; ++w2) {
      if (w2 == w) continue;
      const int a0 = max(g0, w2 * kWave);
      const int len = min(g1, w2 * kWave + kWave) - a0;
      const uint64_t lo_k = sk[a0], hi_k = sk[a0 + len - 1];
      int l2, e2;
      if (ke < lo_k) {
        l2 = e2 = 0;
      } else if (ke > hi_k) {
        l2 = e2 = len;
      } else if (lo_k == hi_k) {  // the whole chunk equals ke
        l2 = 0;
        e2 = len;
      } else {
        l2 = count_below(sk + a0, len, ke, false);
        e2 = count_below(sk + a0, len, ke, true);
      }
      lt += l2;
      leq += e2;
      stable += w2 < w ? e2 : l2;
    }
    const int64_t np = ts + g0 + stable;
    const uint32_t nh = (uint32_t)(ts + g0 + lt);
    const uint32_t size = (uint32_t)(leq - lt);
    const bool fin = size == 1;
    rank_next[iv[k]] = nh;
    // a group that keeps its order and head rewrites nothing else
    if (np != p_old || nh != oh || fin) {
      sa[np] = iv[k];
      gp[np] = fin ? kJustFinished : nh;
    }
    if (!fin && stable == lt) {  // the first entry of its new group
      if (nh != oh || size != osz) gsz[nh] = size;
      big = max(big, size);
      if (b + 1 < nl && (int64_t)nh < te && (int64_t)nh + size > te)
        skip_out = (uint32_t)((int64_t)nh + size - te);
    }
  }
  big = (uint32_t)wave_max_i32((int)big);
  if (ln == 0) gmax[wv] = big;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t gm = 0;
    for (int w = 0; w < NW; ++w) gm = max(gm, gmax[w]);
    if (gm) atomicMax(&state[kMaxGrp + round + 1], gm);
    if (b + 1 < nl) skip_next[b + 1] = skip_out;
  }
}

// ------------------------------------------------------------ outputs
// keys[r * W + j] = corpus[sa[r] + j] (-1 at or past n), ranks r < rows;
// first4[r * 4 + j] the same for j < 4 when first4 is not null.
__global__ __launch_bounds__(256) void k_rank_keys(const int32_t* corpus,
                                                 const int32_t* sa, int64_t n,
                                                 int64_t rows, int W,
                                                 int32_t* keys,
                                                 int32_t* first4) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * W) return;
  const int64_t r = e / W;
  const int j = (int)(e - r * W);
  const int64_t p = (int64_t)sa[r] + j;
  const int32_t v = p < n && p >= 0 ? corpus[p] : -1;
  keys[e] = v;
  if (first4 && j < 4) first4[r * 4 + j] = v;
}

// The same rows four tokens per thread with one 16-byte store (keys
// 16-byte aligned, W % 4 == 0): a quarter of the threads and store
// instructions for the 128 B-per-rank write that bounds the kernel.
__global__ __launch_bounds__(256) void k_rank_keys4(const int32_t* corpus,
                                                  const int32_t* sa, int64_t n,
                                                  int64_t rows, int W,
                                                  int32_t* keys,
                                                  int32_t* first4) {
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
  if (first4 && e == r * W4) reinterpret_cast<int4*>(first4)[r] = v;
}

template <typename T>
__global__ __launch_bounds__(256) void k_sa_out(const uint32_t* sa, int64_t m,
                                                int64_t n_total, T* out) {
  // four outputs per thread; sa is a 256-byte aligned workspace array
  const int64_t j0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (j0 >= n_total) return;
  uint32_t v[4];
  if (j0 + 4 <= m) {
    const uint4 q = *reinterpret_cast<const uint4*>(sa + j0);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u)
      v[u] = j0 + u < m ? sa[j0 + u] : (uint32_t)(j0 + u);
  }
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (j0 + u < n_total) out[j0 + u] = (T)v[u];
}

static int bits_for(uint64_t maxval) {
  int b = 0;
  while (b < 64 && (maxval >> b) != 0) ++b;
  return b;
}

static int passes_of(int nbits) {
  return (nbits + kDigitBits - 1) / kDigitBits;
}

// Key bits of a doubling round's radix part: q * (m + 1) + k2 with the
// group ordinal q < big_groups_max(m), k2 <= m.
static int round_bits(int64_t m) {
  return bits_for((uint64_t)(big_groups_max(m) - 1) * (uint64_t)(m + 1) +
                  (uint64_t)m);
}

// Low bits of the token round's keys that hold the position (0: the
// round keeps separate value and position arrays): the 36-bit token key
// sits above them when both fit 64 bits.
static int token_round_vb(int64_t m) {
  const int vb = bits_for((uint64_t)(m > 1 ? m - 1 : 1));
  return 2 * kPairBits + vb <= 64 ? vb : 0;
}

// LSD radix sort of round r's list (written to keyA / valA) by the low
// `nbits` bits of its keys (above the vb value bits of the token round's
// packed keys), then the group heads of the sorted order.
static int sort_and_rank(SaWs& w, int64_t nb, int64_t m, int round,
                         const int32_t* text, hipStream_t stream) {
  const int vb = round == 0 ? token_round_vb(m) : 0;
  const int nbits = round == 0 ? 2 * kPairBits : round_bits(m);
  uint64_t* keys[2] = {w.keyA, w.keyB};
  uint32_t* vals[2] = {w.valA, w.valB};
  int x = 0;
  for (int sh = vb; sh < vb + nbits; sh += kDigitBits) {
    // (the token round's first counts come from k_sa_init)
    if (round > 0 || sh > vb)
      hipLaunchKernelGGL(k_rs_hist<kRsThreads>, dim3((unsigned)nb),
                         dim3(kRsThreads), 0, stream, keys[x], sh, w.hist, nb,
                         w.state, round);
    hipLaunchKernelGGL(k_rs_rowscan<kRsThreads>, dim3(kScanBlocks),
                       dim3(kRsThreads), 0, stream, w.hist, nb, w.rowsum,
                       w.state, round);
    // (the token round's first pass keys the text itself)
    if (vb && sh == vb)
      hipLaunchKernelGGL((k_rs_scatter<kRsThreads, false, true>),
                         dim3((unsigned)nb), dim3(kRsThreads), 0, stream,
                         nullptr, nullptr, keys[x ^ 1], nullptr, sh, w.hist,
                         nb, w.rowsum, w.state, round, text);
    else if (vb)
      hipLaunchKernelGGL((k_rs_scatter<kRsThreads, false>),
                         dim3((unsigned)nb), dim3(kRsThreads), 0, stream,
                         keys[x], nullptr, keys[x ^ 1], nullptr, sh, w.hist,
                         nb, w.rowsum, w.state, round, nullptr);
    else
      hipLaunchKernelGGL(k_rs_scatter<kRsThreads>, dim3((unsigned)nb),
                         dim3(kRsThreads), 0, stream, keys[x], vals[x],
                         keys[x ^ 1], vals[x ^ 1], sh, w.hist, nb, w.rowsum,
                         w.state, round, nullptr);
    x ^= 1;
  }
  const int nx = (round + 1) & 1;
  hipLaunchKernelGGL(k_grp_reduce<kRsThreads>, dim3((unsigned)nb),
                     dim3(kRsThreads), 0, stream, keys[x], w.pos, vb,
                     w.blkmax, w.state, round);
  hipLaunchKernelGGL(k_grp_rank<kRsThreads>, dim3((unsigned)nb),
                     dim3(kRsThreads), 0, stream, keys[x], vals[x], w.pos,
                     vb, w.blkmax, w.rank[nx], w.sa, w.gp, w.gsz, w.skip[nx],
                     w.tmax[nx], w.state, round);
  return (int)hipGetLastError();
}

// Doubling round r >= 1: the local launch (groups of at most kCap; it
// also finishes the build or stalls it), then, when `global_path`, the
// radix launches for the groups above kCap.
static int doubling_round(SaWs& w, int64_t nb, int64_t m, int round,
                          int global_path, int expect_done,
                          hipStream_t stream) {
  const int cur = round & 1, nx = (round + 1) & 1;
  const int64_t nl = (m + kPosTile - 1) / kPosTile;
  // A round enqueued with its radix part has groups above the cap, and
  // groups of up to the cap beside them: its tiles go largest group first.
  // (In rounds of small groups only the order cost more than it saved:
  // 45-60 us rounds went 15-20 us slower on the template corpus.)
  if (global_path)
    hipLaunchKernelGGL(k_sa_order<1024>, dim3(1), dim3(1024), 0, stream,
                       w.tmax[cur], w.tmax[nx], w.order, nl, w.state);
  if (expect_done)
    hipLaunchKernelGGL((k_sa_local<kSaLocalThreads, true>),
                       dim3((unsigned)nl), dim3(kSaLocalThreads), 0, stream,
                       w.gp, w.gsz, w.sa, w.rank[cur], w.rank[nx],
                       w.skip[cur], w.skip[nx],
                       global_path ? w.order : nullptr, m, nl, round,
                       global_path, w.state);
  else
    hipLaunchKernelGGL((k_sa_local<kSaLocalThreads, false>),
                       dim3((unsigned)nl), dim3(kSaLocalThreads), 0, stream,
                       w.gp, w.gsz, w.sa, w.rank[cur], w.rank[nx],
                       w.skip[cur], w.skip[nx],
                       global_path ? w.order : nullptr, m, nl, round,
                       global_path, w.state);
  if (!global_path) return (int)hipGetLastError();
  // (blkmax holds the head counts until the group-head pass needs it)
  hipLaunchKernelGGL(k_pos_count<kRsThreads>, dim3((unsigned)nb),
                     dim3(kRsThreads), 0, stream, w.gp, w.gsz, w.tcnt,
                     w.blkmax, m, w.state, round);
  hipLaunchKernelGGL(k_pos_gather<kRsThreads>, dim3((unsigned)nb),
                     dim3(kRsThreads), 0, stream, w.gp, w.gsz, w.sa,
                     w.rank[cur], w.tcnt, w.blkmax, m, nb, round, w.keyA,
                     w.valA, w.pos, w.state);
  return sort_and_rank(w, nb, m, round, nullptr, stream);
}

// ---------------------------------------------------------- delta index
// The delta's positions grouped by a hash bucket of their token, ascending
// within a bucket, and each bucket's first index: a decode step's delta
// workgroup then visits only the positions whose token hashes like the
// newest pattern token's instead of scanning the whole delta.  The
// grouping is a stable LSD radix sort of (bucket, position) in two 9-bit
// passes with the launches above (a stand-in state block: one list of all
// D positions, round 0); positions at or past the live length take the
// key `buckets`, after every real bucket.

static_assert(2 * kDigitBits >= kDeltaBucketBitsMax + 1,
              "two radix passes cover a bucket key");

struct DixWs {
  uint64_t* keyA;    // [D] bucket keys; sorted after the second pass
  uint64_t* keyB;    // [D]
  uint32_t* pos;     // [D] positions; sorted after the second pass
  uint32_t* valB;    // [D]
  uint32_t* hist;    // [NB][512]
  uint32_t* rowsum;  // [512]
  uint32_t* state;   // [kStateWords]
};

static size_t dix_ws_layout(int64_t D, void* base, DixWs* w) {
  const size_t N = (size_t)(D > 0 ? D : 1);
  const size_t NB = (N + kTile - 1) / kTile;
  size_t off = 0;
  char* c = (char*)base;
  auto take = [&](size_t bytes) -> void* {
    void* ptr = c ? (void*)(c + off) : nullptr;
    off += ws_align(bytes);
    return ptr;
  };
  DixWs s;
  s.keyA = (uint64_t*)take(N * 8);
  s.keyB = (uint64_t*)take(N * 8);
  s.pos = (uint32_t*)take(N * 4);
  s.valB = (uint32_t*)take(N * 4);
  s.hist = (uint32_t*)take((size_t)kRadix * NB * 4);
  s.rowsum = (uint32_t*)take(kRadix * 4);
  s.state = (uint32_t*)take(kStateWords * 4);
  if (w) *w = s;
  return off;
}

__global__ __launch_bounds__(256) void k_dix_init(
    const int32_t* __restrict__ delta, const int64_t* __restrict__ delta_len,
    int64_t D, int hbits, uint64_t* key, uint32_t* pos, uint32_t* state) {
  int64_t dl = *delta_len;
  dl = dl < 0 ? 0 : (dl > D ? D : dl);
  const uint32_t past = 1u << hbits;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < D;
       p += stride) {
    key[p] = p < dl ? delta_bucket(delta[p], hbits) : past;
    pos[p] = (uint32_t)p;
  }
  if (blockIdx.x == 0 && threadIdx.x < kStateWords)
    state[threadIdx.x] = threadIdx.x == kLen ? (uint32_t)D : 0u;
}

// Entry j of the index: its position q and the tokens x(q), x(q - 1),
// x(q - 2) (-1 before position 0), so a row's first test of an entry
// needs no load that depends on the position.
__global__ __launch_bounds__(256) void k_dix_entries(
    const uint32_t* __restrict__ pos, const int32_t* __restrict__ delta,
    int64_t D, int4* ent) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < D;
       j += stride) {
    const int64_t q = pos[j];
    ent[j] = make_int4((int32_t)q, delta[q], q >= 1 ? delta[q - 1] : -1,
                       q >= 2 ? delta[q - 2] : -1);
  }
}

// start[b] = the first sorted index whose key is at least b, b = 0 .. H.
__global__ __launch_bounds__(256) void k_dix_start(
    const uint64_t* __restrict__ key, int64_t D, int hbits,
    uint32_t* start) {
  const int64_t H = (int64_t)1 << hbits;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b <= H;
       b += stride) {
    int64_t lo = 0, hi = D;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (key[mid] < (uint64_t)b)
        lo = mid + 1;
      else
        hi = mid;
    }
    start[b] = (uint32_t)lo;
  }
}

}  // namespace sfx

using namespace sfx;

extern "C" int sfx_sa_keys(const int32_t* corpus, const int32_t* sa,
                           int64_t n, int64_t rows, int64_t width,
                           int32_t* keys, int32_t* first4,
                           hipStream_t stream) {
  if (n < 0 || rows < 0 || rows > n || n > 0x7fffffffLL || width < 4 ||
      width > 32 || (width & 3) || (((uintptr_t)first4) & 15))
    return SFX_EINVAL;
  if (rows == 0) return 0;
  if (!corpus || !sa || !keys) return SFX_EINVAL;
  const int64_t total = rows * width;
  if ((((uintptr_t)keys) & 15) == 0) {
    const int64_t total4 = total / 4;
    hipLaunchKernelGGL(k_rank_keys4, dim3((unsigned)((total4 + 255) / 256)),
                       dim3(256), 0, stream, corpus, sa, n, rows, (int)width,
                       keys, first4);
  } else {
    hipLaunchKernelGGL(k_rank_keys, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, stream, corpus, sa, n, rows, (int)width,
                       keys, first4);
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
  const unsigned out_blocks = (unsigned)((n_total + 1023) / 1024);
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
  const unsigned eb = (unsigned)((m + kInitThreads * kInitItems - 1) /
                                 (kInitThreads * kInitItems));
  // per-block token ranges in the per-tile arrays, unused until round 1
  const int64_t rb = (m + kRangeThreads * 8 - 1) / (kRangeThreads * 8);
  const int parts = (int)(rb < kInitParts ? rb : kInitParts);
  int32_t* plo = reinterpret_cast<int32_t*>(w.tcnt);
  int32_t* phi = reinterpret_cast<int32_t*>(w.blkmax);
  hipLaunchKernelGGL(k_sa_range, dim3((unsigned)parts), dim3(kRangeThreads),
                     0, stream, text, m, plo, phi);
  hipLaunchKernelGGL(k_sa_init, dim3(eb), dim3(kInitThreads), 0, stream, text,
                     m, w.keyA, w.valA, w.pos, token_round_vb(m), plo, phi,
                     parts, w.skip[0], w.skip[1], w.tmax[0], w.tmax[1],
                     (m + kPosTile - 1) / kPosTile, w.hist, nb, w.state);
  return sort_and_rank(w, nb, m, 0, text, stream);
}

// Rounds first .. first + count - 1 (round r doubles h = h0 * 2^(r-1),
// h0 = 1 or 2 as round 0 decided; with h0 = 2 the last round finds none).
// flags: SFX_SA_ROUNDS_RADIX enqueues the radix launches,
// SFX_SA_ROUNDS_EXPECT_FINAL has the local launches read the state first.
int build_rounds(int64_t m, int first, int count, int flags,
                 void* workspace, hipStream_t stream) {
  if (m <= 1) return 0;
  SaWs w;
  sa_ws_layout(m, workspace, &w);
  const int64_t nb = (m + kTile - 1) / kTile;
  const int last = total_rounds(m);
  const int global_path = (flags & SFX_SA_ROUNDS_RADIX) ? 1 : 0;
  const int expect_done = (flags & SFX_SA_ROUNDS_EXPECT_FINAL) ? 1 : 0;
  for (int r = first < 1 ? 1 : first; r < first + count && r <= last; ++r) {
    const int rc =
        doubling_round(w, nb, m, r, global_path, expect_done, stream);
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
  rc = build_rounds(m, 1, total_rounds(m), SFX_SA_ROUNDS_RADIX, workspace,
                    stream);
  if (rc) return rc;
  return build_finish(m, n_total, sa_out, sa_is64, workspace, stream);
}

extern "C" int sfx_sa_group_cap(void) { return kCap; }

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
                                   int32_t flags, void* workspace,
                                   size_t workspace_bytes,
                                   hipStream_t stream) {
  if (m < 0 || m > 0x7fffffffLL || first < 1 || count < 0) return SFX_EINVAL;
  if (!ws_ok(m, workspace, workspace_bytes)) return SFX_EINVAL;
  if (flags & ~(SFX_SA_ROUNDS_RADIX | SFX_SA_ROUNDS_EXPECT_FINAL))
    return SFX_EINVAL;
  return build_rounds(m, first, count, flags, workspace, stream);
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

extern "C" size_t sfx_delta_index_bytes(int64_t delta_capacity) {
  if (delta_capacity < 1 || delta_capacity > (1ll << 30)) return 0;
  return dix_ws_layout(delta_capacity, nullptr, nullptr);
}

extern "C" int sfx_delta_index_build(const int32_t* delta,
                                     const int64_t* delta_len,
                                     int64_t delta_capacity, int32_t* entries,
                                     uint32_t* start, int64_t buckets,
                                     void* workspace, size_t workspace_bytes,
                                     hipStream_t stream) {
  const int64_t D = delta_capacity;
  if (!delta || !delta_len || !entries || !start || !workspace)
    return SFX_EINVAL;
  if ((uintptr_t)entries & 15) return SFX_EINVAL;
  if (D < 1 || D > (1ll << 30)) return SFX_EINVAL;
  if (buckets < (1ll << kDeltaBucketBitsMin) ||
      buckets > (1ll << kDeltaBucketBitsMax) || (buckets & (buckets - 1)))
    return SFX_EINVAL;
  if (((uintptr_t)workspace & 255) ||
      workspace_bytes < dix_ws_layout(D, nullptr, nullptr))
    return SFX_EINVAL;
  const int hbits = __builtin_ctzll((unsigned long long)buckets);
  DixWs w;
  dix_ws_layout(D, workspace, &w);
  const int64_t nb = (D + kTile - 1) / kTile;
  const unsigned gb = (unsigned)((D + 255) / 256 < 2048 ? (D + 255) / 256
                                                         : 2048);
  hipLaunchKernelGGL(k_dix_init, dim3(gb), dim3(256), 0, stream, delta,
                     delta_len, D, hbits, w.keyA, w.pos, w.state);
  uint64_t* keys[2] = {w.keyA, w.keyB};
  uint32_t* vals[2] = {w.pos, w.valB};
  int x = 0;
  for (int sh = 0; sh <= hbits; sh += kDigitBits) {
    hipLaunchKernelGGL(k_rs_hist<kRsThreads>, dim3((unsigned)nb),
                       dim3(kRsThreads), 0, stream, keys[x], sh, w.hist, nb,
                       w.state, 0);
    hipLaunchKernelGGL(k_rs_rowscan<kRsThreads>, dim3(kScanBlocks),
                       dim3(kRsThreads), 0, stream, w.hist, nb, w.rowsum,
                       w.state, 0);
    hipLaunchKernelGGL(k_rs_scatter<kRsThreads>, dim3((unsigned)nb),
                       dim3(kRsThreads), 0, stream, keys[x], vals[x],
                       keys[x ^ 1], vals[x ^ 1], sh, w.hist, nb, w.rowsum,
                       w.state, 0, nullptr);
    x ^= 1;
  }
  // two passes (keys of at most 18 bits): the sorted data is back in
  // keyA and pos
  hipLaunchKernelGGL(k_dix_entries, dim3(gb), dim3(256), 0, stream, w.pos,
                     delta, D, reinterpret_cast<int4*>(entries));
  const int64_t H = buckets;
  const unsigned sb = (unsigned)((H + 256) / 256);
  hipLaunchKernelGGL(k_dix_start, dim3(sb), dim3(256), 0, stream, w.keyA, D,
                     hbits, start);
  return (int)hipGetLastError();
}
