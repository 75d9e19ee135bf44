// Local (per-request) suffix matcher: one 512-thread workgroup per row
// (1024 threads for the local-only decode step).
//
// The row is staged once in LDS (coalesced int4 loads), the step's sampled
// tokens are scattered into LDS and HBM, and everything else runs out of
// LDS: the newest-first pattern, match_back (leading-match count of the
// tokens ending at i against the pattern, early exit per position, kept as
// u8), a 33-bin histogram whose suffix sums give every support threshold's
// candidate length, the ordered ballot/mbcnt compaction of the first R
// occurrence ends per candidate, and one wave per candidate running the
// majority-vote expansion straight off the LDS row.  Rows too long for
// LDS stay in HBM and are streamed through it in chunks instead.
//
// Follows suffix_gpu/local_matcher.py:83-263 and proposer.py:135-184,
// 322-327.

#include "launch.h"
#include "local_impl.h"

namespace sfx {

static_assert(kLocalThreads == kLocalThreadsDefault,
              "launch.h's default thread count");

template <bool kStream>
__global__ __launch_bounds__(kLocalThreads) void k_local(LocalArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  local_body<kStream>(a, smem, blockIdx.x);
}

template <bool kStream>
__global__ __launch_bounds__(kWideThreads) void k_local_wide(LocalArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  local_body<kStream, kWideThreads>(a, smem, blockIdx.x);
}

static size_t layout_bytes(const sfx_params& p, int64_t S, int chunk,
                           int nthreads, int mb_full) {
  if ((chunk == 0 || mb_full) && S > (int64_t)kMaxLds) return (size_t)-1;
  if (chunk == 0 && S > (int64_t)kMaxLds / 4) return (size_t)-1;
  const LocalLayout L =
      local_layout((int)S, p.max_pattern_len, p.num_thresholds,
                   p.max_occurrences, p.k, nthreads / kWave, chunk, mb_full);
  return (size_t)L.total;
}

// A streamed row keeps its whole match array in LDS where some chunk
// length allows it (one staging pass instead of two).
int local_chunk(const sfx_params& p, int64_t S, size_t cap, int nthreads,
                int* mb_full) {
  if (mb_full) *mb_full = 0;
  if (layout_bytes(p, S, 0, nthreads, 0) <= cap) return 0;
  for (int chunk = kMaxStreamChunk; chunk >= kMinStreamChunk; chunk /= 2)
    if (layout_bytes(p, S, chunk, nthreads, 1) <= cap) {
      if (mb_full) *mb_full = 1;
      return chunk;
    }
  for (int chunk = kMaxStreamChunk; chunk >= kMinStreamChunk; chunk /= 2)
    if (layout_bytes(p, S, chunk, nthreads, 0) <= cap) return chunk;
  return -1;
}

size_t local_lds_bytes(const sfx_params& p, int64_t S, int chunk,
                       int nthreads, int mb_full) {
  return chunk < 0 ? (size_t)-1
                   : layout_bytes(p, S, chunk, nthreads, mb_full);
}

int launch_local_step(LocalArgs a, hipStream_t stream) {
  a.chunk = local_chunk(a.p, a.bt.seq, kMaxLds, kWideThreads, &a.mb_full);
  if (a.chunk < 0) return -1;
  if (a.bt.batch == 0) return 0;
  const size_t lds =
      local_lds_bytes(a.p, a.bt.seq, a.chunk, kWideThreads, a.mb_full);
  if (a.chunk == 0) {
    static std::atomic<uint64_t> lds_opt{0};
    allow_max_lds((const void*)k_local_wide<false>, lds_opt);
    hipLaunchKernelGGL(k_local_wide<false>, dim3((unsigned)a.bt.batch),
                       dim3(kWideThreads), lds, stream, a);
  } else {
    static std::atomic<uint64_t> lds_opt{0};
    allow_max_lds((const void*)k_local_wide<true>, lds_opt);
    hipLaunchKernelGGL(k_local_wide<true>, dim3((unsigned)a.bt.batch),
                       dim3(kWideThreads), lds, stream, a);
  }
  return (int)hipGetLastError();
}

int check_local(const sfx_params& p, const sfx_batch& bt) {
  if (bt.batch < 0 || bt.seq < 1 || !bt.tokens || !bt.num_tokens)
    return SFX_EINVAL;
  if (p.k < 1 || p.k > 4096 || p.max_pattern_len < 1 ||
      p.max_pattern_len > 255 || p.max_occurrences < 1 ||
      p.max_occurrences > 2048 || p.num_thresholds < 1 ||
      p.num_thresholds > SFX_MAX_CANDIDATES)
    return SFX_EINVAL;
  if (bt.sampled && bt.num_sampled < 0) return SFX_EINVAL;
  if (bt.seq > kMaxSeq) return SFX_EINVAL;
  if (local_chunk(p, bt.seq) < 0) return SFX_EINVAL;
  return 0;
}

int launch_local(LocalArgs a, hipStream_t stream) {
  if (a.bt.batch == 0) return 0;
  a.chunk = local_chunk(a.p, a.bt.seq, kMaxLds, kLocalThreadsDefault,
                        &a.mb_full);
  const size_t lds = local_lds_bytes(a.p, a.bt.seq, a.chunk,
                                     kLocalThreadsDefault, a.mb_full);
  if (a.chunk == 0) {
    static std::atomic<uint64_t> lds_opt{0};
    allow_max_lds((const void*)k_local<false>, lds_opt);
    hipLaunchKernelGGL(k_local<false>, dim3((unsigned)a.bt.batch),
                       dim3(kLocalThreads), lds, stream, a);
  } else {
    static std::atomic<uint64_t> lds_opt{0};
    allow_max_lds((const void*)k_local<true>, lds_opt);
    hipLaunchKernelGGL(k_local<true>, dim3((unsigned)a.bt.batch),
                       dim3(kLocalThreads), lds, stream, a);
  }
  return (int)hipGetLastError();
}

}  // namespace sfx

using namespace sfx;

extern "C" int sfx_local_gather(const sfx_params* p, const sfx_batch* bt,
                                int64_t* cand, int32_t* cont, int64_t* occ,
                                hipStream_t stream) {
  if (!p || !bt) return SFX_EINVAL;
  int rc = check_local(*p, *bt);
  if (rc) return rc;
  LocalArgs a = {};
  a.p = *p;
  a.bt = *bt;
  a.mode = kLocalGather;
  a.cand_out = cand;
  a.cont_out = cont;
  a.occ_out = occ;
  return launch_local(a, stream);
}

extern "C" int sfx_local_forward(const sfx_params* p, const sfx_batch* bt,
                                 int32_t* draft, int32_t* num_valid,
                                 int64_t* match_len, int64_t* occ,
                                 float* score, hipStream_t stream) {
  if (!p || !bt || !draft || !num_valid) return SFX_EINVAL;
  int rc = check_local(*p, *bt);
  if (rc) return rc;
  LocalArgs a = {};
  a.p = *p;
  a.bt = *bt;
  a.mode = kLocalForward;
  a.draft = draft;
  a.num_valid = num_valid;
  a.len_out = match_len;
  a.occ1_out = occ;
  a.score_out = score;
  return launch_local(a, stream);
}
