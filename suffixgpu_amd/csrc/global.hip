// Global (cross-request) match: SA interval search + delta scan + merge.
//
// Grid: 1 + dparts 512-thread workgroups per query row, interleaved.
//   * SA role: for every length l = 1..min(qlen, P) the suffix of length l
//     of the query is searched by an 8-lane k-ary interval search
//     (sa_search.h); each cap then takes its longest non-empty interval
//     (suffix_gpu/sa_search.py:110-163).
//   * Delta roles: each takes an equal share of the committed delta:
//     match_back with an early-exit compare per position, a block max, and
//     the ordered compaction of its first R ends per cap
//     (global_index.py:465-546).
// Whichever workgroup finishes a row last (atomic handover in the
// workspace) combines the delta parts and merges the two sources per cap
// (global_index.py:311-370): SA vs delta
// choice, adjacent-duplicate zeroing, strided SA sampling, continuation
// gather into LDS, and (decode step / draft) one wave per cap running the
// majority-vote expansion, then the first-argmax cap.  In the decode step
// the row is then handed to the local kernel's result (pick.h).

#include "global_impl.h"
#include "launch.h"

namespace sfx {

__global__ __launch_bounds__(kGlobalThreads) void k_global(GlobalArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int per = 1 + a.dparts;
  global_body(a, smem, (int)(blockIdx.x / per), (int)(blockIdx.x % per));
}


int delta_parts_of(const sfx_index& ix, int64_t batch) {
  return ix.delta_entries ? 1 : delta_parts_for(batch, ix.delta_capacity);
}

int mb_lds_bytes(const sfx_index& ix, int parts) {
  if (ix.delta_entries) return 0;  // the indexed delta role keeps no u8 array
  const int64_t cap = delta_part_cap(ix.delta_capacity, parts);
  if (cap > kMbLdsMax) return 0;
  const int n = (int)cap;
  const int seg = (((n + kGlobalThreads - 1) / kGlobalThreads) + 15) & ~15;
  return seg * kGlobalThreads;
}

int merge_waves_for(const sfx_params& p, const sfx_index& ix, int parts,
                    size_t* lds, size_t cap, int dend_parts) {
  const int NW = kGlobalThreads / kWave;
  const int C = p.num_caps;
  int nmw = C < NW ? C : NW;
  if (nmw < 1) nmw = 1;
  for (; nmw >= 1; --nmw) {
    const GlobalLayout L = global_layout(p.max_pattern_len, C,
                                         p.max_occurrences, p.k, nmw,
                                         mb_lds_bytes(ix, parts), 0,
                                         dend_parts, ix.delta_entries ? 1 : 0);
    if ((size_t)L.total <= cap) {
      *lds = (size_t)L.total;
      return nmw;
    }
  }
  return 0;
}

int delta_chunk_for(const sfx_params& p, const sfx_index& ix, int parts,
                    int nmw, int dend_parts, size_t cap, size_t* lds) {
  const int P = p.max_pattern_len;
  const int halo = (P + 3) & ~3;
  const int mb = mb_lds_bytes(ix, parts);
  const int dindex = ix.delta_entries ? 1 : 0;
  const GlobalLayout L0 = global_layout(P, p.num_caps, p.max_occurrences,
                                        p.k, nmw, mb, kDeltaChunk,
                                        dend_parts, dindex);
  *lds = (size_t)L0.total;
  if (dindex) return kDeltaChunk;  // (no delta staging)
  // the staged words and the match bytes sit after the header
  const int64_t avail = (int64_t)cap - L0.dtok - ((mb + 15) & ~15);
  const int64_t most = (delta_part_cap(ix.delta_capacity, parts) + 255) &
                       ~(int64_t)255;
  int64_t ch = (avail / 4 - halo) & ~(int64_t)255;
  ch = ch < most ? ch : most;
  if (ch <= kDeltaChunk) return kDeltaChunk;
  const GlobalLayout L = global_layout(P, p.num_caps, p.max_occurrences, p.k,
                                       nmw, mb, (int)ch, dend_parts);
  if ((size_t)L.total > cap) return kDeltaChunk;
  *lds = (size_t)L.total;
  return (int)ch;
}

int check_global(const sfx_params& p, const sfx_index& ix, int64_t batch) {
  if (p.num_caps < 1 || p.num_caps > SFX_MAX_CANDIDATES) return SFX_EINVAL;
  if (p.k < 1 || p.k > 4096 || p.max_pattern_len < 1 ||
      p.max_pattern_len > 255 || p.max_occurrences < 1 ||
      p.max_occurrences > 2048)
    return SFX_EINVAL;
  if (!ix.corpus || !ix.sa || !ix.delta || !ix.delta_len) return SFX_EINVAL;
  if (ix.capacity < 1 || ix.capacity > 0x7fffffffLL) return SFX_EINVAL;
  if (ix.delta_capacity < 1 || ix.delta_capacity > 0x7fffffffLL)
    return SFX_EINVAL;
  if (ix.sa_key &&
      (ix.key_width < 4 || ix.key_width > 32 || (ix.key_width & 3) ||
       ((uintptr_t)ix.sa_key & 15)))
    return SFX_EINVAL;
  // A selector needs the first key buffer; the second (NULL: none while
  // the selector is set) follows the same alignment rule.
  if (ix.key_select && (!ix.sa_key || ((uintptr_t)ix.sa_key_alt & 15)))
    return SFX_EINVAL;
  // n-gram tables: a power-of-two slot count of at least one bucket,
  // 256-byte aligned tables, the second one only with a selector
  if ((ix.gram || ix.gram_alt) &&
      (ix.gram_slots < kGramBucket || ix.gram_slots % kGramBucket ||
       ix.gram_slots > (1ll << 31) || ((uintptr_t)ix.gram & 255) ||
       ((uintptr_t)ix.gram_alt & 255) || (ix.gram_alt && !ix.key_select)))
    return SFX_EINVAL;
  // the delta token index: both arrays and a bucket count of 2^10 .. 2^17
  if ((ix.delta_entries || ix.delta_start) &&
      (!ix.delta_entries || !ix.delta_start ||
       ix.delta_buckets < (1ll << kDeltaBucketBitsMin) ||
       ix.delta_buckets > (1ll << kDeltaBucketBitsMax) ||
       (ix.delta_buckets & (ix.delta_buckets - 1)) ||
       ((uintptr_t)ix.delta_entries & 15)))
    return SFX_EINVAL;
  size_t lds = 0;
  const int parts = delta_parts_of(ix, batch);
  if (merge_waves_for(p, ix, parts, &lds) < 1) return SFX_EINVAL;
  return 0;
}

static int launch_global(GlobalArgs& a, hipStream_t stream) {
  if (a.B == 0) return 0;
  size_t lds = 0;
  a.dparts = delta_parts_of(a.ix, a.B);
  a.merge_waves = merge_waves_for(a.p, a.ix, a.dparts, &lds);
  a.mb_lds = mb_lds_bytes(a.ix, a.dparts);
  a.dchunk = delta_chunk_for(a.p, a.ix, a.dparts, a.merge_waves, 0,
                             kMaxLds, &lds);
  static std::atomic<uint64_t> lds_opt{0};
  allow_max_lds((const void*)k_global, lds_opt);
  const unsigned blocks = (unsigned)((1 + a.dparts) * a.B);
  lds = one_per_cu_lds(lds, blocks);
  hipLaunchKernelGGL(k_global, dim3(blocks), dim3(kGlobalThreads), lds,
                     stream, a);
  return (int)hipGetLastError();
}

}  // namespace sfx

using namespace sfx;

extern "C" size_t sfx_global_query_workspace_size(const sfx_params* p,
                                                  int64_t batch,
                                                  int64_t delta_capacity) {
  if (!p || batch < 0) return 0;
  return step_ws_layout(*p, batch, delta_capacity, nullptr, nullptr);
}

extern "C" int sfx_global_query(const sfx_params* p, const sfx_index* ix,
                                const int32_t* query, int64_t batch,
                                int64_t width, const int64_t* qlen,
                                const sfx_global_out* out, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
  if (!p || !ix || !out || batch < 0) return SFX_EINVAL;
  int rc = check_global(*p, *ix, batch);
  if (rc) return rc;
  if (batch > 0 && (!query || !qlen || width < 1)) return SFX_EINVAL;
  const size_t need =
      step_ws_layout(*p, batch, ix->delta_capacity, nullptr, nullptr);
  if (!workspace || workspace_bytes < need) return SFX_EINVAL;
  GlobalArgs a = {};
  a.p = *p;
  a.ix = *ix;
  a.B = batch;
  a.step = 0;
  a.query = query;
  a.qwidth = width;
  a.qlen = qlen;
  a.out = *out;
  a.need_expand = (out->draft || out->emit || out->draft_len ||
                   out->draft_occ || out->draft_score)
                      ? 1
                      : 0;
  step_ws_layout(*p, batch, ix->delta_capacity, workspace, &a.ws);
  return launch_global(a, stream);
}
