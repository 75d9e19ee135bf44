// Final local-vs-global selection of one row (suffix_gpu/proposer.py:
// 305-327): the global winner replaces the local one only on a strictly
// greater score; the chain is padded with -1 past the emission count.
#pragma once

#include "sfx_common.h"
#include "step_ws.h"

namespace sfx {

// Executed by the whole block of whichever of row b's SA, last delta and
// local workgroups arrives last.  Global candidate per cap: SA when its
// length is at least the delta's, else the delta (global_index.py:
// 321-325); a cap repeating the previous cap's (length, source) is dropped
// (:329-337); the global winner is the first argmax of the raw score
// (proposer.py:308-314) and replaces the local one only on a strictly
// greater score; the chain is padded with -1 past the emission count
// (:322-327).  misc: 3 ints of LDS.
__device__ __forceinline__ void final_pick(const sfx_params& p,
                                           const StepWs& ws, int b,
                                           int32_t* draft, int32_t* num_valid,
                                           int* misc) {
  const int C = p.num_caps;
  const int K = p.k;
  SFX_TRACE_POINT(13);
  if (threadIdx.x < kWave) {
    // Lane c holds cap c's global candidate; every load is issued at once.
    const int c = threadIdx.x;
    const bool on = c < C;
    const int64_t i = (int64_t)b * C + (on ? c : 0);
    int sl = 0, dl = 0, snv = 0, dnv = 0;
    float ssc = 0.0f, dsc = 0.0f;
    // (ws_load: the handover into this pick does not invalidate caches)
    if (on) {
      sl = ws_load(ws.sa_len + i);
      dl = ws_load(ws.dl_c + i);
      ssc = ws_load(ws.sa_score + i);
      dsc = ws_load(ws.dn_score + i);
      snv = ws_load(ws.sa_nv + i);
      dnv = ws_load(ws.dn_nv + i);
    }
    const float lscore = ws_load(ws.l_score + b);
    const int lemit = ws_load(ws.l_emit + b);
    // the SA lengths published for the delta workgroups: every producer
    // has arrived, so none reads them again this step
    if (on) ws.sa_known[(int64_t)b * SFX_MAX_CANDIDATES + c] = 0;
    const bool use_sa = sl >= dl && sl > 0;
    const bool use_d = dl > sl && dl > 0;
    const int len = use_sa ? sl : (use_d ? dl : 0);
    const int src = (use_sa ? 1 : 0) + (use_d ? 2 : 0);
    const int plen = __shfl_up(len, 1);
    const int psrc = __shfl_up(src, 1);
    const bool dup = c > 0 && len == plen && src == psrc && len > 0;
    const int esrc = dup ? 0 : src;
    const int elen = dup ? 0 : len;
    const float sc = esrc == 1 ? ssc : (esrc == 2 ? dsc : 0.0f);
    const int nv = esrc == 1 ? snv : (esrc == 2 ? dnv : 0);
    // First argmax: scores are sums of probabilities (>= 0), so their bit
    // patterns order like the values; lanes past C (0) lose every tie to
    // a lower cap.
    const uint32_t key = on ? __float_as_uint(sc) : 0u;
    const uint32_t top = wave_all_max(key);
    const int best = __builtin_amdgcn_readfirstlane(
        __builtin_ctzll(ballot(on && key == top)));
    const float bscore = __uint_as_float(
        (uint32_t)__builtin_amdgcn_readlane((int)key, best));
    const int bnv = __builtin_amdgcn_readlane(nv, best);
    const int blen = __builtin_amdgcn_readlane(elen, best);
    const int bsrc = __builtin_amdgcn_readlane(esrc, best);
    if (c == 0) {
      const int64_t cap = spec_cap(p, blen);
      const int64_t cap0 = cap > 0 ? cap : 0;
      const int gemit = (int)((int64_t)bnv < cap0 ? bnv : cap0);
      const bool g = bscore > lscore;
      misc[0] = g ? gemit : lemit;
      misc[1] = g ? bsrc : 0;
      misc[2] = best;
    }
  }
  __syncthreads();
  const int nv = misc[0];
  const int which = misc[1];
  const int64_t i = (int64_t)b * C + misc[2];
  const int32_t* chain = which == 0   ? ws.l_chain + (int64_t)b * K
                         : which == 1 ? ws.sa_chain + i * K
                                      : ws.dn_chain + i * K;
  for (int j = threadIdx.x; j < K; j += blockDim.x)
    draft[(int64_t)b * K + j] = j < nv ? ws_load(chain + j) : -1;
  if (threadIdx.x == 0) num_valid[b] = nv;
  SFX_TRACE_POINT(14);
}

// Row state of a decode step: committed count q after the update and
// whether the row drafts (proposer.py:203-212, or the caller's mask).
struct RowState {
  int64_t base;  // count before the update
  int64_t cnt;   // accepted count (0 without an update)
  int64_t q;     // count after the update
  bool mask;
};

// Called by every lane of the wave (the accepted count is a ballot over
// the row's sampled ids, one id per lane).
__device__ __forceinline__ RowState row_state(const sfx_batch& bt, int b) {
  RowState st;
  st.base = load_count(bt.num_tokens, bt.num_tokens_is64, b);
  st.cnt = 0;
  if (bt.sampled) {
    if (bt.valid_count) {
      st.cnt = load_count(bt.valid_count, bt.valid_count_is64, b);
    } else {
      const int32_t* sp = bt.sampled + (int64_t)b * bt.num_sampled;
      for (int64_t j0 = 0; j0 < bt.num_sampled; j0 += kWave) {
        const int64_t j = j0 + lane_id();
        st.cnt += popc(ballot(j < bt.num_sampled && sp[j] != -1));
      }
    }
    st.q = st.base + st.cnt;
    st.mask = st.cnt > 0 && st.q < bt.limit;
  } else {
    st.q = st.base;
    st.mask = bt.mask ? bt.mask[b] != 0 : true;
  }
  return st;
}

// Token at position x (0 <= x < S) of row b as it reads after this step's
// scatter, without depending on the scatter having been written: the
// sampled id when the update writes x, else the resident token.
__device__ __forceinline__ int32_t updated_token(const sfx_batch& bt, int b,
                                                 const RowState& st,
                                                 int64_t x) {
  if (bt.sampled) {
    const int64_t j = x - st.base;
    if (j >= 0 && j < st.cnt && j < bt.num_sampled) {
      const int32_t v = bt.sampled[(int64_t)b * bt.num_sampled + j];
      if (v != -1) return v;
    }
  }
  return bt.tokens[(int64_t)b * bt.seq + x];
}

}  // namespace sfx
