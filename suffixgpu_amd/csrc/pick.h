// Final local-vs-global selection of one row (suffix_gpu/proposer.py:
// 305-327): the global winner replaces the local one only on a strictly
// greater score; the chain is padded with -1 past the emission count.
#pragma once

#include "sfx_common.h"
#include "step_ws.h"

namespace sfx {

// Executed by the whole block of whichever kernel arrived last for row b.
__device__ __forceinline__ void pick_row(int b, int K, const StepWs& ws,
                                         int32_t* draft, int32_t* num_valid) {
  const float ls = ws.l_score[b];
  const float gs = ws.g_score[b];
  const bool g = gs > ls;
  const int nv = g ? ws.g_emit[b] : ws.l_emit[b];
  const int32_t* chain = g ? ws.g_chain + (int64_t)b * K
                           : ws.l_chain + (int64_t)b * K;
  for (int j = threadIdx.x; j < K; j += blockDim.x)
    draft[(int64_t)b * K + j] = j < nv ? chain[j] : -1;
  if (threadIdx.x == 0) num_valid[b] = nv;
}

// Row state of a decode step: committed count q after the update and
// whether the row drafts (proposer.py:203-212, or the caller's mask).
struct RowState {
  int64_t base;  // count before the update
  int64_t cnt;   // accepted count (0 without an update)
  int64_t q;     // count after the update
  bool mask;
};

__device__ __forceinline__ RowState row_state(const sfx_batch& bt, int b) {
  RowState st;
  st.base = load_count(bt.num_tokens, bt.num_tokens_is64, b);
  st.cnt = 0;
  if (bt.sampled) {
    if (bt.valid_count) {
      st.cnt = load_count(bt.valid_count, bt.valid_count_is64, b);
    } else {
      const int32_t* sp = bt.sampled + (int64_t)b * bt.num_sampled;
      for (int64_t j = 0; j < bt.num_sampled; ++j) st.cnt += sp[j] != -1;
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
