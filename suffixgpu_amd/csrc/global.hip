// Global (cross-request) match: SA interval search + delta scan + merge.
//
// Grid: two 512-thread workgroups per query row, interleaved.
//   * SA role: for every length l = 1..min(qlen, P) the suffix of length l
//     of the query is searched by an 8-lane k-ary interval search
//     (sa_search.h); each cap then takes its longest non-empty interval
//     (suffix_gpu/sa_search.py:110-163).
//   * Delta role: match_back over the committed delta with an early-exit
//     compare per position, a block max, and the ordered compaction of the
//     first R ends per cap (global_index.py:465-546).
// Whichever role finishes a row second (atomic handover in the workspace)
// merges the two sources per cap (global_index.py:311-370): SA vs delta
// choice, adjacent-duplicate zeroing, strided SA sampling, continuation
// gather into LDS, and (decode step / draft) one wave per cap running the
// majority-vote expansion, then the first-argmax cap.  In the decode step
// the row is then handed to the local kernel's result (pick.h).

#include "launch.h"
#include "pick.h"
#include "sa_search.h"
#include "sfx_common.h"
#include "step_ws.h"

namespace sfx {

constexpr int kGlobalThreads = 512;
constexpr int kSearchGroup = 8;

struct GlobalArgs {
  sfx_params p;
  sfx_index ix;
  int64_t B;
  int step;
  sfx_batch bt;
  const int32_t* query;
  int64_t qwidth;
  const int64_t* qlen;
  sfx_global_out out;
  int need_expand;
  int32_t* draft;
  int32_t* num_valid;
  StepWs ws;
  int merge_waves;
};

struct GlobalLayout {
  int rpat, lb, ub, found, wcnt, wpre, red, misc, mpos, mcache, mA, chain,
      nv, score, rlen, rocc, total;
};

__host__ __device__ inline int g_take(int& off, int bytes) {
  const int o = off;
  off += (bytes + 15) & ~15;
  return o;
}

__host__ __device__ inline GlobalLayout global_layout(int P, int C, int R,
                                                      int K, int nmw) {
  constexpr int NW = kGlobalThreads / kWave;
  const int Rp = (R + 3) & ~3;
  GlobalLayout L;
  int off = 0;
  L.rpat = g_take(off, P * 4);
  L.lb = g_take(off, P * 8);
  L.ub = g_take(off, P * 8);
  L.found = g_take(off, C * 4);
  L.wcnt = g_take(off, NW * C * 4);
  L.wpre = g_take(off, NW * C * 4);
  L.red = g_take(off, NW * 4);
  L.misc = g_take(off, 64);
  L.mpos = g_take(off, nmw * Rp * 4);
  L.mcache = g_take(off, nmw * R * K * 4);
  L.mA = g_take(off, nmw * Rp * 4);
  L.chain = g_take(off, C * K * 4);
  L.nv = g_take(off, C * 4);
  L.score = g_take(off, C * 4);
  L.rlen = g_take(off, C * 4);
  L.rocc = g_take(off, C * 4);
  L.total = off;
  return L;
}

// Leading-match count of delta tokens ending at i (exclusive) against the
// newest-first pattern; x(j < 0) = -1 (global_index.py:503-515).
__device__ __forceinline__ int delta_mb(const int32_t* __restrict__ delta,
                                        const int32_t* rpat, int P,
                                        int64_t i) {
  int m = 0;
  for (int t = 0; t < P; ++t) {
    const int64_t j = i - 1 - t;
    const int32_t x = j >= 0 ? delta[j] : -1;
    if (x != rpat[t]) break;
    ++m;
  }
  return m;
}

__global__ __launch_bounds__(kGlobalThreads) void k_global(GlobalArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NT = kGlobalThreads;
  constexpr int NW = NT / kWave;
  const sfx_params& p = a.p;
  const int b = (int)(blockIdx.x >> 1);
  const bool sa_role = (blockIdx.x & 1) == 0;
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int ln = tid % kWave;
  const int P = p.max_pattern_len;
  const int C = p.num_caps;
  const int R = p.max_occurrences;
  const int K = p.k;
  const int Rp = (R + 3) & ~3;
  const GlobalLayout L = global_layout(P, C, R, K, a.merge_waves);
  int32_t* rpat = (int32_t*)(smem + L.rpat);
  int64_t* lbs = (int64_t*)(smem + L.lb);
  int64_t* ubs = (int64_t*)(smem + L.ub);
  int32_t* found = (int32_t*)(smem + L.found);
  int32_t* wcnt = (int32_t*)(smem + L.wcnt);
  int32_t* wpre = (int32_t*)(smem + L.wpre);
  int32_t* red = (int32_t*)(smem + L.red);
  int* misc = (int*)(smem + L.misc);
  const int64_t N = a.ix.capacity;
  const int64_t D = a.ix.delta_capacity;

  // Query tail, newest first: rpat[t] = tail token t back from the end;
  // -3 past the start (global_index.py:493-501).
  int64_t qlen;
  if (a.step) {
    const RowState st = row_state(a.bt, b);
    if (!st.mask) return;  // masked rows: the local kernel writes them
    const int64_t q = st.q;
    qlen = q < P ? q : P;
    for (int t = tid; t < P; t += NT) {
      const int64_t idx = q - 1 - t;
      int32_t v = -3;
      if (idx >= 0) {
        const int64_t x = idx < a.bt.seq - 1 ? idx : a.bt.seq - 1;
        v = updated_token(a.bt, b, st, x);
      }
      rpat[t] = v;
    }
  } else {
    qlen = a.qlen[b];
    const int64_t Q = a.qwidth;
    for (int t = tid; t < P; t += NT) {
      const int64_t idx = qlen - 1 - t;
      int32_t v = -3;
      if (idx >= 0) v = a.query[(int64_t)b * Q + (idx < Q - 1 ? idx : Q - 1)];
      rpat[t] = v;
    }
  }
  const int plen = (int)(qlen < 0 ? 0 : (qlen < P ? qlen : P));
  __syncthreads();

  if (sa_role) {
    // ---- SA interval search for every suffix length of the tail.
    constexpr int G = kSearchGroup;
    const int ngroups = NT / G;
    const int g = tid / G;
    for (int l = g + 1; l <= P; l += ngroups) {
      int64_t lo = 0, hi = 0;
      if (l <= plen) {
        auto pat_at = [&](int j) -> int32_t { return rpat[l - 1 - j]; };
        kary_bounds<G>(a.ix.sa, a.ix.corpus, N, pat_at, l, lo, hi);
      }
      if (tid % G == 0) {
        lbs[l - 1] = lo;
        ubs[l - 1] = hi;
      }
    }
    __syncthreads();
    for (int c = tid; c < C; c += NT) {
      const int cap = p.caps[c];
      int best = 0;
      for (int l = 1; l <= P && l <= cap; ++l)
        if (l <= plen && ubs[l - 1] > lbs[l - 1]) best = l;
      const int64_t s = best ? lbs[best - 1] : 0;
      const int64_t e = best ? ubs[best - 1] : 0;
      a.ws.sa_len[(int64_t)b * C + c] = best;
      a.ws.sa_s[(int64_t)b * C + c] = (int32_t)s;
      a.ws.sa_e[(int64_t)b * C + c] = (int32_t)e;
      if (a.out.sa_len) a.out.sa_len[(int64_t)b * C + c] = best;
      if (a.out.sa_start) a.out.sa_start[(int64_t)b * C + c] = s;
      if (a.out.sa_end) a.out.sa_end[(int64_t)b * C + c] = e;
    }
  } else {
    // ---- Delta scan over ends i in [0, delta_len].
    int64_t dl = *a.ix.delta_len;
    dl = dl < 0 ? 0 : (dl > D ? D : dl);
    int mx = 0;
    for (int64_t i = tid; i <= dl; i += NT)
      mx = max(mx, delta_mb(a.ix.delta, rpat, P, i));
    mx = wave_max_i32(mx);
    if (ln == 0) red[wv] = mx;
    __syncthreads();
    if (tid == 0) {
      int m = 0;
      for (int w = 0; w < NW; ++w) m = max(m, red[w]);
      misc[0] = m;
      for (int c = 0; c < C; ++c) found[c] = 0;
    }
    __syncthreads();
    const int lo_full = misc[0];
    // lo_c = min(max match, cap_c); first R ascending ends with mb >= lo_c.
    if (lo_full > 0) {
      for (int64_t base = 0; base <= dl; base += NT) {
        const int64_t i = base + tid;
        const int m = i <= dl ? delta_mb(a.ix.delta, rpat, P, i) : 0;
        for (int c = 0; c < C; ++c) {
          const int lo = min(lo_full, p.caps[c]);
          const uint64_t bm = ballot(lo > 0 && m >= lo);
          if (ln == 0) wcnt[wv * C + c] = popc(bm);
        }
        __syncthreads();
        if (tid < C) {
          int run = found[tid];
          for (int w = 0; w < NW; ++w) {
            wpre[w * C + tid] = run;
            run += wcnt[w * C + tid];
          }
          found[tid] = run;
        }
        __syncthreads();
        for (int c = 0; c < C; ++c) {
          const int lo = min(lo_full, p.caps[c]);
          const bool hit = lo > 0 && m >= lo;
          const uint64_t bm = ballot(hit);
          if (hit) {
            const int slot = wpre[wv * C + c] + rank_lt(bm);
            if (slot < R)
              a.ws.d_end[((int64_t)b * C + c) * R + slot] = (int32_t)i;
          }
        }
        __syncthreads();
        bool done = true;
        for (int c = 0; c < C; ++c)
          if (min(lo_full, p.caps[c]) > 0 && found[c] < R) done = false;
        if (done) break;
      }
    }
    __syncthreads();
    for (int c = tid; c < C; c += NT) {
      const int lo = min(lo_full, p.caps[c]);
      const int cnt = lo > 0 ? min(found[c], R) : 0;
      a.ws.d_len[(int64_t)b * C + c] = lo;
      a.ws.d_cnt[(int64_t)b * C + c] = cnt;
      if (a.out.d_len) a.out.d_len[(int64_t)b * C + c] = lo;
      if (a.out.d_cnt) a.out.d_cnt[(int64_t)b * C + c] = cnt;
    }
    if (a.out.d_pos) {
      for (int e = tid; e < C * R; e += NT) {
        const int c = e / R;
        const int r = e % R;
        const int lo = min(lo_full, p.caps[c]);
        const int cnt = lo > 0 ? min(found[c], R) : 0;
        const int64_t end =
            r < cnt ? (int64_t)a.ws.d_end[((int64_t)b * C + c) * R + r] : 0;
        int64_t v = end - lo;
        v = v < 0 ? 0 : v;
        a.out.d_pos[((int64_t)b * C + c) * R + r] = v;
      }
    }
  }

  // ---- Handover: the second role to finish merges the row.
  if (!block_arrive(a.ws.join + b, 2u, misc + 1)) return;

  const int nmw = a.merge_waves;
  int32_t* chain = (int32_t*)(smem + L.chain);
  int32_t* res_nv = (int32_t*)(smem + L.nv);
  float* res_score = (float*)(smem + L.score);
  int32_t* res_len = (int32_t*)(smem + L.rlen);
  int32_t* res_occ = (int32_t*)(smem + L.rocc);
  int64_t dl_live = *a.ix.delta_len;
  for (int c = wv; c < C && wv < nmw; c += nmw) {
    // Source selection per cap, before and after dedup (:321-337).
    auto pre = [&](int cc, int& len, int& src) {
      const int sl = a.ws.sa_len[(int64_t)b * C + cc];
      const int dlen = a.ws.d_len[(int64_t)b * C + cc];
      const bool use_sa = sl >= dlen && sl > 0;
      const bool use_d = dlen > sl && dlen > 0;
      len = use_sa ? sl : (use_d ? dlen : 0);
      src = (use_sa ? 1 : 0) + (use_d ? 2 : 0);
    };
    int len, src;
    pre(c, len, src);
    if (c > 0) {
      int plen0, psrc;
      pre(c - 1, plen0, psrc);
      if (len == plen0 && src == psrc && len > 0) {
        len = 0;
        src = 0;
      }
    }
    const int64_t sa_s = a.ws.sa_s[(int64_t)b * C + c];
    const int64_t ilen = (int64_t)a.ws.sa_e[(int64_t)b * C + c] - sa_s;
    int occ = 0;
    if (src == 1) occ = (int)(ilen < R ? ilen : R);
    if (src == 2) occ = a.ws.d_cnt[(int64_t)b * C + c];
    int32_t* mpos = (int32_t*)(smem + L.mpos) + wv * Rp;
    int32_t* mcache = (int32_t*)(smem + L.mcache) + (int64_t)wv * R * K;
    // Occurrence starts: strided SA sample (:339-352) or delta ends - len.
    for (int r = ln; r < occ; r += kWave) {
      int32_t pos;
      if (src == 1) {
        int64_t idx = ilen > R ? sa_s + ((int64_t)r * ilen) / R : sa_s + r;
        idx = idx < 0 ? 0 : (idx > N - 1 ? N - 1 : idx);
        pos = a.ix.sa[idx];
      } else {
        const int64_t e =
            (int64_t)a.ws.d_end[((int64_t)b * C + c) * R + r] - len;
        pos = (int32_t)(e < 0 ? 0 : e);
      }
      mpos[r] = pos;
    }
    wave_lds_sync();
    // Continuations (:443-463): in range, not PAD, not negative.
    const int32_t* srcbuf = src == 1 ? a.ix.corpus : a.ix.delta;
    const int64_t nbuf = src == 1 ? N : D;
    const int64_t slen = src == 1 ? N : dl_live;
    for (int e = ln; e < occ * K; e += kWave) {
      const int r = e / K;
      const int j = e % K;
      const int64_t idx = (int64_t)mpos[r] + len + j;
      int32_t v = -1;
      if (idx < slen && idx >= 0) {
        const int32_t t = srcbuf[idx < nbuf - 1 ? idx : nbuf - 1];
        if (t != kPad && t >= 0) v = t;
      }
      mcache[e] = v;
    }
    wave_lds_sync();
    if (a.out.len && ln == 0) a.out.len[(int64_t)b * C + c] = len;
    if (a.out.occ && ln == 0) a.out.occ[(int64_t)b * C + c] = occ;
    if (a.out.cont) {
      int32_t* o = a.out.cont + ((int64_t)b * C + c) * R * K;
      for (int e = ln; e < R * K; e += kWave)
        o[e] = e < occ * K ? mcache[e] : -1;
    }
    if (a.need_expand) {
      const int64_t cap = spec_cap(p, len);
      auto cont_at = [&](int r, int d) -> int32_t { return mcache[r * K + d]; };
      const ExpandResult er = expand_wave<false>(
          cont_at, NoWeight(), R, occ, K, cap, p.min_token_prob, p.alpha,
          (int32_t*)(smem + L.mA) + wv * Rp, nullptr, chain + c * K);
      if (ln == 0) {
        res_nv[c] = er.nv;
        res_score[c] = er.score;
        res_len[c] = len;
        res_occ[c] = occ;
      }
    }
  }
  if (!a.need_expand) return;
  __syncthreads();
  // Best cap: first argmax of the raw score (proposer.py:308-314,
  // global_index.py:427-436).
  if (tid == 0) {
    int best = 0;
    for (int c = 1; c < C; ++c)
      if (res_score[c] > res_score[best]) best = c;
    const int64_t cap = spec_cap(p, res_len[best]);
    const int64_t cap0 = cap > 0 ? cap : 0;
    misc[2] = best;
    misc[3] = (int)((int64_t)res_nv[best] < cap0 ? res_nv[best] : cap0);
  }
  __syncthreads();
  const int best = misc[2];
  const int emit = misc[3];
  const int32_t* bchain = chain + best * K;
  if (!a.step) {
    if (a.out.draft)
      for (int j = tid; j < K; j += NT)
        a.out.draft[(int64_t)b * K + j] = j < emit ? bchain[j] : -1;
    if (tid == 0) {
      if (a.out.emit) a.out.emit[b] = emit;
      if (a.out.draft_len) a.out.draft_len[b] = res_len[best];
      if (a.out.draft_occ) a.out.draft_occ[b] = res_occ[best];
      if (a.out.draft_score) a.out.draft_score[b] = res_score[best];
    }
    return;
  }
  for (int j = tid; j < K; j += NT)
    a.ws.g_chain[(int64_t)b * K + j] = bchain[j];
  if (tid == 0) {
    a.ws.g_emit[b] = emit;
    a.ws.g_score[b] = res_score[best];
  }
  if (block_arrive(a.ws.pick + b, 2u, misc + 4))
    pick_row(b, K, a.ws, a.draft, a.num_valid);
}

static int merge_waves_for(const sfx_params& p, size_t* lds) {
  const int NW = kGlobalThreads / kWave;
  const int C = p.num_caps;
  int nmw = C < NW ? C : NW;
  if (nmw < 1) nmw = 1;
  for (; nmw >= 1; --nmw) {
    const GlobalLayout L =
        global_layout(p.max_pattern_len, C, p.max_occurrences, p.k, nmw);
    if ((size_t)L.total <= kMaxLds) {
      *lds = (size_t)L.total;
      return nmw;
    }
  }
  return 0;
}

int check_global(const sfx_params& p, const sfx_index& ix) {
  if (p.num_caps < 1 || p.num_caps > SFX_MAX_CANDIDATES) return SFX_EINVAL;
  if (p.k < 1 || p.k > 4096 || p.max_pattern_len < 1 ||
      p.max_pattern_len > 255 || p.max_occurrences < 1 ||
      p.max_occurrences > 2048)
    return SFX_EINVAL;
  if (!ix.corpus || !ix.sa || !ix.delta || !ix.delta_len) return SFX_EINVAL;
  if (ix.capacity < 1 || ix.capacity > 0x7fffffffLL) return SFX_EINVAL;
  if (ix.delta_capacity < 1 || ix.delta_capacity > 0x7fffffffLL)
    return SFX_EINVAL;
  size_t lds = 0;
  if (merge_waves_for(p, &lds) < 1) return SFX_EINVAL;
  return 0;
}

static int launch_global(GlobalArgs& a, hipStream_t stream) {
  if (a.B == 0) return 0;
  size_t lds = 0;
  a.merge_waves = merge_waves_for(a.p, &lds);
  static bool attr_done = false;
  if (!attr_done) {
    hipFuncSetAttribute((const void*)k_global,
                        hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)kMaxLds);
    attr_done = true;
  }
  hipLaunchKernelGGL(k_global, dim3((unsigned)(2 * a.B)),
                     dim3(kGlobalThreads), lds, stream, a);
  return (int)hipGetLastError();
}

int global_step(const sfx_params& p, const sfx_index& ix,
                const sfx_batch& bt, int32_t* draft, int32_t* num_valid,
                const StepWs& ws, hipStream_t stream) {
  GlobalArgs a = {};
  a.p = p;
  a.ix = ix;
  a.B = bt.batch;
  a.step = 1;
  a.bt = bt;
  a.need_expand = 1;
  a.draft = draft;
  a.num_valid = num_valid;
  a.ws = ws;
  return launch_global(a, stream);
}

}  // namespace sfx

using namespace sfx;

extern "C" size_t sfx_global_query_workspace_size(const sfx_params* p,
                                                  int64_t batch) {
  if (!p || batch < 0) return 0;
  return step_ws_layout(*p, batch, nullptr, nullptr);
}

extern "C" int sfx_global_query(const sfx_params* p, const sfx_index* ix,
                                const int32_t* query, int64_t batch,
                                int64_t width, const int64_t* qlen,
                                const sfx_global_out* out, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
  if (!p || !ix || !out || batch < 0) return SFX_EINVAL;
  int rc = check_global(*p, *ix);
  if (rc) return rc;
  if (batch > 0 && (!query || !qlen || width < 1)) return SFX_EINVAL;
  const size_t need = step_ws_layout(*p, batch, nullptr, nullptr);
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
  step_ws_layout(*p, batch, workspace, &a.ws);
  return launch_global(a, stream);
}
