// Local (per-request) suffix matcher: one 1024-thread workgroup per row.
//
// The row is staged once in LDS (coalesced int4 loads), the step's sampled
// tokens are scattered into LDS and HBM, and everything else runs out of
// LDS: the newest-first pattern, match_back (leading-match count of the
// tokens ending at i against the pattern, early exit per position, kept as
// u8), a 33-bin histogram whose suffix sums give every support threshold's
// candidate length, the ordered ballot/mbcnt compaction of the first R
// occurrence ends per candidate, and one wave per candidate running the
// majority-vote expansion straight off the LDS row.
//
// Follows suffix_gpu/local_matcher.py:83-263 and proposer.py:135-184,
// 322-327.

#include "launch.h"
#include "pick.h"
#include "sfx_common.h"
#include "step_ws.h"

namespace sfx {

enum LocalMode { kLocalGather = 0, kLocalForward = 1, kLocalStep = 2 };

struct LocalArgs {
  sfx_params p;
  sfx_batch bt;
  int mode;
  int global_on;
  int64_t* cand_out;   // gather
  int32_t* cont_out;
  int64_t* occ_out;
  int32_t* draft;      // forward / step
  int32_t* num_valid;
  int64_t* len_out;    // forward
  int64_t* occ1_out;
  float* score_out;
  int32_t* new_counts;  // step
  StepWs ws;
};

struct LocalLayout {
  int row, mb, pat, hist, cand, found, wcnt, wpre, occ, A, chain, nv, score,
      misc, total;
};

__host__ __device__ inline int lds_take(int& off, int bytes) {
  const int o = off;
  off += (bytes + 15) & ~15;
  return o;
}

__host__ __device__ inline LocalLayout local_layout(int S, int P, int C,
                                                    int R, int K,
                                                    int nwaves) {
  LocalLayout L;
  int off = 0;
  L.row = lds_take(off, S * 4);
  L.mb = lds_take(off, S);
  L.pat = lds_take(off, P * 4);
  L.hist = lds_take(off, (P + 1) * 4);
  L.cand = lds_take(off, C * 4);
  L.found = lds_take(off, C * 4);
  L.wcnt = lds_take(off, nwaves * C * 4);
  L.wpre = lds_take(off, nwaves * C * 4);
  L.occ = lds_take(off, C * R * 4);
  L.A = lds_take(off, nwaves * ((R + 3) & ~3) * 4);
  L.chain = lds_take(off, C * K * 4);
  L.nv = lds_take(off, C * 4);
  L.score = lds_take(off, C * 4);
  L.misc = lds_take(off, 64);
  L.total = off;
  return L;
}

constexpr int kLocalThreads = 1024;

__global__ __launch_bounds__(kLocalThreads) void k_local(LocalArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NT = kLocalThreads;
  constexpr int NW = NT / kWave;
  const sfx_params& p = a.p;
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int ln = tid % kWave;
  const int S = (int)a.bt.seq;
  const int P = p.max_pattern_len;
  const int C = p.num_thresholds;
  const int R = p.max_occurrences;
  const int K = p.k;
  const LocalLayout L = local_layout(S, P, C, R, K, NW);
  int32_t* row = (int32_t*)(smem + L.row);
  uint8_t* mbuf = (uint8_t*)(smem + L.mb);
  int32_t* pat = (int32_t*)(smem + L.pat);
  int32_t* hist = (int32_t*)(smem + L.hist);
  int32_t* cand = (int32_t*)(smem + L.cand);
  int32_t* found = (int32_t*)(smem + L.found);
  int32_t* wcnt = (int32_t*)(smem + L.wcnt);
  int32_t* wpre = (int32_t*)(smem + L.wpre);
  int32_t* occ = (int32_t*)(smem + L.occ);
  int32_t* Abuf = (int32_t*)(smem + L.A);
  int32_t* chain = (int32_t*)(smem + L.chain);
  int32_t* res_nv = (int32_t*)(smem + L.nv);
  float* res_score = (float*)(smem + L.score);
  int* misc = (int*)(smem + L.misc);

  const RowState st = row_state(a.bt, b);
  const int64_t q = st.q;

  // Stage the row, then apply this step's scatter (proposer.py:162-184).
  int32_t* grow = a.bt.tokens + (int64_t)b * S;
  if ((S & 3) == 0 && (((uintptr_t)grow) & 15) == 0) {
    const int4* src = reinterpret_cast<const int4*>(grow);
    int4* dst = reinterpret_cast<int4*>(row);
    for (int i = tid; i < S / 4; i += NT) dst[i] = src[i];
  } else {
    for (int i = tid; i < S; i += NT) row[i] = grow[i];
  }
  __syncthreads();
  if (a.bt.sampled) {
    const int32_t* sp = a.bt.sampled + (int64_t)b * a.bt.num_sampled;
    for (int64_t j = tid; j < a.bt.num_sampled; j += NT) {
      const int64_t pos = st.base + j;
      const int32_t v = sp[j];
      if (j < st.cnt && v != -1 && pos < S && pos >= 0) {
        row[pos] = v;
        grow[pos] = v;
      }
    }
    if (a.new_counts && tid == 0) a.new_counts[b] = (int32_t)q;
  }
  __syncthreads();

  if (a.mode == kLocalStep && !st.mask) {
    for (int j = tid; j < K; j += NT) a.draft[(int64_t)b * K + j] = -1;
    if (tid == 0) a.num_valid[b] = 0;
    return;
  }

  // Newest-first pattern, -2 fill (local_matcher.py:103-112).
  for (int t = tid; t < P; t += NT) {
    const int64_t idx = q - 1 - t;
    pat[t] = idx >= 0 ? row[idx < S - 1 ? idx : S - 1] : -2;
  }
  for (int i = tid; i <= P; i += NT) hist[i] = 0;
  __syncthreads();

  // match_back, zero at i >= q (local_matcher.py:114-132).
  for (int i = tid; i < S; i += NT) {
    int m = 0;
    if ((int64_t)i < q) {
      for (int t = 0; t < P; ++t) {
        const int j = i - 1 - t;
        const int32_t x = j >= 0 ? row[j] : -1;
        if (x != pat[t]) break;
        ++m;
      }
    }
    mbuf[i] = (uint8_t)m;
    if (m > 0) atomicAdd(&hist[m], 1);
  }
  __syncthreads();

  // Candidates: thr-th largest match_back = largest L with #{mb >= L} >=
  // thr; zero below min_match_len or when masked; adjacent duplicates
  // zeroed (local_matcher.py:134-157).
  if (tid == 0) {
    int ge = 0;
    for (int Lv = P; Lv >= 1; --Lv) {
      ge += hist[Lv];
      hist[Lv] = ge;
    }
    int maxthr = p.thresholds[0];
    for (int c = 1; c < C; ++c) maxthr = max(maxthr, p.thresholds[c]);
    const int w = min(maxthr, S);
    int prev_raw = -1;
    for (int c = 0; c < C; ++c) {
      const int thr = p.thresholds[c];
      int v = 0;
      if (thr <= w) {
        const int t = thr < 1 ? 1 : thr;
        for (int Lv = P; Lv >= 1; --Lv) {
          if (hist[Lv] >= t) {
            v = Lv;
            break;
          }
        }
      }
      if (!(v >= p.min_match_len && st.mask)) v = 0;
      const int raw = v;
      if (c > 0 && raw == prev_raw) v = 0;
      prev_raw = raw;
      cand[c] = v;
      found[c] = 0;
    }
  }
  __syncthreads();

  // First R ascending ends per candidate: ordered block compaction
  // (triton_kernels.py:217-243 semantics, early exit once all are full).
  for (int base = 0; base < S; base += NT) {
    const int i = base + tid;
    const int m = i < S ? mbuf[i] : 0;
    for (int c = 0; c < C; ++c) {
      const int cv = cand[c];
      const uint64_t bm = ballot(cv > 0 && m >= cv);
      if (ln == 0) wcnt[wv * C + c] = popc(bm);
    }
    __syncthreads();
    if (tid < C) {
      int run = found[tid];
      for (int w2 = 0; w2 < NW; ++w2) {
        wpre[w2 * C + tid] = run;
        run += wcnt[w2 * C + tid];
      }
      found[tid] = run;
    }
    __syncthreads();
    for (int c = 0; c < C; ++c) {
      const int cv = cand[c];
      const bool hit = cv > 0 && m >= cv;
      const uint64_t bm = ballot(hit);
      if (hit) {
        const int slot = wpre[wv * C + c] + rank_lt(bm);
        if (slot < R) occ[c * R + slot] = i;
      }
    }
    __syncthreads();
    bool done = true;
    for (int c = 0; c < C; ++c)
      if (cand[c] > 0 && found[c] < R) done = false;
    if (done) break;
  }

  if (a.mode == kLocalGather) {
    for (int c = tid; c < C; c += NT) {
      if (a.cand_out) a.cand_out[(int64_t)b * C + c] = cand[c];
      if (a.occ_out) a.occ_out[(int64_t)b * C + c] = min(found[c], R);
    }
    if (a.cont_out) {
      const int total = C * R * K;
      int32_t* out = a.cont_out + (int64_t)b * total;
      for (int e = tid; e < total; e += NT) {
        const int c = e / (R * K);
        const int r = (e / K) % R;
        const int j = e % K;
        int32_t v = -1;
        if (r < min(found[c], R)) {
          const int64_t idx = (int64_t)occ[c * R + r] + j;
          if (idx < q) v = row[idx < S - 1 ? idx : S - 1];
        }
        out[e] = v;
      }
    }
    return;
  }

  // One wave per candidate: majority-vote expansion from the LDS row.
  for (int c = wv; c < C; c += NW) {
    const int cv = cand[c];
    const int64_t oc = cv > 0 ? (int64_t)min(found[c], R) : 0;
    const int64_t cap = spec_cap(p, cv);
    const int32_t* oc_list = occ + c * R;
    auto cont_at = [&](int r, int d) -> int32_t {
      const int64_t idx = (int64_t)oc_list[r] + d;
      return idx < q ? row[idx < S - 1 ? idx : S - 1] : -1;
    };
    const ExpandResult er = expand_wave<false>(
        cont_at, NoWeight(), R, oc, K, cap, p.min_token_prob, p.alpha,
        Abuf + wv * ((R + 3) & ~3), nullptr, chain + c * K);
    if (ln == 0) {
      res_nv[c] = er.nv;
      res_score[c] = er.score;
    }
  }
  __syncthreads();

  // select_local_best (local_matcher.py:245-263).
  if (tid == 0) {
    int best = 0;
    float bkey = local_key(res_score[0], cand[0]);
    for (int c = 1; c < C; ++c) {
      const float key = local_key(res_score[c], cand[c]);
      if (key > bkey) {
        bkey = key;
        best = c;
      }
    }
    const int64_t cap = spec_cap(p, cand[best]);
    const int64_t cap0 = cap > 0 ? cap : 0;
    misc[0] = best;
    misc[1] = (int)((int64_t)res_nv[best] < cap0 ? res_nv[best] : cap0);
  }
  __syncthreads();
  const int best = misc[0];
  const int emit = misc[1];
  const int32_t* bchain = chain + best * K;

  if (a.mode == kLocalForward) {
    for (int j = tid; j < K; j += NT)
      a.draft[(int64_t)b * K + j] = j < emit ? bchain[j] : -1;
    if (tid == 0) {
      a.num_valid[b] = emit;
      if (a.len_out) a.len_out[b] = cand[best];
      if (a.occ1_out)
        a.occ1_out[b] = cand[best] > 0 ? min(found[best], R) : 0;
      if (a.score_out) a.score_out[b] = res_score[best];
    }
    return;
  }

  // Decode step.
  if (!a.global_on) {
    for (int j = tid; j < K; j += NT)
      a.draft[(int64_t)b * K + j] = j < emit ? bchain[j] : -1;
    if (tid == 0) a.num_valid[b] = emit;
    return;
  }
  for (int j = tid; j < K; j += NT)
    a.ws.l_chain[(int64_t)b * K + j] = bchain[j];
  if (tid == 0) {
    a.ws.l_emit[b] = emit;
    a.ws.l_score[b] = res_score[best];
  }
  if (block_arrive(a.ws.pick + b, 2u, misc + 2))
    pick_row(b, K, a.ws, a.draft, a.num_valid);
}

size_t local_lds_bytes(const sfx_params& p, int64_t S) {
  const LocalLayout L =
      local_layout((int)S, p.max_pattern_len, p.num_thresholds,
                   p.max_occurrences, p.k, kLocalThreads / kWave);
  return (size_t)L.total;
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
  if (local_lds_bytes(p, bt.seq) > kMaxLds) return SFX_EINVAL;
  return 0;
}

int launch_local(const LocalArgs& a, hipStream_t stream) {
  if (a.bt.batch == 0) return 0;
  const size_t lds = local_lds_bytes(a.p, a.bt.seq);
  static bool attr_done = false;
  if (!attr_done) {
    hipFuncSetAttribute((const void*)k_local,
                        hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)kMaxLds);
    attr_done = true;
  }
  hipLaunchKernelGGL(k_local, dim3((unsigned)a.bt.batch), dim3(kLocalThreads),
                     lds, stream, a);
  return (int)hipGetLastError();
}

int local_step(const sfx_params& p, const sfx_batch& bt, bool global_on,
               int32_t* draft, int32_t* num_valid, int32_t* new_counts,
               const StepWs& ws, hipStream_t stream) {
  LocalArgs a = {};
  a.p = p;
  a.bt = bt;
  a.mode = kLocalStep;
  a.global_on = global_on ? 1 : 0;
  a.draft = draft;
  a.num_valid = num_valid;
  a.new_counts = new_counts;
  a.ws = ws;
  return launch_local(a, stream);
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
