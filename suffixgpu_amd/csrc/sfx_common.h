// Shared device helpers for the gfx950 drafter kernels: wave64 primitives,
// the fp32 rules of the chain score, and the wave-level majority-vote
// chain expansion used by the local, global and standalone expand paths.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "suffixgpu_amd.h"

namespace sfx {

constexpr int kWave = 64;
constexpr int32_t kPad = 0x7fffffff;  // corpus fill past the end
constexpr int32_t kSep = -2;          // document separator

// ------------------------------------------------------------ wave64 ops
__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

__device__ __forceinline__ int popc(uint64_t m) { return __popcll(m); }

// Number of set bits of m in lanes below the calling lane.
__device__ __forceinline__ int rank_lt(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi(
      (unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = __shfl_xor(v, o);
    v = w > v ? w : v;
  }
  return v;
}

__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

// Order LDS traffic of the calling wave (writes before later reads).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ int64_t load_count(const void* p, int is64,
                                              int64_t i) {
  return is64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

// ------------------------------------------------------------ fp32 rules
// The chain probability and scores follow torch's fp32 CPU arithmetic:
// every operation rounds to fp32 (no FMA contraction; the library is built
// with -ffp-contract=off as well) and the division is IEEE-correct.

// max(0, floor(fl32(f) * fl32(L) + fl32(off))) as int64
// (suffix_gpu/local_matcher.py:76-81).  Float->int64 conversions that
// overflow produce INT64_MIN on the reference's x86 host and then clamp to
// 0; the same happens here.
__device__ __forceinline__ int64_t spec_cap(const sfx_params& p,
                                            int64_t len) {
  if (!p.has_spec_factor) return p.k;
  float v = __fadd_rn(__fmul_rn(p.spec_factor, (float)len), p.spec_offset);
  if (!(v < 9.2233720368547758e18f)) return 0;  // overflow or NaN
  if (!(v >= 0.0f)) return 0;
  return (int64_t)floorf(v);
}

// score + fl32(fl32(len) * fl32(1e-6)) (local_matcher.py:259-260).
__device__ __forceinline__ float local_key(float score, int64_t len) {
  return __fadd_rn(score, __fmul_rn((float)len, 1e-6f));
}

// ---------------------------------------------------- majority-vote expand
struct ExpandResult {
  int nv;       // number of valid chain slots (a prefix)
  float score;  // sum of the chain probability over valid slots < cap
};

// Wave-cooperative depth-wise majority vote of one candidate
// (suffix_gpu/expand.py:59-147 == triton_kernels.py:139-215).
//
// Occurrence r (< R) is row r of the candidate's continuation block;
// cont_at(r, d) returns its token at depth d and is only called for rows
// still on the chain (r < occ and every earlier depth voted for them).
// Per depth the active rows (token != -1) are compacted into A (in row
// order), every lane counts the votes of its compacted entries by
// broadcast LDS reads, and a 64-bit wave max picks (max votes, min token).
// chain_out[0..K) receives the chain (-1 past the first invalid depth).
// A holds R ints; W (weighted votes only) R floats, both LDS.
template <bool kWeighted, class ContFn, class WeightFn>
__device__ ExpandResult expand_wave(ContFn cont_at, WeightFn weight_at,
                                    int R, int64_t occ, int K, int64_t cap,
                                    float min_prob, float alpha, int* A,
                                    float* W, int32_t* chain_out) {
  const int ln = lane_id();
  const int nslot = (R + kWave - 1) / kWave;  // <= 32 (R <= 2048)
  uint32_t ok = 0;
  for (int s = 0; s < nslot; ++s) {
    int r = s * kWave + ln;
    if (r < R && (int64_t)r < occ) ok |= 1u << s;
  }
  float prob = 1.0f;
  float score = 0.0f;
  int nv = 0;
  int d = 0;
  for (; d < K; ++d) {
    int nact = 0;
    for (int s = 0; s < nslot; ++s) {
      const int r = s * kWave + ln;
      const bool okr = (ok >> s) & 1u;
      int c = -1;
      if (okr) c = cont_at(r, d);
      const bool act = okr && c != -1;
      const uint64_t m = ballot(act);
      if (act) {
        const int pos = nact + rank_lt(m);
        A[pos] = c;
        if (kWeighted) W[pos] = weight_at(r);
      }
      nact += popc(m);
      if (!act) ok &= ~(1u << s);
    }
    wave_lds_sync();
    if (nact == 0) break;
    uint64_t best = 0;
    for (int i = ln; i < nact; i += kWave) {
      const int x = A[i];
      uint32_t vbits;
      if (!kWeighted) {
        int v = 0;
        int j = 0;
        for (; j + 4 <= nact; j += 4) {
          const int4 q = *reinterpret_cast<const int4*>(A + j);
          v += (q.x == x) + (q.y == x) + (q.z == x) + (q.w == x);
        }
        for (; j < nact; ++j) v += (A[j] == x);
        vbits = (uint32_t)v;
      } else {
        float v = 0.0f;
        for (int j = 0; j < nact; ++j)
          if (A[j] == x) v = __fadd_rn(v, W[j]);
        vbits = __float_as_uint(v);
      }
      // max votes first, then the smallest (signed) token
      const uint64_t key =
          ((uint64_t)vbits << 32) |
          (uint64_t)(0xffffffffu - ((uint32_t)x ^ 0x80000000u));
      best = key > best ? key : best;
    }
    best = wave_max_u64(best);
    const uint32_t vbits = (uint32_t)(best >> 32);
    const int tok = (int)((0xffffffffu - (uint32_t)best) ^ 0x80000000u);
    float vf;
    float denom;
    if (!kWeighted) {
      vf = (float)(int)vbits;
      denom = __fadd_rn((float)(nact > 1 ? nact : 1), alpha);
    } else {
      vf = __uint_as_float(vbits);
      float a = 0.0f;
      for (int j = 0; j < nact; ++j) a = __fadd_rn(a, W[j]);
      denom = __fadd_rn(a, alpha);
    }
    prob = __fmul_rn(prob, __fdiv_rn(vf, denom));
    const bool valid = (vf > 0.0f) && (prob >= min_prob);
    if (!valid) break;
    if (ln == 0) chain_out[d] = tok;
    if ((int64_t)d < cap) score = __fadd_rn(score, prob);
    ++nv;
    for (int s = 0; s < nslot; ++s) {
      if ((ok >> s) & 1u) {
        if (cont_at(s * kWave + ln, d) != tok) ok &= ~(1u << s);
      }
    }
    wave_lds_sync();
  }
  for (int dd = d + ln; dd < K; dd += kWave) chain_out[dd] = -1;
  ExpandResult res;
  res.nv = nv;
  res.score = score;
  return res;
}

struct NoWeight {
  __device__ float operator()(int) const { return 0.0f; }
};

// -------------------------------------------------- block-level handover
// Publish this block's global writes, count its arrival on ctr and return
// (to every thread) whether it was the last of `expected` arrivals.  The
// last arriver resets the counter, so the workspace is zero again after
// every call.  Call from uniform control flow.
__device__ __forceinline__ bool block_arrive(unsigned* ctr,
                                             unsigned expected,
                                             int* lds_flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned old = atomicAdd(ctr, 1u);
    int last = (old == expected - 1);
    if (last) atomicExch(ctr, 0u);
    *lds_flag = last;
  }
  __syncthreads();
  const bool last = *lds_flag != 0;
  if (last) __threadfence();
  return last;
}

}  // namespace sfx
