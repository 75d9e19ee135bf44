// Workspace layout shared by the fused-step kernels and the global query.
//
// Per row b (B rows), C = number of global caps, K = draft length,
// R = max occurrences.  The two handover counters must be zero before a
// call; the kernels leave them zero.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "suffixgpu_amd.h"

namespace sfx {

struct StepWs {
  unsigned* join;    // [B] SA-search + delta-scan arrivals
  unsigned* pick;    // [B] local + global arrivals
  int32_t* l_chain;  // [B,K] best local chain (uncapped)
  int32_t* l_emit;   // [B]
  float* l_score;    // [B]
  int32_t* g_chain;  // [B,K] best global chain (uncapped)
  int32_t* g_emit;   // [B]
  float* g_score;    // [B]
  int32_t* sa_len;   // [B,C]
  int32_t* sa_s;     // [B,C]
  int32_t* sa_e;     // [B,C]
  int32_t* d_len;    // [B,C]
  int32_t* d_cnt;    // [B,C]
  int32_t* d_end;    // [B,C,R] ascending end positions in the delta
  uint8_t* d_mb;     // [B,D+1] delta match_back when it does not fit LDS
};

// Largest delta (capacity + 1 positions) whose per-row match_back bytes
// stay in LDS; longer deltas use StepWs::d_mb.
constexpr int64_t kDeltaMbLdsMax = 65540;

// Bytes per row of delta match_back: the positions plus the tail that the
// 16-byte-word segment reads of a <= 1024-thread block may touch.
__host__ __device__ inline int64_t delta_mb_stride(int64_t delta_capacity) {
  return ((delta_capacity + 1 + 15) & ~(int64_t)15) + 16 * 1024;
}

inline size_t ws_align(size_t x) { return (x + 255) & ~(size_t)255; }

// Returns the byte size; fills `ws` when base != nullptr.
inline size_t step_ws_layout(const sfx_params& p, int64_t B,
                             int64_t delta_capacity, void* base,
                             StepWs* ws) {
  const size_t C = p.num_caps > 0 ? (size_t)p.num_caps : 1;
  const size_t K = (size_t)p.k;
  const size_t R = (size_t)p.max_occurrences;
  const size_t b = (size_t)B;
  size_t off = 0;
  char* c = (char*)base;
  auto take = [&](size_t bytes) -> void* {
    void* ptr = c ? (void*)(c + off) : nullptr;
    off += ws_align(bytes);
    return ptr;
  };
  StepWs w;
  w.join = (unsigned*)take(b * 4);
  w.pick = (unsigned*)take(b * 4);
  w.l_chain = (int32_t*)take(b * K * 4);
  w.l_emit = (int32_t*)take(b * 4);
  w.l_score = (float*)take(b * 4);
  w.g_chain = (int32_t*)take(b * K * 4);
  w.g_emit = (int32_t*)take(b * 4);
  w.g_score = (float*)take(b * 4);
  w.sa_len = (int32_t*)take(b * C * 4);
  w.sa_s = (int32_t*)take(b * C * 4);
  w.sa_e = (int32_t*)take(b * C * 4);
  w.d_len = (int32_t*)take(b * C * 4);
  w.d_cnt = (int32_t*)take(b * C * 4);
  w.d_end = (int32_t*)take(b * C * R * 4);
  const int64_t dcap = delta_capacity > 0 ? delta_capacity : 0;
  w.d_mb = (uint8_t*)take(dcap + 1 > kDeltaMbLdsMax
                              ? b * (size_t)delta_mb_stride(dcap)
                              : 0);
  if (ws) *ws = w;
  return off;
}

}  // namespace sfx
