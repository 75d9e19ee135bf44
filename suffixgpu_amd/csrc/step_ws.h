// Workspace layout shared by the fused-step kernels and the global query.
//
// Per row b (B rows), C = number of global caps, K = draft length,
// R = max occurrences.  The handover counters must be zero before a call;
// the kernels leave them zero.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "suffixgpu_amd.h"

namespace sfx {

struct StepWs {
  unsigned* join;     // [B] SA-search + delta-part arrivals (query)
  unsigned* djoin;    // [B] delta-part arrivals (step)
  unsigned* pick;     // [B] step: SA, last delta part and local arrivals
  int32_t* sa_known;  // [B,SFX_MAX_CANDIDATES] step: SA length of cap c + 1,
                      // published by the SA workgroup, 0 until then (the
                      // final pick clears it)
  int32_t* l_chain;   // [B,K] best local chain (uncapped)
  int32_t* l_emit;    // [B]
  float* l_score;     // [B]
  int32_t* sa_len;    // [B,C]
  int32_t* sa_s;      // [B,C]
  int32_t* sa_e;      // [B,C]
  int32_t* sa_nv;     // [B,C] step: expansion of the SA candidate per cap
  float* sa_score;    // [B,C]
  int32_t* sa_chain;  // [B,C,K]
  int32_t* dl_c;      // [B,C] step: row delta length per cap
  int32_t* dn_nv;     // [B,C] step: expansion of the delta candidate
  float* dn_score;    // [B,C]
  int32_t* dn_chain;  // [B,C,K]
  int32_t* d_mx;      // [B,KD] largest match length in each delta part
  int32_t* d_cnt;     // [B,KD,C] hits (<= R) at the part's own threshold
  int32_t* d_map;     // [B,KD,C] the part's list of cap c (caps with equal
                      // thresholds share one)
  int32_t* d_end;     // [B,KD,C,R] ascending end positions in the delta
  uint8_t* d_mb;      // [B*KD, stride] match lengths when LDS is too small
};

// The delta scan of a row is split over up to kMaxDeltaParts workgroups,
// each taking an equal share of the live delta (a device value).  The
// split stops where the step's grid would exceed kGridSlots workgroups:
// 1.25 per CU of an MI355X (256 CUs).  At B = 64 that is three parts (320
// workgroups, a quarter of the CUs holding two, in half-CU LDS layouts):
// step p50 49.2 -> 47.5 us against two parts at one workgroup per CU;
// four parts (384) measured 50.4 us.
// A batch whose grid exceeds two workgroups per CU even with one part
// (3 B > 512) runs in waves of workgroups anyway; its split stops at
// kWaveGridSlots (four per CU) instead.  At B = 256, D = 2^16 with a full
// delta that is two parts: step 123 -> 97 us against one part; three
// parts measured 103 us, four 107 us.
constexpr int kMaxDeltaParts = 4;
constexpr int64_t kDeltaPartSpan = 16384;
constexpr int64_t kCus = 256;
constexpr int64_t kGridSlots = 320;
constexpr int64_t kWaveGridSlots = 4 * kCus;

__host__ __device__ inline int delta_parts_for(int64_t B,
                                               int64_t delta_capacity) {
  const int64_t n = (delta_capacity > 0 ? delta_capacity : 0) + 1;
  int64_t parts = (n + kDeltaPartSpan - 1) / kDeltaPartSpan;
  parts = parts < 1 ? 1 : (parts > kMaxDeltaParts ? kMaxDeltaParts : parts);
  const int64_t slots = 3 * B > 2 * kCus ? kWaveGridSlots : kGridSlots;
  while (parts > 1 && B * (2 + parts) > slots) --parts;
  return (int)parts;
}

// Most positions one part can hold: its share of the capacity plus the
// 16-position alignment of the part bounds.
__host__ __device__ inline int64_t delta_part_cap(int64_t delta_capacity,
                                                  int parts) {
  const int64_t n = (delta_capacity > 0 ? delta_capacity : 0) + 1;
  return (n + parts - 1) / parts + 16;
}

// [lo, hi) of part k of the positions 0 .. n-1; lo is a multiple of 16.
__host__ __device__ inline void delta_part_range(int64_t n, int parts, int k,
                                                 int64_t* lo, int64_t* hi) {
  *lo = k == 0 ? 0 : ((k * n / parts) & ~(int64_t)15);
  *hi = k == parts - 1 ? n : (((k + 1) * n / parts) & ~(int64_t)15);
}

// Delta token index (sfx_delta_index_build): bucket of a token among
// 2^hbits buckets, by Fibonacci hashing of its 32 bits.
constexpr int kDeltaBucketBitsMin = 10;
constexpr int kDeltaBucketBitsMax = 17;
__host__ __device__ inline uint32_t delta_bucket(int32_t t, int hbits) {
  return ((uint32_t)t * 0x9E3779B1u) >> (32 - hbits);
}

// Largest delta part (positions) whose match_back bytes stay in LDS;
// longer parts use StepWs::d_mb.
constexpr int64_t kDeltaMbLdsMax = 65540;

// Bytes per delta part of match_back: its positions plus the tail that the
// 16-byte-word segment reads of a <= 1024-thread block may touch.
__host__ __device__ inline int64_t delta_mb_stride(int64_t part_cap) {
  return ((part_cap + 15) & ~(int64_t)15) + 16 * 1024;
}

inline size_t ws_align(size_t x) { return (x + 255) & ~(size_t)255; }

// Returns the byte size; fills `ws` when base != nullptr.  The three
// handover counter arrays and sa_known (the words that must be zero when
// a call starts and that every call leaves zero) come first, sized for
// `counter_rows` rows (B when negative), so a caller that fixes
// counter_rows keeps them at the same offsets for every batch size:
// kZeroWordsPerRow words per row.
constexpr int64_t kZeroWordsPerRow = 3 + SFX_MAX_CANDIDATES;
inline size_t step_ws_layout(const sfx_params& p, int64_t B,
                             int64_t delta_capacity, void* base,
                             StepWs* ws, int64_t counter_rows = -1) {
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
  const size_t cr = counter_rows < 0 ? b : (size_t)counter_rows;
  StepWs w;
  w.join = (unsigned*)take(cr * 4);
  w.djoin = (unsigned*)take(cr * 4);
  w.pick = (unsigned*)take(cr * 4);
  w.sa_known = (int32_t*)take(cr * SFX_MAX_CANDIDATES * 4);
  w.l_chain = (int32_t*)take(b * K * 4);
  w.l_emit = (int32_t*)take(b * 4);
  w.l_score = (float*)take(b * 4);
  w.sa_len = (int32_t*)take(b * C * 4);
  w.sa_s = (int32_t*)take(b * C * 4);
  w.sa_e = (int32_t*)take(b * C * 4);
  w.sa_nv = (int32_t*)take(b * C * 4);
  w.sa_score = (float*)take(b * C * 4);
  w.sa_chain = (int32_t*)take(b * C * K * 4);
  w.dl_c = (int32_t*)take(b * C * 4);
  w.dn_nv = (int32_t*)take(b * C * 4);
  w.dn_score = (float*)take(b * C * 4);
  w.dn_chain = (int32_t*)take(b * C * K * 4);
  const int KD = delta_parts_for(B, delta_capacity);
  w.d_mx = (int32_t*)take(b * KD * 4);
  w.d_cnt = (int32_t*)take(b * KD * C * 4);
  w.d_map = (int32_t*)take(b * KD * C * 4);
  w.d_end = (int32_t*)take(b * KD * C * R * 4);
  const int64_t pcap = delta_part_cap(delta_capacity, KD);
  w.d_mb = (uint8_t*)take(pcap > kDeltaMbLdsMax
                              ? b * KD * (size_t)delta_mb_stride(pcap)
                              : 0);
  if (ws) *ws = w;
  return off;
}

}  // namespace sfx
