// Host-side launchers shared between the translation units of the library.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

#include "step_ws.h"
#include "suffixgpu_amd.h"

namespace sfx {

// LDS available to one workgroup on gfx950 (160 KiB per CU).
constexpr size_t kMaxLds = 160 * 1024;

// Opts `fn` into the full LDS of a CU on the current device, once per
// device (`done` holds one bit per device ordinal).
inline void allow_max_lds(const void* fn, std::atomic<uint64_t>& done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)kMaxLds);
    return;
  }
  const uint64_t bit = 1ull << dev;
  if (done.load(std::memory_order_acquire) & bit) return;
  hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                      (int)kMaxLds);
  done.fetch_or(bit, std::memory_order_release);
}

// Compute units of the current device (cached per device ordinal).
inline int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount,
                            dev) != hipSuccess ||
      n < 1)
    n = 256;
  cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

// When a grid fits the device one workgroup per CU, ask for more than half
// of a CU's LDS so no two of them share a CU.
inline size_t one_per_cu_lds(size_t lds, unsigned blocks) {
  const size_t half = kMaxLds / 2 + 1024;
  if (blocks <= (unsigned)device_cus() && lds < half) return half;
  return lds;
}

// Longest row (tokens) the local matcher takes: positions stay int32.
constexpr int64_t kMaxSeq = int64_t(1) << 30;
// Rows whose whole-row LDS layout does not fit are streamed in chunks of
// the largest power of two in [kMinStreamChunk, kMaxStreamChunk] that fits.
constexpr int kMaxStreamChunk = 16384;
constexpr int kMinStreamChunk = 1024;

// Two workgroups of a kernel share a CU when each takes at most this much
// LDS (the step kernels' register use allows two 512-thread groups per CU).
constexpr size_t kHalfLds = kMaxLds / 2;
// Three share a CU at this much LDS each (256-byte aligned): the step
// kernels stay at or below 80 VGPRs, 6 waves per SIMD.
constexpr size_t kThirdLds = (kMaxLds / 3) & ~size_t(255);

int check_local(const sfx_params& p, const sfx_batch& bt);
// Local layout within `cap` bytes of LDS for `nthreads` per row: 0 = whole
// row, > 0 = streamed chunk length, -1 = nothing fits; *mb_full tells
// whether a streamed layout holds the whole row's match lengths.
constexpr int kLocalThreadsDefault = 512;
int local_chunk(const sfx_params& p, int64_t S, size_t cap = kMaxLds,
                int nthreads = kLocalThreadsDefault, int* mb_full = nullptr);
size_t local_lds_bytes(const sfx_params& p, int64_t S, int chunk,
                       int nthreads = kLocalThreadsDefault, int mb_full = 0);

int check_global(const sfx_params& p, const sfx_index& ix, int64_t batch);
int mb_lds_bytes(const sfx_index& ix, int parts);
// Delta workgroups per row: one with the delta token index, else
// delta_parts_for's split of the delta.
int delta_parts_of(const sfx_index& ix, int64_t batch);
// Merge waves (one per cap expansion) whose layout fits `cap`, with the
// delta parts' end lists in LDS when dend_parts > 0 (decode step).
int merge_waves_for(const sfx_params& p, const sfx_index& ix, int parts,
                    size_t* lds, size_t cap = kMaxLds, int dend_parts = 0);
// Delta positions a part stages per chunk: the most that fit `cap` beside
// the rest of the layout (a whole part when it fits), at least 8192; *lds
// = the layout's bytes.
int delta_chunk_for(const sfx_params& p, const sfx_index& ix, int parts,
                    int nmw, int dend_parts, size_t cap, size_t* lds);

}  // namespace sfx
