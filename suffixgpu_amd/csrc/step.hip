// Fused decode step (suffix_gpu/proposer.py:186-327) in one launch.
//
// With global memory each request row gets 2 + dparts 512-thread
// workgroups: SA interval search, dparts delta-scan parts, local match,
// ordered by role.  The SA and delta workgroups hand over through the
// workspace and the last of them merges the row's global candidates;
// local and global results meet the same way and the later one writes the
// row's draft.  Nothing waits on another workgroup,
// so any scheduling order completes.  Local-only drafting is one workgroup
// per row.  One kernel node per step keeps a captured HIP graph minimal.

#include <mutex>

#include "global_impl.h"
#include "launch.h"
#include "local_impl.h"

namespace sfx {

static_assert(kLocalThreads == kGlobalThreads,
              "the fused step runs every role with one block size");

struct StepArgs {
  LocalArgs l;
  GlobalArgs g;
  int global_on;
};

template <bool kStream>
__global__ __launch_bounds__(kGlobalThreads) void k_step(StepArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  if (!a.global_on) {
    local_body<kStream>(a.l, smem, blockIdx.x);
    return;
  }
  // Blocks are ordered by role (role 0: SA, 1..dparts: delta parts,
  // per - 1: local): local, then the delta parts, then SA.  A grid beyond
  // the workgroups that run at once finishes in waves, so the order
  // decides which roles start at once.  With the delta token index (one
  // delta workgroup per row, whose bucket walk ends with the delta
  // expansion) B = 256, S = 16384 with a full 2^16 delta measured
  // 48.7-49.5 us with SA second and 42.4-43.3 us with the delta second.
  // (Scanning the delta, two parts per row, SA second had measured 94-97
  // us and row by row 112-115 us.)  At B = 64 (one wave) the orders
  // measured the same within 0.3 us.  The order is a fixed function of
  // the block index: an order chosen by a kernel argument made the
  // compiler spill the streamed variant to scratch.
  const int per = 2 + a.g.dparts;
  const int B = (int)a.g.B;
  const int slot = (int)(blockIdx.x / B);
  const int b = (int)(blockIdx.x % B);
  const int role = slot == 0 ? per - 1 : (slot == per - 1 ? 0 : slot);
  if (role == per - 1)
    local_body<kStream>(a.l, smem, b);
  else
    global_body<!kStream>(a.g, smem, b, role);
}

}  // namespace sfx

using namespace sfx;

extern "C" size_t sfx_step_workspace_size(const sfx_params* p,
                                          int64_t batch,
                                          int64_t delta_capacity) {
  if (!p || batch < 0) return 0;
  return step_ws_layout(*p, batch, delta_capacity, nullptr, nullptr);
}

// ------------------------------------------------- allocation-free form
// The step's workspace as a file-scope device array: each GPU the library
// runs on holds one copy until the process ends, and every call on that
// GPU shares it.  Its handover counters sit at fixed offsets (arrays of
// SFX_NOALLOC_MAX_ROWS rows), are cleared once per device at set-up and are
// left zero by every step, so calls of any batch size can follow each
// other; calls that overlap on one GPU race on them.
static __device__ __align__(256) unsigned char
    scratch[(size_t)SFX_NOALLOC_SCRATCH_BYTES];

static __global__ __launch_bounds__(256) void k_zero_words(uint32_t* w,
                                                           int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    w[i] = 0u;
}

namespace {

// The fused step over `workspace` laid out with counter arrays of
// `counter_rows` rows (-1: the batch size).
int launch_step(const sfx_params* p, const sfx_index* ix, const sfx_batch* bt,
                int32_t* draft, int32_t* num_valid, int32_t* new_counts,
                void* workspace, size_t workspace_bytes, int64_t counter_rows,
                hipStream_t stream) {
  if (!p || !bt || !draft || !num_valid) return SFX_EINVAL;
  int rc = check_local(*p, *bt);
  if (rc) return rc;
  if (bt->sampled && bt->limit < 0) return SFX_EINVAL;
  const bool global_on = ix != nullptr;
  StepArgs a = {};
  a.global_on = global_on ? 1 : 0;
  a.l.p = *p;
  a.l.bt = *bt;
  a.l.mode = kLocalStep;
  a.l.global_on = a.global_on;
  a.l.draft = draft;
  a.l.num_valid = num_valid;
  a.l.new_counts = new_counts;
  if (!global_on && bt->seq >= kWideMinSeq) {
    // local-only rows of 8192 tokens or more: one 1024-thread workgroup
    // per row when its layout fits
    rc = launch_local_step(a.l, stream);
    if (rc >= 0) return rc;
  }
  const int dparts = global_on ? delta_parts_of(*ix, bt->batch) : 0;
  const unsigned blocks =
      (unsigned)(bt->batch * (global_on ? 2 + dparts : 1));
  // A grid larger than the CU count runs in waves of workgroups; when every
  // role fits half a CU's LDS, two groups share each CU and the waves halve,
  // and past twice the CU count, a third: three groups per CU.  Otherwise
  // each role takes the LDS layout that suits it best.
  size_t cap = kMaxLds;
  auto fits = [&](size_t c) {
    size_t glds = 0;
    return local_chunk(*p, bt->seq, c) >= 0 &&
           (!global_on || merge_waves_for(*p, *ix, dparts, &glds, c) > 0);
  };
  const unsigned cus = (unsigned)device_cus();
  if (blocks > 2 * cus && fits(kThirdLds))
    cap = kThirdLds;
  else if (blocks > cus && fits(kHalfLds))
    cap = kHalfLds;
  a.l.chunk = local_chunk(*p, bt->seq, cap, kLocalThreadsDefault,
                          &a.l.mb_full);
  size_t lds = local_lds_bytes(*p, bt->seq, a.l.chunk, kLocalThreadsDefault,
                               a.l.mb_full);
  if (global_on) {
    rc = check_global(*p, *ix, bt->batch);
    if (rc) return rc;
    const size_t need = step_ws_layout(*p, bt->batch, ix->delta_capacity,
                                       nullptr, nullptr, counter_rows);
    if (!workspace || workspace_bytes < need) return SFX_EINVAL;
    step_ws_layout(*p, bt->batch, ix->delta_capacity, workspace, &a.l.ws,
                   counter_rows);
    a.g.p = *p;
    a.g.ix = *ix;
    a.g.B = bt->batch;
    a.g.step = 1;
    a.g.bt = *bt;
    a.g.need_expand = 1;
    a.g.draft = draft;
    a.g.num_valid = num_valid;
    a.g.ws = a.l.ws;
    size_t glds = 0;
    a.g.dparts = dparts;
    // the parts' end lists in LDS at the join, unless they would take a
    // merge wave away
    a.g.dend = 1;
    a.g.merge_waves = merge_waves_for(*p, *ix, dparts, &glds, cap, dparts);
    size_t glds0 = 0;
    const int nmw0 = merge_waves_for(*p, *ix, dparts, &glds0, cap, 0);
    if (nmw0 > a.g.merge_waves) {
      a.g.dend = 0;
      a.g.merge_waves = nmw0;
    }
    a.g.mb_lds = mb_lds_bytes(*ix, dparts);
    a.g.dchunk = delta_chunk_for(*p, *ix, dparts, a.g.merge_waves,
                                 a.g.dend ? dparts : 0, cap, &glds);
    lds = lds > glds ? lds : glds;
  }
  if (lds > kMaxLds) return SFX_EINVAL;
  if (bt->batch == 0) return 0;
  lds = one_per_cu_lds(lds, blocks);
  if (a.l.chunk == 0) {
    static std::atomic<uint64_t> lds_opt{0};
    allow_max_lds((const void*)k_step<false>, lds_opt);
    hipLaunchKernelGGL(k_step<false>, dim3(blocks), dim3(kGlobalThreads), lds,
                       stream, a);
  } else {
    static std::atomic<uint64_t> lds_opt{0};
    allow_max_lds((const void*)k_step<true>, lds_opt);
    hipLaunchKernelGGL(k_step<true>, dim3(blocks), dim3(kGlobalThreads), lds,
                       stream, a);
  }
  return (int)hipGetLastError();
}

constexpr int64_t kScratchRows = SFX_NOALLOC_MAX_ROWS;
constexpr int kMaxDevices = 64;

std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices] = {};

// This device's copy of `scratch` (the device current on this host
// thread).  The first call on a device resolves the address with
// hipGetSymbolAddress -- in host code the array's name is not a device
// address -- and clears the counter arrays with a fill kernel on `stream`.
int scratch_of_current_device(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return SFX_EINVAL;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr) return SFX_EINVAL;
    // join, djoin, pick and sa_known: the words every step leaves zero
    const int64_t words = kZeroWordsPerRow * kScratchRows;
    hipLaunchKernelGGL(k_zero_words, dim3(64), dim3(256), 0, stream,
                       (uint32_t*)ptr, words);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    scratch_ptr[dev] = ptr;
  }
  *out = scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int sfx_propose_step(const sfx_params* p, const sfx_index* ix,
                                const sfx_batch* bt, int32_t* draft,
                                int32_t* num_valid, int32_t* new_counts,
                                void* workspace, size_t workspace_bytes,
                                hipStream_t stream) {
  return launch_step(p, ix, bt, draft, num_valid, new_counts, workspace,
                     workspace_bytes, -1, stream);
}

extern "C" int sfx_propose_step_noalloc(const sfx_params* p,
                                        const sfx_index* ix,
                                        const sfx_batch* bt, int32_t* draft,
                                        int32_t* num_valid,
                                        int32_t* new_counts,
                                        hipStream_t stream) {
  if (!p || !bt) return SFX_EINVAL;
  if (!ix)  // local-only steps use no workspace
    return launch_step(p, nullptr, bt, draft, num_valid, new_counts, nullptr,
                       0, -1, stream);
  if (bt->batch < 0) return SFX_EINVAL;
  if (bt->batch > kScratchRows ||
      step_ws_layout(*p, bt->batch, ix->delta_capacity, nullptr, nullptr,
                     kScratchRows) > (size_t)SFX_NOALLOC_SCRATCH_BYTES)
    return SFX_ENOSCRATCH;
  void* ws = nullptr;
  const int rc = scratch_of_current_device(stream, &ws);
  if (rc) return rc;
  return launch_step(p, ix, bt, draft, num_valid, new_counts, ws,
                     (size_t)SFX_NOALLOC_SCRATCH_BYTES, kScratchRows, stream);
}
