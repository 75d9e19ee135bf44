// Device-side ingest of finished responses into the global index
// (suffix_gpu/global_index.py:86-215 append_documents, _make_room,
// _drop_oldest_docs, maybe_rebuild, _plan_rebuild and the snapshot of
// _launch_rebuild), with the document lengths and every decision on the
// device: the caller passes device row indices and lengths and nothing is
// read back.
//
// The state (sfx_ingest_layout) holds a header (sfx_ingest_header), the
// doc lengths of the corpus and of the delta as rings, a copy plan and a
// scratch delta.  One call runs three launches on the caller's stream:
//
//  k_ingest_plan  (one thread) replays the reference's decisions document
//    by document.  The documents of the delta at the call and the ones the
//    call appends form one sequence; drops and snapshots only ever take
//    its oldest documents, so at the end the delta is a suffix of the
//    sequence and a snapshot (at most one per call: it stays in flight
//    until the host swaps it in) a contiguous run of it.  The plan is a
//    list of segments: the kept corpus range and the delta part of a
//    snapshot into the staging corpus, PAD after them, the surviving delta
//    and each appended document (with its separator) into the delta.
//  k_ingest_move  copies the segments, a flat index space over all of them
//    split across the grid.  The old delta is only read here.
//  k_ingest_commit copies the scratch delta over the delta when its old
//    part moved, and stores the new length in the index's delta_len word.
//
// A rebuild that is running when the reference's append_documents polls
// (global_index.py:111,140) may or may not have finished; here it has not:
// it finishes when the host swaps it in (sfx_ingest_swapped), and the host
// starts the build of a staged snapshot from its next poll.  Both are
// schedules the reference can take.

#include <hip/hip_runtime.h>

#include "launch.h"
#include "sfx_common.h"

namespace sfx {

struct IngestSeg {
  int64_t flat;     // first flat index of the segment
  int64_t src_off;  // element offset in the source
  int64_t dst_off;  // element offset in the destination
  int32_t n_src;    // elements read from the source
  int32_t len;      // elements written (n_src, + 1 with the separator)
  int32_t src;      // kSrc*
  int32_t dst;      // kDst*
};
static_assert(sizeof(IngestSeg) == 40, "segment layout");

constexpr int32_t kSrcCorpus = 0, kSrcDelta = 1, kSrcRows = 2, kSrcPad = 3;
constexpr int32_t kDstStaging = 0, kDstScratch = 1, kDstDelta = 2;
constexpr int kIngestFixedSegs = 4;
constexpr int64_t kIngestMaxSegs = SFX_INGEST_MAX_DOCS + kIngestFixedSegs;

// Private plan fields after the public header.
struct IngestPlan {
  int64_t nseg;         // segments of the last call
  int64_t flat_total;   // elements the move writes
  int64_t scratch_len;  // delta elements staged in scratch (0: in place)
  int64_t final_len;    // delta length after the call
  int64_t pad[12];
};
static_assert(sizeof(IngestPlan) == 128, "plan block");

struct IngestLayout {
  int64_t acap, dcap;  // ring slots
  int64_t plan, segs, aring, dring, scratch, total;  // byte offsets
};

__host__ __device__ inline int64_t ing_align(int64_t x) {
  return (x + 255) & ~(int64_t)255;
}

__host__ __device__ inline IngestLayout ingest_layout(int64_t N, int64_t D) {
  IngestLayout L;
  L.acap = N / 2 + 2;  // every document holds at least one token and SEP
  L.dcap = D / 2 + 2;
  int64_t off = ing_align((int64_t)sizeof(sfx_ingest_header));
  L.plan = off;
  off = ing_align(off + (int64_t)sizeof(IngestPlan));
  L.segs = off;
  off = ing_align(off + kIngestMaxSegs * (int64_t)sizeof(IngestSeg));
  L.aring = off;
  off = ing_align(off + L.acap * 4);
  L.dring = off;
  off = ing_align(off + L.dcap * 4);
  L.scratch = off;
  off = ing_align(off + D * 4);
  L.total = off;
  return L;
}

struct IngestArgs {
  unsigned char* state;
  int64_t N, D;           // corpus and delta capacity
  const int32_t* corpus;  // live corpus
  int32_t* staging;       // staging corpus
  int32_t* delta;
  int64_t* delta_len;     // the index's device length word
  const int32_t* tokens;  // [rows, seq]
  int64_t rows, seq;
  const void* row_idx;
  int32_t row_is64;
  const void* lengths;
  int32_t len_is64;
  int64_t ndocs;
  int64_t threshold;      // rebuild_threshold
  // ingest_active (active != 0): row_idx holds slot keys, document i is
  // tokens[i, ...], and ingested[nslots] the tokens taken per slot so far
  int32_t active, final;
  int64_t* ingested;
  int64_t nslots, chunk, overlap;
};

__device__ __forceinline__ int64_t ld_idx(const void* p, int is64,
                                          int64_t i) {
  return is64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

// ---------------------------------------------------------------- plan
__global__ void k_ingest_plan(IngestArgs a) {
  if (threadIdx.x != 0) return;
  const IngestLayout L = ingest_layout(a.N, a.D);
  sfx_ingest_header* h = reinterpret_cast<sfx_ingest_header*>(a.state);
  IngestPlan* q = reinterpret_cast<IngestPlan*>(a.state + L.plan);
  IngestSeg* seg = reinterpret_cast<IngestSeg*>(a.state + L.segs);
  int32_t* aring = reinterpret_cast<int32_t*>(a.state + L.aring);
  int32_t* dring = reinterpret_cast<int32_t*>(a.state + L.dring);
  const int64_t N = a.N, D = a.D;

  int64_t active_len = h->active_len;
  int64_t delta_len = h->delta_len;
  int64_t a_head = h->active_head, a_cnt = h->active_docs;
  int64_t d_head = h->delta_head, d_cnt = h->delta_docs;
  int64_t in_flight = h->in_flight;
  // The sequence: the delta's documents at the call (old, indices
  // < old_cnt, at delta[0, old_len) in order), then the appended ones.
  // The delta holds [F, T); old_tok = old-document tokens before F.
  const int64_t old_cnt = d_cnt, old_len = delta_len;
  int64_t F = 0, T = old_cnt, old_tok = 0;
  int64_t nk = 0;  // appended documents (segment k describes number k)
  // snapshot of this call
  bool snap = false;
  int64_t Fs = 0, sa = 0, s_old_off = 0, s_old_len = 0, keep_start = 0,
          n_keep = 0, n_new = 0;
  int64_t dropped_docs = 0, dropped_tok = 0, bad = 0;
  // the reference calls append_documents (and so maybe_rebuild) only when
  // the call yields a document, even an empty one (proposer.py:349-352,
  // 387-390)
  bool any_doc = false;

  auto pop_delta = [&]() -> int64_t {  // the oldest delta document
    const int64_t ln = dring[d_head];
    d_head = d_head + 1 == L.dcap ? 0 : d_head + 1;
    --d_cnt;
    if (F < old_cnt) old_tok += ln;
    ++F;
    return ln;
  };
  auto launch_rebuild = [&]() {  // global_index.py:147-215 (snapshot)
    if (in_flight) return;
    // eviction of the oldest whole corpus documents (:150-157)
    int64_t ks = 0, ev = 0;
    while (ev < a_cnt && active_len - ks + delta_len > N) {
      int64_t slot = a_head + ev;
      if (slot >= L.acap) slot -= L.acap;
      ks += aring[slot];
      ++ev;
    }
    const int64_t nk_tok = active_len - ks;
    const int64_t lim = delta_len < N - nk_tok ? delta_len : N - nk_tok;
    int64_t acc = 0, na = 0;  // whole delta documents (:158-167)
    while (na < d_cnt) {
      int64_t slot = d_head + na;
      if (slot >= L.dcap) slot -= L.dcap;
      const int64_t ln = dring[slot];
      if (acc + ln > lim) break;
      acc += ln;
      ++na;
    }
    if (nk_tok + acc == 0) return;  // nothing to build (:170-171)
    snap = true;
    Fs = F;
    sa = na;
    keep_start = ks;
    n_keep = nk_tok;
    n_new = nk_tok + acc;
    s_old_off = old_tok;
    // corpus ring: drop the evicted documents, append the absorbed ones
    a_head += ev;
    if (a_head >= L.acap) a_head -= L.acap;
    a_cnt -= ev;
    for (int64_t i = 0; i < na; ++i) {
      const int64_t f0 = F;
      const int64_t ln = pop_delta();
      if (f0 < old_cnt) s_old_len += ln;
      int64_t slot = a_head + a_cnt;
      if (slot >= L.acap) slot -= L.acap;
      aring[slot] = (int32_t)ln;
      ++a_cnt;
    }
    active_len = n_new;
    delta_len -= acc;
    in_flight = 1;
  };
  auto drop_oldest = [&](int64_t drop) {  // global_index.py:120-133
    int64_t acc = 0;
    while (d_cnt > 0 && acc < drop) {
      const int64_t ln = pop_delta();
      acc += ln;
      ++dropped_docs;
    }
    dropped_tok += acc;
    delta_len -= acc;
  };

  for (int64_t i = 0; i < a.ndocs; ++i) {  // global_index.py:86-108
    int64_t r, start, n;
    if (!a.active) {
      // harvest_finished / harvest_rows (proposer.py:329-352):
      // token_ids_gpu[r][:ln] for ln > 0, r a Python index (negative
      // counts from the end; outside [-rows, rows) the reference raises,
      // here the row is skipped and counted)
      r = ld_idx(a.row_idx, a.row_is64, i);
      if (r < -a.rows || r >= a.rows) {
        ++bad;
        continue;
      }
      if (r < 0) r += a.rows;
      const int64_t ln = ld_idx(a.lengths, a.len_is64, i);
      if (ln <= 0) continue;
      any_doc = true;
      start = 0;
      n = ln < a.seq ? ln : a.seq;
    } else {
      // ingest_active (proposer.py:354-390): a slot emits row[start:ln]
      // once ln - done >= chunk (or, when final, anything new), start =
      // max(0, done - overlap), as a Python slice of the row; final
      // forgets the slot (done reads 0 again)
      const int64_t key = ld_idx(a.row_idx, a.row_is64, i);
      if (key < 0 || key >= a.nslots) {
        ++bad;
        continue;
      }
      const int64_t ln = ld_idx(a.lengths, a.len_is64, i);
      const int64_t done = a.ingested[key];
      r = i;
      start = 0;
      n = 0;
      if (ln - done >= a.chunk || (a.final && ln > done)) {
        int64_t st = done - a.overlap;
        st = st < 0 ? 0 : (st > a.seq ? a.seq : st);
        const int64_t stop = ln < 0 ? (a.seq + ln > 0 ? a.seq + ln : 0)
                                    : (ln < a.seq ? ln : a.seq);
        start = st;
        n = stop > st ? stop - st : 0;
        a.ingested[key] = ln;
        any_doc = true;
      }
      if (a.final) a.ingested[key] = 0;
      if (n <= 0) continue;  // append_documents skips empty documents
    }
    if (n + 1 > D) {  // the last D - 1 tokens
      start += n - (D - 1);
      n = D - 1;
    }
    if (delta_len + n + 1 > D) {  // _make_room(n + 1)
      launch_rebuild();
      if (delta_len + n + 1 > D) drop_oldest(delta_len + n + 1 - D);
    }
    IngestSeg s;
    s.flat = 0;
    s.src_off = r * a.seq + start;
    s.dst_off = -1;
    s.n_src = (int32_t)n;
    s.len = (int32_t)(n + 1);
    s.src = kSrcRows;
    s.dst = -1;
    seg[nk++] = s;
    int64_t slot = d_head + d_cnt;
    if (slot >= L.dcap) slot -= L.dcap;
    dring[slot] = (int32_t)(n + 1);
    ++d_cnt;
    ++T;
    delta_len += n + 1;
  }
  // maybe_rebuild (global_index.py:138-145)
  if (any_doc && !in_flight && delta_len != 0 && delta_len >= a.threshold)
    launch_rebuild();

  // ---- destinations.  Final delta: [F, T); snapshot: [Fs, Fs + sa).
  const int64_t Ff = F;
  const bool moved = Ff > 0;  // the old part (or nothing) moves down
  int64_t fin_old_len = Ff < old_cnt ? old_len - old_tok : 0;
  int64_t s_pos = n_keep + s_old_len;  // next staging slot of the snapshot
  int64_t d_pos = fin_old_len;         // next delta slot
  for (int64_t k = 0; k < nk; ++k) {
    const int64_t c = old_cnt + k;
    IngestSeg& s = seg[k];
    if (snap && c >= Fs && c < Fs + sa) {
      s.dst = kDstStaging;
      s.dst_off = s_pos;
      s_pos += s.len;
    } else if (c >= Ff) {
      s.dst = moved ? kDstScratch : kDstDelta;
      s.dst_off = d_pos;
      d_pos += s.len;
    } else {
      s.len = 0;  // dropped before it was written
      s.dst = kDstDelta;
      s.dst_off = 0;
    }
  }
  int64_t ns = nk;
  auto add = [&](int32_t src, int64_t src_off, int32_t dst, int64_t dst_off,
                 int64_t len) {
    IngestSeg s;
    s.flat = 0;
    s.src_off = src_off;
    s.dst_off = dst_off;
    s.n_src = (int32_t)len;
    s.len = (int32_t)len;
    s.src = src;
    s.dst = dst;
    seg[ns++] = s;
  };
  // (lengths of up to N elements fit int32: N < 2^31)
  if (snap) {
    add(kSrcCorpus, keep_start, kDstStaging, 0, n_keep);
    add(kSrcDelta, s_old_off, kDstStaging, n_keep, s_old_len);
    add(kSrcPad, 0, kDstStaging, n_new, N - n_new);
  }
  if (moved && fin_old_len > 0)
    add(kSrcDelta, old_tok, kDstScratch, 0, fin_old_len);
  int64_t flat = 0;
  for (int64_t k = 0; k < ns; ++k) {
    seg[k].flat = flat;
    flat += seg[k].len;
  }
  q->nseg = ns;
  q->flat_total = flat;
  q->scratch_len = moved ? delta_len : 0;
  q->final_len = delta_len;

  h->active_len = active_len;
  h->delta_len = delta_len;
  h->active_head = a_head;
  h->active_docs = a_cnt;
  h->delta_head = d_head;
  h->delta_docs = d_cnt;
  if (snap) {
    h->in_flight = 1;
    h->snap_seq += 1;
    h->snap_n_new = n_new;
    h->snap_m = n_new + 1 < N ? n_new + 1 : N;
  }
  h->docs_in += nk;
  h->docs_dropped += dropped_docs;
  h->tokens_dropped += dropped_tok;
  h->bad_rows += bad;
}

// ---------------------------------------------------------------- move
constexpr int kMoveThreads = 256;
constexpr int64_t kMoveChunk = 4096;  // flat elements per block and pass

__global__ __launch_bounds__(kMoveThreads) void k_ingest_move(IngestArgs a) {
  const IngestLayout L = ingest_layout(a.N, a.D);
  const IngestPlan* q = reinterpret_cast<const IngestPlan*>(a.state + L.plan);
  const IngestSeg* seg =
      reinterpret_cast<const IngestSeg*>(a.state + L.segs);
  int32_t* scratch = reinterpret_cast<int32_t*>(a.state + L.scratch);
  const int64_t total = q->flat_total;
  const int64_t ns = q->nseg;
  __shared__ int64_t s0;
  for (int64_t base = (int64_t)blockIdx.x * kMoveChunk; base < total;
       base += (int64_t)gridDim.x * kMoveChunk) {
    __syncthreads();
    if (threadIdx.x == 0) {  // last segment starting at or before base
      int64_t lo = 0, hi = ns - 1;
      while (lo < hi) {
        const int64_t mid = (lo + hi + 1) / 2;
        if (seg[mid].flat <= base)
          lo = mid;
        else
          hi = mid - 1;
      }
      s0 = lo;
    }
    __syncthreads();
    int64_t s = s0;
    const int64_t end = base + kMoveChunk < total ? base + kMoveChunk : total;
    for (int64_t f = base + threadIdx.x; f < end; f += kMoveThreads) {
      while (s + 1 < ns && seg[s + 1].flat <= f) ++s;
      const IngestSeg& g = seg[s];
      const int64_t j = f - g.flat;
      int32_t v;
      if (j >= g.n_src)
        v = -2;  // SEP_TOKEN after an appended document
      else if (g.src == kSrcCorpus)
        v = a.corpus[g.src_off + j];
      else if (g.src == kSrcDelta)
        v = a.delta[g.src_off + j];
      else if (g.src == kSrcRows)
        v = a.tokens[g.src_off + j];
      else
        v = kPad;
      int32_t* dst = g.dst == kDstStaging   ? a.staging
                     : g.dst == kDstScratch ? scratch
                                            : a.delta;
      dst[g.dst_off + j] = v;
    }
  }
}

__global__ __launch_bounds__(kMoveThreads) void k_ingest_commit(
    IngestArgs a) {
  const IngestLayout L = ingest_layout(a.N, a.D);
  const IngestPlan* q = reinterpret_cast<const IngestPlan*>(a.state + L.plan);
  const int32_t* scratch =
      reinterpret_cast<const int32_t*>(a.state + L.scratch);
  const int64_t n = q->scratch_len;
  for (int64_t i = (int64_t)blockIdx.x * kMoveThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kMoveThreads)
    a.delta[i] = scratch[i];
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.delta_len = q->final_len;
}

__global__ void k_ingest_swapped(unsigned char* state) {
  if (threadIdx.x != 0) return;
  sfx_ingest_header* h = reinterpret_cast<sfx_ingest_header*>(state);
  h->in_flight = 0;
  h->live_active_len = h->active_len;
}

}  // namespace sfx

using namespace sfx;

extern "C" int sfx_ingest_layout(int64_t capacity, int64_t delta_capacity,
                                 int64_t* out) {
  if (!out || capacity < 1 || capacity > 0x7fffffffLL || delta_capacity < 1 ||
      delta_capacity > 0x7fffffffLL)
    return SFX_EINVAL;
  const IngestLayout L = ingest_layout(capacity, delta_capacity);
  out[0] = L.total;
  out[1] = L.acap;
  out[2] = L.dcap;
  out[3] = L.aring;
  out[4] = L.dring;
  out[5] = L.scratch;
  return 0;
}

namespace {

bool ingest_geometry_ok(const void* state, const int32_t* corpus,
                        int64_t capacity, const int32_t* delta,
                        int64_t delta_capacity, const int64_t* delta_len,
                        const int32_t* staging_corpus, const int32_t* tokens,
                        int64_t rows, int64_t seq, const void* row_idx,
                        const void* lengths, int64_t ndocs) {
  return state && corpus && delta && delta_len && staging_corpus &&
         ndocs >= 0 && ndocs <= SFX_INGEST_MAX_DOCS && capacity >= 1 &&
         capacity <= 0x7fffffffLL && delta_capacity >= 1 &&
         delta_capacity <= 0x7fffffffLL &&
         !(ndocs > 0 && (!tokens || !row_idx || !lengths || rows < 1 ||
                         seq < 1 || rows > (INT64_MAX / seq))) &&
         !((uintptr_t)state & 255);
}

IngestArgs ingest_args(void* state, const int32_t* corpus, int64_t capacity,
                       int32_t* delta, int64_t delta_capacity,
                       int64_t* delta_len, int32_t* staging_corpus,
                       const int32_t* tokens, int64_t rows, int64_t seq,
                       const void* row_idx, int32_t row_idx_is64,
                       const void* lengths, int32_t lengths_is64,
                       int64_t ndocs, int64_t rebuild_threshold) {
  IngestArgs a;
  a.state = (unsigned char*)state;
  a.N = capacity;
  a.D = delta_capacity;
  a.corpus = corpus;
  a.staging = staging_corpus;
  a.delta = delta;
  a.delta_len = delta_len;
  a.tokens = tokens;
  a.rows = rows;
  a.seq = seq;
  a.row_idx = row_idx;
  a.row_is64 = row_idx_is64 ? 1 : 0;
  a.lengths = lengths;
  a.len_is64 = lengths_is64 ? 1 : 0;
  a.ndocs = ndocs;
  a.threshold = rebuild_threshold;
  a.active = 0;
  a.final = 0;
  a.ingested = nullptr;
  a.nslots = 0;
  a.chunk = 0;
  a.overlap = 0;
  return a;
}

int ingest_launch(const IngestArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(k_ingest_plan, dim3(1), dim3(64), 0, stream, a);
  hipLaunchKernelGGL(k_ingest_move, dim3(1024), dim3(kMoveThreads), 0,
                     stream, a);
  hipLaunchKernelGGL(k_ingest_commit, dim3(64), dim3(kMoveThreads), 0,
                     stream, a);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" int sfx_ingest_docs(void* state, const int32_t* corpus,
                               int64_t capacity, int32_t* delta,
                               int64_t delta_capacity, int64_t* delta_len,
                               int32_t* staging_corpus, const int32_t* tokens,
                               int64_t rows, int64_t seq,
                               const void* row_idx, int32_t row_idx_is64,
                               const void* lengths, int32_t lengths_is64,
                               int64_t ndocs, int64_t rebuild_threshold,
                               hipStream_t stream) {
  if (!ingest_geometry_ok(state, corpus, capacity, delta, delta_capacity,
                          delta_len, staging_corpus, tokens, rows, seq,
                          row_idx, lengths, ndocs))
    return SFX_EINVAL;
  return ingest_launch(
      ingest_args(state, corpus, capacity, delta, delta_capacity, delta_len,
                  staging_corpus, tokens, rows, seq, row_idx, row_idx_is64,
                  lengths, lengths_is64, ndocs, rebuild_threshold),
      stream);
}

extern "C" int sfx_ingest_active(void* state, const int32_t* corpus,
                                 int64_t capacity, int32_t* delta,
                                 int64_t delta_capacity, int64_t* delta_len,
                                 int32_t* staging_corpus,
                                 const int32_t* tokens, int64_t rows,
                                 int64_t seq, const void* keys,
                                 int32_t keys_is64, const void* lengths,
                                 int32_t lengths_is64, int64_t ndocs,
                                 int64_t* ingested, int64_t nslots,
                                 int32_t final, int64_t chunk,
                                 int64_t overlap, int64_t rebuild_threshold,
                                 hipStream_t stream) {
  if (!ingest_geometry_ok(state, corpus, capacity, delta, delta_capacity,
                          delta_len, staging_corpus, tokens, rows, seq, keys,
                          lengths, ndocs) ||
      (ndocs > 0 && (!ingested || nslots < 1 || rows < ndocs)))
    return SFX_EINVAL;
  IngestArgs a =
      ingest_args(state, corpus, capacity, delta, delta_capacity, delta_len,
                  staging_corpus, tokens, rows, seq, keys, keys_is64,
                  lengths, lengths_is64, ndocs, rebuild_threshold);
  a.active = 1;
  a.final = final ? 1 : 0;
  a.ingested = ingested;
  a.nslots = nslots;
  a.chunk = chunk;
  a.overlap = overlap;
  return ingest_launch(a, stream);
}

extern "C" int sfx_ingest_swapped(void* state, hipStream_t stream) {
  if (!state || ((uintptr_t)state & 255)) return SFX_EINVAL;
  hipLaunchKernelGGL(k_ingest_swapped, dim3(1), dim3(64), 0, stream,
                     (unsigned char*)state);
  return (int)hipGetLastError();
}
