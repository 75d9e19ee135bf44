/*
 * suffixgpu_amd -- C ABI of the MI355X (gfx950) SuffixGPU drafter kernels.
 *
 * Every entry point takes device pointers, plain integer sizes and a
 * hipStream_t, enqueues work on that stream and returns without waiting.
 * None of them allocates device or host memory or synchronises.  Scratch
 * memory is a caller-provided workspace whose size the matching
 * *_workspace_size() function reports; the one exception,
 * sfx_propose_step_noalloc, keeps its scratch in a static device array.
 * Workspaces of the fused step must be zero-filled once when allocated;
 * the kernels leave them zeroed again at the end of every call.
 *
 * Return value: 0 on success, SFX_EINVAL (-1) for an argument the kernels
 * cannot accept (reported before anything is enqueued), otherwise the
 * hipError_t of the failing launch.
 *
 * Token contract (as in the reference): buffer tokens are int32 in
 * [0, INT32_MAX).  -1 pads, -2 (SEP) separates documents in the global
 * corpus, INT32_MAX (PAD) fills the corpus past its end.
 */
#ifndef SUFFIXGPU_AMD_H
#define SUFFIXGPU_AMD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SFX_EINVAL (-1)
#define SFX_MAX_CANDIDATES 32
#define SFX_ABI_VERSION 15

/* Drafter configuration shared by the local and global paths.
 * Mirrors the constructor arguments of SuffixGPUDrafter
 * (suffix_gpu/proposer.py:33-108) and LocalMatchKernel
 * (suffix_gpu/local_matcher.py:52-74). */
typedef struct sfx_params {
    int32_t k;               /* draft length K = chain depth              */
    int32_t max_pattern_len; /* P (<= 255)                               */
    int32_t max_occurrences; /* R (<= 2048)                              */
    int32_t min_match_len;   /* already max(1, min_match_len)            */
    int32_t num_thresholds;  /* C_l: local support thresholds            */
    int32_t num_caps;        /* C_g: global length caps (0: local only)  */
    int32_t has_spec_factor; /* 0: emission cap = k                      */
    float spec_factor;       /* max_spec_factor (as fp32)                */
    float spec_offset;       /* max_spec_offset (as fp32)                */
    float min_token_prob;    /* as fp32                                  */
    float alpha;             /* vote_smoothing_alpha (as fp32)           */
    int32_t thresholds[SFX_MAX_CANDIDATES]; /* local support thresholds */
    int32_t caps[SFX_MAX_CANDIDATES];       /* global caps, descending  */
} sfx_params;

/* Global index buffers (suffix_gpu/global_index.py:63-74), plus the key
 * array of the suffix array (no reference counterpart): row r holds the
 * first key_width tokens of the suffix at sa[r] (-1 past the end), built
 * by sfx_sa_keys() with every suffix array; NULL disables it.
 *
 * With key_select != NULL the kernels read the device word *key_select
 * when they run and take sa_key_alt and gram_alt when it is nonzero, sa_key
 * and gram otherwise; a NULL second buffer means none (the search then
 * compares through sa and corpus, exact and slower).  Double buffers let a
 * rebuild write the idle pair and sfx_index_swap() flip the word; single
 * buffers let the swap set the word while the new array's key rows and
 * table are written, and a later sfx_index_swap() with capacity 0 clear
 * it.  Either way graphs captured over this struct follow the word. */
typedef struct sfx_index {
    const int32_t* corpus;    /* [capacity] PAD-filled ring               */
    const int32_t* sa;        /* [capacity] suffix array of corpus        */
    int64_t capacity;         /* N                                        */
    const int32_t* delta;     /* [delta_capacity] append-only delta       */
    int64_t delta_capacity;   /* D                                        */
    const int64_t* delta_len; /* device scalar: committed delta length    */
    const int32_t* sa_key;    /* [capacity, key_width] or NULL; 16-byte
                                 aligned                                 */
    int64_t key_width;        /* 4..32, a multiple of 4                   */
    const int32_t* sa_key_alt; /* second key-row buffer (same layout) or
                                  NULL (none while selected)             */
    const int32_t* key_select; /* device int32 selecting sa_key_alt and
                                  gram_alt when nonzero, or NULL (sa_key
                                  and gram are live)                     */
    const void* gram;          /* n-gram range table of sa_key's suffix
                                  array (sfx_gram_build), or NULL         */
    const void* gram_alt;      /* the table of sa_key_alt's, or NULL      */
    int64_t gram_slots;        /* slots per table, a multiple of 16      */
    const int32_t* delta_entries; /* delta token index of the live delta
                                     (sfx_delta_index_build), 16-byte
                                     aligned, or NULL: each decode row then
                                     scans the delta                     */
    const uint32_t* delta_start;  /* [delta_buckets + 1] its bucket starts */
    int64_t delta_buckets;       /* a power of two, 2^10 .. 2^17          */
} sfx_index;

/* One decode step's batch (suffix_gpu/proposer.py:135-214).
 * sampled == NULL means propose() without a state update; then `mask`
 * (optional bool [B]) selects the drafting rows. */
typedef struct sfx_batch {
    int32_t* tokens;          /* [B,S] resident token rows (updated)      */
    int64_t batch;            /* B                                        */
    int64_t seq;              /* S                                        */
    const void* num_tokens;   /* [B] committed counts, int32 or int64     */
    int32_t num_tokens_is64;
    const int32_t* sampled;   /* [B,T] last step's ids, -1 padded, or NULL */
    int64_t num_sampled;      /* T                                        */
    const void* valid_count;  /* [B] optional count, int32 or int64       */
    int32_t valid_count_is64;
    const uint8_t* mask;      /* [B] optional rows allowed to draft       */
    int64_t limit;            /* length limit: S or min(max_model_len, S) */
} sfx_batch;

int sfx_abi_version(void);

/* ---- reference operator boundary (suffix_gpu/triton_kernels.py) ------- */

/* triton_kernels.py:392-402 scatter_append + proposer.py:162-184:
 * tokens[b, base+j] = sampled[b, j] for j < cnt, sampled != -1, base+j < S;
 * new_counts[b] = base + cnt (cnt = #(sampled != -1) when valid_count is
 * NULL).  new_counts may be NULL. */
int sfx_scatter_append(const sfx_batch* batch, int32_t* new_counts,
                       hipStream_t stream);

/* triton_kernels.py:259-281 match_back: out[b,i] = number of leading t < P
 * with x(i-1-t) == pat[b,t], x(j) = src[b*row_stride + j] (j >= 0) else -1.
 * row_stride 0 shares one 1-D source (the delta). */
int sfx_match_back(const int32_t* src, int64_t row_stride,
                   const int32_t* pat, int64_t batch, int64_t pattern_len,
                   int64_t n_out, int32_t* out, hipStream_t stream);

/* triton_kernels.py:362-389 first_occurrences: the first R ascending
 * columns with mb[b, i] >= thr[b*C + c] (thr > 0), zero padded; count
 * clamped to R. */
int sfx_first_occurrences(const int32_t* mb, int64_t n_cols,
                          const int64_t* thr, int64_t rows, int64_t per_row,
                          int64_t max_occ, int64_t* pos, int64_t* count,
                          hipStream_t stream);

/* triton_kernels.py:284-302 sa_search / sa_search.py:66-107: exact lower
 * and upper bounds of each pattern (row-major [B, M], plen[b] valid) among
 * the suffixes listed by sa; a corpus read at or past n compares as -1.
 * 1 <= n < 2^31. */
int sfx_sa_search(const int32_t* sa, const int32_t* corpus, int64_t n,
                  const int32_t* pattern, int64_t batch, int64_t width,
                  const int64_t* plen, int64_t* lower, int64_t* upper,
                  hipStream_t stream);

/* triton_kernels.py:305-338 expand_chain / expand.py:59-147: depth-wise
 * majority vote with fp32 chain-probability scoring.  weights may be NULL
 * (unit votes); cap may be NULL (cap = K). */
int sfx_expand_chain(const int32_t* cont, int64_t rows, int64_t max_occ,
                     int64_t k, const int64_t* num_occ, const int64_t* cap,
                     const float* weights, float min_token_prob, float alpha,
                     int32_t* chain, int64_t* num_valid, int64_t* num_emit,
                     float* score, hipStream_t stream);

/* ---- local path (suffix_gpu/local_matcher.py) ------------------------- */

/* local_matcher.py:83-196 gather_candidates: cand [B,C_l] i64,
 * cont [B,C_l,R,K] i32, occ [B,C_l] i64.  Any output may be NULL. */
int sfx_local_gather(const sfx_params* p, const sfx_batch* batch,
                     int64_t* cand, int32_t* cont, int64_t* occ,
                     hipStream_t stream);

/* local_matcher.py:198-242 forward: draft [B,K] i32 (padded past the
 * emission count), num_valid [B] i32, match_len [B] i64, occ [B] i64,
 * score [B] f32.  Outputs other than draft/num_valid may be NULL. */
int sfx_local_forward(const sfx_params* p, const sfx_batch* batch,
                      int32_t* draft, int32_t* num_valid, int64_t* match_len,
                      int64_t* occ, float* score, hipStream_t stream);

/* ---- global path (suffix_gpu/global_index.py, sa_search.py) ----------- */

/* Queries are newest-last tails: query [B,Q] i32 with qlen [B] i64
 * (global_index.py:286-370 _query_backoff, :465-546 _delta_match_backoff,
 * sa_search.py:110-163 suffix_match_backoff, global_index.py:372-441
 * draft).  Every output may be NULL:
 *   sa_len/sa_start/sa_end  [B,C_g] i64  suffix_match_backoff
 *   d_len/d_pos/d_cnt       [B,C_g] i64, [B,C_g,R] i64, [B,C_g] i64
 *   len/cont/occ            [B,C_g] i64, [B,C_g,R,K] i32, [B,C_g] i64
 *   draft/emit/dlen/docc/dscore  best-cap draft: [B,K] i32, [B] i64 x3,
 *                                [B] f32
 * workspace: sfx_global_query_workspace_size() bytes, zero-filled once
 * (its size depends on the index's delta capacity; 0 for local-only). */
typedef struct sfx_global_out {
    int64_t* sa_len; int64_t* sa_start; int64_t* sa_end;
    int64_t* d_len; int64_t* d_pos; int64_t* d_cnt;
    int64_t* len; int32_t* cont; int64_t* occ;
    int32_t* draft; int64_t* emit; int64_t* draft_len; int64_t* draft_occ;
    float* draft_score;
} sfx_global_out;

size_t sfx_global_query_workspace_size(const sfx_params* p, int64_t batch,
                                       int64_t delta_capacity);
int sfx_global_query(const sfx_params* p, const sfx_index* index,
                     const int32_t* query, int64_t batch, int64_t width,
                     const int64_t* qlen, const sfx_global_out* out,
                     void* workspace, size_t workspace_bytes,
                     hipStream_t stream);

/* ---- fused decode step (suffix_gpu/proposer.py:186-327) --------------- */

/* propose_with_update (batch->sampled != NULL) or propose (== NULL), one
 * kernel launch on `stream`.  Local-only when index == NULL.  With an
 * index, every row runs an SA-search, a delta-scan and a local workgroup
 * that hand results over through the workspace; whichever finishes a row
 * last writes that row's draft [B,K] i32 and num_valid [B] i32.
 * new_counts [B] i32 may be NULL.  workspace: sfx_step_workspace_size()
 * bytes (0 for local-only), zero-filled once; calls sharing a workspace
 * must not overlap. */
size_t sfx_step_workspace_size(const sfx_params* p, int64_t batch,
                               int64_t delta_capacity);
int sfx_propose_step(const sfx_params* p, const sfx_index* index,
                     const sfx_batch* batch, int32_t* draft,
                     int32_t* num_valid, int32_t* new_counts,
                     void* workspace, size_t workspace_bytes,
                     hipStream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): sfx_propose_step with no workspace argument.  The
 * step's scratch is a static device array of SFX_NOALLOC_SCRATCH_BYTES
 * bytes that every GPU the library runs on holds until the process ends;
 * the call allocates nothing.  A batch of more than SFX_NOALLOC_MAX_ROWS
 * rows, or one whose step needs more scratch than the array holds (large
 * delta capacities with many rows), returns SFX_ENOSCRATCH before anything
 * is enqueued.  Every call on one GPU shares that GPU's array: calls that
 * overlap on a GPU (from two streams, or concurrent replays of graphs that
 * hold this call) race and corrupt each other's drafts.  `stream` must
 * belong to the device current on the calling thread. */
#define SFX_ENOSCRATCH (-2)
#define SFX_NOALLOC_SCRATCH_BYTES 16777216 /* 16 MiB */
#define SFX_NOALLOC_MAX_ROWS 4096
int sfx_propose_step_noalloc(const sfx_params* p, const sfx_index* index,
                             const sfx_batch* batch, int32_t* draft,
                             int32_t* num_valid, int32_t* new_counts,
                             hipStream_t stream);

/* ---- suffix-array rebuild (suffix_gpu/suffix_array.py:15-63,
 *      global_index.py:217-223) ------------------------------------------ */

/* sa[0:m] = suffix array of text[0:m] (signed int32 order, a proper prefix
 * first); sa[m:n_total] = m .. n_total-1.  Prefix doubling: each round
 * re-sorts only the suffixes whose group is not yet a singleton (inside a
 * workgroup for a group of at most 2048, by LSD radix sorts for a larger
 * one), and the rounds stop on the device once none is left, with no host
 * synchronisation.  sa_is64 selects int64 output. */
size_t sfx_sa_build_workspace_size(int64_t m);

/* keys[r * width + j] = j-th token of the suffix at sa[r] (corpus reads at
 * or past n give -1), for r < rows <= n and j < width (4..32, multiple of
 * 4); when first4 (16-byte aligned) is not NULL, first4[r * 4 + j] holds
 * the same for j < 4, a compact input for sfx_gram_build (key_width 4).
 * A rebuild whose ranks from some r on are the padding suffixes of the
 * previous build in the same buffer rewrites only the rows below. */
int sfx_sa_keys(const int32_t* corpus, const int32_t* sa, int64_t n,
                int64_t rows, int64_t width, int32_t* keys, int32_t* first4,
                hipStream_t stream);
int sfx_sa_build(const int32_t* text, int64_t m, int64_t n_total, void* sa,
                 int32_t sa_is64, void* workspace, size_t workspace_bytes,
                 hipStream_t stream);

/* No reference counterpart.  The n-gram range table of a suffix array:
 * for every distinct run of the first k tokens (k = 1..4, real tokens
 * only) among the sorted suffixes, the rank range of the suffixes that
 * start with it, so that an interval search starts inside the range of its
 * pattern's first tokens.  `table` (256-byte aligned, sfx_gram_table_bytes
 * bytes for `slots` slots, a multiple of 16 in buckets of 16, 24 bytes a
 * slot) is rebuilt in place from the key rows (key_width 4..32, 16-byte
 * aligned) of
 * ranks 0..m-1, enqueued on `stream` with no host read; it needs no
 * initial contents (a zero-filled table reads as unusable).  The build
 * counts the distinct runs of each length and stores those of 1..k
 * tokens for the largest k whose runs fill at most 3/4 of the slots; the
 * table's first word then holds the longest length all of whose runs are
 * stored (0..4; 0 if an insert of a 1-token run found no room), and
 * searches look up at most that many leading tokens. */
size_t sfx_gram_table_bytes(int64_t slots);
int sfx_gram_build(const int32_t* keys, int64_t key_width, int64_t m,
                   void* table, int64_t slots, hipStream_t stream);

/* No reference counterpart.  The delta token index: entries[0 .. D), four
 * int32 each {q, x(q), x(q - 1), x(q - 2)} (x = -1 before position 0),
 * hold the delta positions q = 0 .. *delta_len - 1 grouped by a hash
 * bucket of their token x(q) (delta_bucket: Fibonacci hashing into
 * `buckets`, a power of two from 2^10 to 2^17), ascending within a
 * bucket, followed by the positions past the live length; start[b]
 * (b = 0 .. buckets) is the first entry of bucket b, so bucket b spans
 * entries[start[b] .. start[b + 1]).  A decode step given it
 * (sfx_index.delta_entries/delta_start/delta_buckets) visits only the
 * entries in its newest pattern token's bucket instead of scanning the
 * delta (global_index.py:465-546 computes the same match lengths over
 * every position).  Rebuild it, on the stream the delta is written on,
 * after every change to the delta or its length.  `entries` is 16-byte
 * aligned; `workspace` (256-byte aligned, sfx_delta_index_bytes(D) bytes)
 * holds nothing between calls.  Enqueued on `stream` with no host read. */
size_t sfx_delta_index_bytes(int64_t delta_capacity);
int sfx_delta_index_build(const int32_t* delta, const int64_t* delta_len,
                          int64_t delta_capacity, int32_t* entries,
                          uint32_t* start, int64_t buckets, void* workspace,
                          size_t workspace_bytes, hipStream_t stream);

/* The same build in steps, for a caller that advances it from a host poll
 * loop and stops enqueueing rounds once the array is final (no reference
 * counterpart; global_index.py:201-252 runs the build as one call):
 *   begin  -- the token round;
 *   rounds -- doubling rounds first .. first+count-1 (round r doubles
 *             h = h0 * 2^(r-1); rounds past sfx_sa_build_rounds_total(m)
 *             are skipped; a round after the array is final returns at
 *             once).  A round sorts its unsorted groups of at most
 *             sfx_sa_group_cap() suffixes inside workgroups (one launch)
 *             and its larger groups by radix launches, which are
 *             enqueued only when flags has SFX_SA_ROUNDS_RADIX.  Without
 *             it a round that has a larger group marks the build stalled
 *             at that round and every later launch returns; enqueueing
 *             rounds again from the stalled round with SFX_SA_ROUNDS_RADIX
 *             resumes the build.  SFX_SA_ROUNDS_EXPECT_FINAL tells the
 *             rounds that the caller expects the array to be final before
 *             them (a rebuild's margin rounds past the rounds the same
 *             text needed before): each of their launches reads the state
 *             words before its tile, so a round with nothing to do reads
 *             64 bytes per workgroup instead of 16 KB, and one with work
 *             starts a memory round trip later.  Results never depend on
 *             it.  Other flag bits are rejected (SFX_EINVAL);
 *   finish -- sa[0:m] from the workspace, sa[m:n_total] the identity.
 * The workspace's u32 state block at sfx_sa_build_flag_offset(m) (64
 * bytes to copy) holds [0] nonzero once the array is final, [2] the round
 * that found it final, [7] the round the build stalled at (0: none) and
 * [8] a mask with bit r set for every round r that ran radix launches,
 * for an asynchronous copy to the host.  sfx_sa_build enqueues the radix
 * launches for every round.  The first 16 * m bytes of the workspace carry
 * nothing from one launch of a build to the next (the radix key buffers):
 * between launches, e.g. after finish, a caller may use them, as the
 * first4 output of sfx_sa_keys. */
int sfx_sa_build_rounds_total(int64_t m);
int64_t sfx_sa_build_flag_offset(int64_t m);
/* The largest group a round sorts inside a workgroup (2048). */
int sfx_sa_group_cap(void);
int sfx_sa_build_begin(const int32_t* text, int64_t m, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);
#define SFX_SA_ROUNDS_RADIX 1
#define SFX_SA_ROUNDS_EXPECT_FINAL 2
int sfx_sa_build_rounds(int64_t m, int32_t first, int32_t count,
                        int32_t flags, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);
int sfx_sa_build_finish(int64_t m, int64_t n_total, void* sa, int32_t sa_is64,
                        void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* global_index.py:235-240 _finish_swap: in-place copy of a finished
 * rebuild into the live buffers (corpus, sa: capacity int32 each), one
 * launch, so graphs captured over the live buffers keep their pointers.
 * The key rows are not copied: when key_select is not NULL the same launch
 * stores key_select_value there (sfx_index.key_select picks the buffers
 * the steps read); capacity 0 stores only the word. */
int sfx_index_swap(int32_t* corpus, int32_t* sa, const int32_t* new_corpus,
                   const int32_t* new_sa, int64_t capacity,
                   int32_t* key_select, int32_t key_select_value,
                   hipStream_t stream);

/* ---- delta writes (global_index.py:86-133, 192-199) ------------------- */

/* One document to append: n tokens from src (device) to delta[dst ..
 * dst + n), followed by SEP (-2) at delta[dst + n]. */
typedef struct sfx_append_doc {
  const int32_t* src;
  int64_t n;
  int64_t dst;
} sfx_append_doc;

#define SFX_APPEND_MAX_DOCS 64

/* global_index.py:86-106 append_documents, the device side of it: the
 * host decides truncation, room and destinations, then appends any number
 * of documents (host array `docs`, one launch per SFX_APPEND_MAX_DOCS) and
 * sets *delta_len = new_len (device int64; skipped when NULL).  Every
 * document must end at or before delta_capacity - 1. */
int sfx_delta_append(const sfx_append_doc* docs, int32_t ndocs,
                     int32_t* delta, int64_t delta_capacity,
                     int64_t* delta_len, int64_t new_len, hipStream_t stream);

/* global_index.py:128-133, 194-199: drop the oldest delta documents or the
 * snapshot absorbed by a rebuild -- delta[0 .. n) = delta[from ..
 * from + n) in place -- and set *delta_len = n (skipped when NULL). */
int sfx_delta_shift(int32_t* delta, int64_t delta_capacity, int64_t from,
                    int64_t n, int64_t* delta_len, hipStream_t stream);

/* ---- device-side ingest (proposer.py:329-343 harvest_finished,
 *      global_index.py:86-215 append_documents through the rebuild
 *      snapshot) ---------------------------------------------------------- */

/* The state's header: the index's document bookkeeping, kept in device
 * memory.  The two doc-length lists (corpus documents oldest first, delta
 * documents oldest first) are rings of int32 lengths, separator included,
 * at the offsets sfx_ingest_layout reports. */
typedef struct sfx_ingest_header {
  int64_t active_len;      /* corpus tokens once a staged build is in */
  int64_t live_active_len; /* corpus tokens of the live suffix array */
  int64_t delta_len;       /* delta tokens */
  int64_t active_head;     /* ring slot of the oldest corpus document */
  int64_t active_docs;     /* corpus documents */
  int64_t delta_head;      /* ring slot of the oldest delta document */
  int64_t delta_docs;      /* delta documents */
  int64_t in_flight;       /* 1: a snapshot is staged, not yet swapped in */
  int64_t snap_seq;        /* snapshots staged so far */
  int64_t snap_n_new;      /* tokens of the last staged corpus */
  int64_t snap_m;          /* suffixes its build sorts (n_new + 1, capped) */
  int64_t docs_in;         /* documents appended so far */
  int64_t docs_dropped;    /* delta documents dropped to make room */
  int64_t tokens_dropped;
  int64_t bad_rows;        /* row indices outside the token buffer */
  int64_t reserved;
} sfx_ingest_header;

#define SFX_INGEST_MAX_DOCS 4096

/* No reference counterpart (the reference takes host lengths and decides
 * on the host).  out[0] = state bytes for an index of this geometry,
 * out[1], out[2] = corpus and delta ring slots, out[3], out[4] = byte
 * offsets of the two rings, out[5] = of the scratch delta.  The state is
 * 256-byte aligned; the caller fills the header and rings once (from its
 * own bookkeeping) before the first sfx_ingest_docs. */
int sfx_ingest_layout(int64_t capacity, int64_t delta_capacity,
                      int64_t* out);

/* harvest_finished with device row indices and lengths: appends
 * tokens[row_idx[i], 0 : min(lengths[i], seq)] for i < ndocs (<=
 * SFX_INGEST_MAX_DOCS; int32 or int64 indices and lengths), each followed
 * by SEP, taking every decision of append_documents on the device --
 * truncation to the last delta_capacity - 1 tokens, making room, dropping
 * the oldest delta documents, and the rebuild snapshot (eviction, whole
 * delta documents, the staging corpus written with PAD after it) of
 * _make_room and maybe_rebuild.  A snapshot bumps header.snap_seq: the
 * caller then builds staging_corpus[0 : snap_m] into the staging suffix
 * array and swaps it in, calling sfx_ingest_swapped after the swap; until
 * then the rebuild counts as running.  A row index is a Python index:
 * -rows <= r < 0 counts from the end (token_ids_gpu[r],
 * proposer.py:342); rows outside [-rows, rows), where the reference raises
 * IndexError, are skipped and counted in header.bad_rows.  Lengths <= 0
 * append nothing.  corpus, delta and delta_len are the index's (sfx_index);
 * the delta and its length word are updated in place.  Three launches on
 * `stream`, no host synchronisation. */
int sfx_ingest_docs(void* state, const int32_t* corpus, int64_t capacity,
                    int32_t* delta, int64_t delta_capacity,
                    int64_t* delta_len, int32_t* staging_corpus,
                    const int32_t* tokens, int64_t rows, int64_t seq,
                    const void* row_idx, int32_t row_idx_is64,
                    const void* lengths, int32_t lengths_is64, int64_t ndocs,
                    int64_t rebuild_threshold, hipStream_t stream);

/* proposer.py:354-390 ingest_active with device slot keys and lengths:
 * in-flight responses fed to the index in chunks.  For i < ndocs, in
 * order, with key = keys[i] (a slot in [0, nslots); others are skipped
 * and counted in header.bad_rows), ln = lengths[i] and done =
 * ingested[key]: when ln - done >= chunk, or final and ln > done, the
 * document tokens[i, max(0, done - overlap) : ln] (a Python slice of row
 * i; overlap is max_pattern_len + k in the reference) is appended and
 * ingested[key] = ln; with final, ingested[key] = 0 afterwards (the
 * reference forgets the key).  The documents then take the same
 * append_documents decisions as sfx_ingest_docs.  ingested is the
 * caller's int64 table of per-slot progress (zeroed once), rows >= ndocs;
 * three launches on `stream`, no host synchronisation. */
int sfx_ingest_active(void* state, const int32_t* corpus, int64_t capacity,
                      int32_t* delta, int64_t delta_capacity,
                      int64_t* delta_len, int32_t* staging_corpus,
                      const int32_t* tokens, int64_t rows, int64_t seq,
                      const void* keys, int32_t keys_is64,
                      const void* lengths, int32_t lengths_is64,
                      int64_t ndocs, int64_t* ingested, int64_t nslots,
                      int32_t final, int64_t chunk, int64_t overlap,
                      int64_t rebuild_threshold, hipStream_t stream);

/* The staged build is live (after sfx_index_swap): the rebuild is no
 * longer running. */
int sfx_ingest_swapped(void* state, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SUFFIXGPU_AMD_H */
