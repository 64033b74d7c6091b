/*
 * dsa_amd.h -- C ABI of the MI355X (gfx950) Lightning-Indexer decode path.
 *
 * Every entry point takes raw device pointers, plain sizes and a hipStream_t
 * passed as `void*` (NULL = the legacy default stream), launches
 * asynchronously on that stream and returns a status code.  The library never
 * allocates device memory: outputs and workspaces are owned by the caller.
 * On a non-zero status dsa_last_error() returns a message for the calling
 * thread.
 *
 * Shapes follow the reference's `temporal_dsa` package (psa1582/dsa):
 *   queries  [64, 128]   fp16 / bf16 (fp32 for the fp32 path)
 *   weights  [64]        fp32 (signed head weights)
 *   keys     [L, 128]    same dtype as queries, or fp8 e4m3fn with one fp32
 *                        scale per 128-key block (scales must be >= 0)
 *   score[s] = sum_h w_h * ReLU(q_h . k_s), fp32 accumulation.
 * All arrays are contiguous row-major.  Block masks are one byte per block
 * (torch.bool or torch.int8); zero means false.
 */
#ifndef DSA_AMD_H
#define DSA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_ABI_VERSION 5

#define DSA_STATUS_OK 0
#define DSA_STATUS_INVALID_ARGUMENT 1
#define DSA_STATUS_HIP_ERROR 2
#define DSA_STATUS_WORKSPACE_TOO_SMALL 3

/* Key / query element types. */
#define DSA_DTYPE_F32 0
#define DSA_DTYPE_F16 1
#define DSA_DTYPE_BF16 2
#define DSA_DTYPE_FP8_E4M3 3 /* keys only; queries are bf16 */
#define DSA_DTYPE_F64 4      /* score rows of dsa_topk_exact only */

/* Message describing the last failure on the calling thread. */
const char* dsa_last_error(void);

/* DSA_ABI_VERSION of the loaded library. */
int dsa_abi_version(void);

/* ------------------------------------------------------------------------
 * Dense indexer scores for a batch of independent decode sequences.
 *
 * Replaces progressive_kernel.py:362-375 (full_scores_triton, batch = 1,
 * `block_size` only affects the reference's launch tiling) and the Q = 1 case
 * of sidecar.py:89-107 (LightningIndexerSidecar.score_encoded).
 *
 *   queries    [batch, 64, 128]    q_dtype (bf16/f16/f32; bf16 when fp8 keys)
 *   weights    [batch, 64]         fp32
 *   keys       [batch, length, 128] key_dtype
 *   key_scales [batch, ceil(length/128)] fp32, fp8 keys only (else NULL)
 *   out        [batch, length]     fp32
 * Strides between sequences are the dense ones (64*128, 64, length*128,
 * ceil(length/128), length).
 * ------------------------------------------------------------------------ */
int dsa_full_scores(const void* queries, const float* weights, const void* keys,
                    const float* key_scales, float* out, int64_t batch, int64_t length,
                    int32_t key_dtype, void* stream);

/* ------------------------------------------------------------------------
 * General query-block scoring: `sequences` query blocks, each scored against
 * one key set.  Sequence s uses
 *   queries + s*q_stride      a [H, 128] block (fp16/bf16), H >= head rows used
 *   weights + s*w_stride      fp32 per head
 *   head_ids + s*ids_stride   int32 ids of the head_count (<= 64) heads used,
 *                             or NULL for heads 0..head_count-1
 *   keys + (s / queries_per_keyset) * key_stride rows   [length, 128]
 *   key_scales + (s / queries_per_keyset) * scale_stride (fp8 keys only)
 *   out + s*out_stride        fp32 [length]
 * causal_offset >= 0 masks key j of query t = s % queries_per_keyset unless
 * j <= t + causal_offset (masked scores are -inf); < 0 disables the mask.
 *
 * Replaces sidecar.py:89-107 (score_encoded: B key sets, Q queries each) and
 * verifier_scoring.py:49-92 (score_head_sparse: fixed [h_v] or per-query
 * [Q, h_v] head ids, one shared key set).  Queries and keys must be 16-byte
 * aligned and q_stride a multiple of 8 elements.
 * ------------------------------------------------------------------------ */
int dsa_score_queries(const void* queries, int64_t q_stride, const float* weights,
                      int64_t w_stride, const int32_t* head_ids, int64_t ids_stride,
                      int32_t head_count, const void* keys, int64_t key_stride,
                      int64_t queries_per_keyset, const float* key_scales, int64_t scale_stride,
                      float* out, int64_t out_stride, int64_t sequences, int64_t length,
                      int64_t causal_offset, int32_t key_dtype, void* stream);

/* ------------------------------------------------------------------------
 * Prefill indexer step in one launch: the scores of dsa_score_queries (all
 * 64 heads, fp16/bf16 keys) and, per query, the exact top-k of its visible
 * keys with stable_topk's set (metrics.py:9-22), in ascending index order as
 * dsa_topk with sorted == 0.
 *
 * Replaces sidecar.py:89-107 (score_encoded over Q queries per key set)
 * followed by a per-query stable top-k of the score rows (metrics.py:9-22).
 *   out            fp32 [sequences, out_stride]: the scores (masked -inf)
 *   out_indices    int64 [sequences, topk_stride]: row s's top-k key ids;
 *                  a query with fewer than k visible keys returns all of
 *                  them, padded with -1
 *   out_values     fp32, same layout, nullable (padding -inf)
 * Each workgroup scores four consecutive queries of one key set; each
 * query's wave then selects from its own row.  Limits: length <= 4096,
 * queries_per_keyset >= 4 and sequences a multiple of it, k >= 1,
 * topk_stride >= k; other arguments as dsa_score_queries.
 * ------------------------------------------------------------------------ */
int dsa_score_queries_topk(const void* queries, int64_t q_stride, const float* weights, int64_t w_stride,
                           const void* keys, int64_t key_stride, int64_t queries_per_keyset, float* out,
                           int64_t out_stride, int64_t sequences, int64_t length, int64_t causal_offset,
                           int32_t key_dtype, int32_t k, int64_t* out_indices, float* out_values,
                           int64_t topk_stride, void* stream);

/* ------------------------------------------------------------------------
 * Statistics of consecutive score rows, for the replay analysis tables
 * (replay.py:403-474, temporal_stats / block_temporal_stats).  dtype codes:
 * DSA_DTYPE_F32 or DSA_DTYPE_F64.
 * ------------------------------------------------------------------------ */

/* x, y [n]: out[7] float64 = mean x, mean y, sum (x-mx)^2, sum (y-my)^2,
 * sum (x-mx)(y-my), mean d, sum (d-md)^2 with d = y - x (subtracted in the
 * rows' precision, as numpy subtracts float32 rows); abs_delta [n] in the
 * rows' dtype receives |d| (nullable).  Pearson's r (metrics.py:40-47) and
 * the drift's mean and std (replay.py:417-419) follow from out. */
int dsa_pair_moments(const void* x, const void* y, int32_t dtype, int64_t n, double* out, void* abs_delta,
                     void* stream);

/* 0-based ascending ranks of a row, ties sharing the mean of their positions
 * (metrics.py:50-61, the input of spearman), from the row sorted descending
 * (sorted [n] in dtype, e.g. dsa_topk_exact with k = n) and the key of each
 * sorted position (order [n]); ranks [n] float64 indexed by key. */
int dsa_average_ranks(const void* sorted, int32_t dtype, const int64_t* order, int64_t n, double* ranks,
                      void* stream);

/* *out += |{b[i]} ∩ {a[j]}| for two ascending key lists of length k (entries
 * -1 are padding at the end and match nothing): the top-k overlap of
 * replay.py:425-426 from the two rows' top-k in index order. */
int dsa_index_overlap(const int64_t* a, const int64_t* b, int64_t k, uint32_t* out, void* stream);

/* Per block b < blocks: streak[b] = cur_max[b] < *threshold ? streak[b] + 1
 * : 0, delta[b] = cur_max[b] - prev_max[b] (float64), and counts[0..3] +=
 * the blocks whose streak is at least 1, 2, 4, 8 (replay.py:448-472; the
 * threshold is the row's k-th largest score, a device value). */
int dsa_block_streaks(const float* prev_max, const float* cur_max, int64_t blocks, const float* threshold,
                      int32_t* streak, double* delta, uint32_t* counts, void* stream);

/* Head routing: per row of weights [rows, heads] (heads <= 64) the `width`
 * head ids with the largest |w| (positive_only == 0) or max(w, 0)
 * (positive_only != 0), ties to the lower id, in rank order.  Output to
 * out_int32 and/or out_int64 [rows, width].
 * Replaces progressive_kernel.py:37-42 (dynamic_head_ids) and
 * verifier_scoring.py:142-159 (dynamic_head_indices). */
int dsa_route_heads(const float* weights, int64_t rows, int64_t heads, int64_t width,
                    int32_t positive_only, int32_t* out_int32, int64_t* out_int64, void* stream);

/* ------------------------------------------------------------------------
 * H8 verifier partial scores and per-block maxima.
 * Replaces progressive_kernel.py:378-404 (h8_block_max_triton) /
 * progressive_kernel.py:218-246 (_h8_block_max_kernel).
 *
 *   selected_heads [8] int32 device array, cold_blocks [ceil(L/bs)] bytes.
 *   key_scales: fp8 e4m3fn keys only (else NULL), one fp32 scale per 128 keys
 *   (as dsa_full_scores); every score, partial or full, is scaled.  The same
 *   holds for dsa_masked_full_scores and dsa_progressive_scores.
 *   partial[s] = sum over the 8 selected heads where the block is cold, else
 *   -inf; block_max[b] = max of partial over the block (-inf if not cold).
 * ------------------------------------------------------------------------ */
int dsa_h8_block_max(const void* queries, const float* weights, const void* keys,
                     const float* key_scales, const int32_t* selected_heads, const uint8_t* cold_blocks,
                     float* partial, float* block_max, int64_t length, int32_t block_size, int32_t key_dtype,
                     void* stream);

/* ------------------------------------------------------------------------
 * Full scores on kept blocks, -inf elsewhere; rejected blocks load no keys.
 * Replaces progressive_kernel.py:407-424 (masked_full_scores_triton).
 * ------------------------------------------------------------------------ */
int dsa_masked_full_scores(const void* queries, const float* weights, const void* keys,
                           const float* key_scales, const uint8_t* keep_blocks, float* out, int64_t length,
                           int32_t block_size, int32_t key_dtype, void* stream);

/* ------------------------------------------------------------------------
 * Fused progressive scoring: direct blocks get all 64 heads; other blocks get
 * the 8 selected heads, their maximum is compared with *threshold and blocks
 * with max >= threshold are promoted to the 56 remaining heads.
 * Replaces progressive_kernel.py:427-475 (progressive_scores_triton) /
 * progressive_kernel.py:277-346 (_progressive_kernel).
 *
 *   selected_heads [8], remaining_heads [56] int32 device arrays
 *   direct_blocks  [nb] bytes, threshold [1] fp32 device scalar
 *   accepted [nb] int8, block_max [nb] fp32 (-inf for direct blocks)
 *   compact == 0: out_scores [L] = score or -inf, out_indices unused (NULL ok)
 *   compact != 0: accepted keys are appended to out_scores/out_indices at
 *                 positions reserved by an atomic add of the block's valid-key
 *                 count on *counter (int32, zeroed by the caller); after the
 *                 call *counter is the exact candidate count.  Block order in
 *                 the compact output is unspecified (keys inside a block stay
 *                 in address order).
 * ------------------------------------------------------------------------ */
int dsa_progressive_scores(const void* queries, const float* weights, const void* keys,
                           const float* key_scales, const int32_t* selected_heads, const int32_t* remaining_heads,
                           const uint8_t* direct_blocks, const float* threshold,
                           float* out_scores, int32_t* out_indices, int8_t* accepted,
                           float* block_max, int32_t* counter, int64_t length,
                           int32_t block_size, int32_t compact, int32_t key_dtype, void* stream);

/* dsa_progressive_scores over `batch` sequences of one length in one launch
 * (the reference's kernel takes one sequence, progressive_kernel.py:277-346):
 * every array is packed per sequence -- queries [batch, 64, 128], weights
 * [batch, 64], keys [batch, length, 128] (fp8 key_scales [batch,
 * ceil(length / 128)]), selected_heads [batch, 8], remaining_heads
 * [batch, 56], direct_blocks, accepted, block_max [batch, blocks],
 * thresholds [batch] (device), out_scores and out_indices [batch, length],
 * counters [batch] (zeroed by the caller for compact output).  Each sequence
 * gives exactly what dsa_progressive_scores gives for it. */
int dsa_progressive_scores_batched(const void* queries, const float* weights, const void* keys,
                                   const float* key_scales, const int32_t* selected_heads,
                                   const int32_t* remaining_heads, const uint8_t* direct_blocks,
                                   const float* thresholds, float* out_scores, int32_t* out_indices,
                                   int8_t* accepted, float* block_max, int32_t* counters, int64_t batch,
                                   int64_t length, int32_t block_size, int32_t compact, int32_t key_dtype,
                                   void* stream);

/* accepted[b] = direct[b] || block_max[b] >= *threshold  (bytes 0/1).
 * Replaces the torch logical_or at progressive_kernel.py:493. */
int dsa_promote_blocks(const uint8_t* direct_blocks, const float* block_max,
                       const float* threshold, uint8_t* accepted, int64_t blocks, void* stream);

/* ------------------------------------------------------------------------
 * Exact top-k per row with the reference's stable_topk semantics
 * (metrics.py:9-22): the k largest values, ties at the cut-off resolved
 * towards the lower index; -0.0 equals +0.0.  NaN is not supported.
 *
 *   scores      [rows, row_stride] fp32, the first `length` entries of a row
 *               are candidates
 *   row_lengths [rows] int32 or NULL: per-row number of valid leading
 *               entries (<= length); rows with fewer than k valid entries
 *               return all of them and pad with index -1 / value -inf
 *   in_indices  [rows, row_stride] int64 or NULL: candidate i of a row stands
 *               for key in_indices[i]; ties then break on that key id.  A row
 *               of in_indices must be strictly increasing.
 *   sorted != 0: output ordered by (value desc, index asc) like stable_topk;
 *   sorted == 0: output ordered by ascending index.
 *   out_indices [rows, k] int64, out_values [rows, k] fp32 (either may be NULL)
 *   k <= 4096 and length <= 32768 per call; longer rows go through
 *   dsa_topk_long.
 * ------------------------------------------------------------------------ */
int dsa_topk(const float* scores, const int64_t* in_indices, int64_t rows, int64_t length,
             int64_t row_stride, const int32_t* row_lengths, int64_t k, int32_t sorted,
             int64_t* out_indices, float* out_values, void* stream);

/* Top-k of rows longer than one workgroup's register tile: rows are cut into
 * chunks whose local top-k candidates are merged exactly.  `workspace` must
 * hold dsa_topk_long_workspace_bytes(rows, length, k) bytes. */
int64_t dsa_topk_long_workspace_bytes(int64_t rows, int64_t length, int64_t k);
int dsa_topk_long(const float* scores, int64_t rows, int64_t length, int64_t k, int32_t sorted,
                  int64_t* out_indices, float* out_values, void* workspace,
                  int64_t workspace_bytes, void* stream);

/* Exact stable top-k of float64 or float32 rows with 64-bit order keys:
 * stable_topk (metrics.py:9-22) for any 0 < k <= length, any length below
 * 2^31, and float64 values that float32 cannot hold.  One workgroup per row:
 * radix select of the cut, a gather in index order and, when `sorted`, a
 * stable radix sort into (descending value, ascending index) order.
 * values [rows][row_stride] (DSA_DTYPE_F64 or DSA_DTYPE_F32), out_indices
 * [rows][k], out_values [rows][k] in the input dtype or NULL.  Sorted output
 * needs dsa_topk_exact_workspace_bytes(rows, k, 1) bytes of workspace
 * (16-byte aligned, no initialisation); unsorted output needs none.  NaN
 * values are outside the contract (the Python mirror rejects them). */
int64_t dsa_topk_exact_workspace_bytes(int64_t rows, int64_t k, int32_t sorted);
int dsa_topk_exact(const void* values, int32_t value_dtype, int64_t rows, int64_t length, int64_t row_stride,
                   int64_t k, int32_t sorted, int64_t* out_indices, void* out_values, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Fused decode step: dense scores of `batch` sequences (as dsa_full_scores)
 * plus the exact top-k of every sequence with the stable_topk rule.
 * Replaces the reference benchmark's full-score launch followed by
 * torch.topk (scripts/benchmark_progressive_dsa.py:117-123) with the
 * selection semantics of metrics.py:9-22.
 *
 *   scores      [batch, length] fp32, written (materialised scores)
 *   out_indices [batch, k] int64 in ascending index order (-1 padding when
 *               length < k); out_values [batch, k] fp32 or NULL
 *   workspace   dsa_score_topk_workspace_bytes(batch, length) bytes, 256-byte
 *               aligned, zero-filled before its first use; every call leaves
 *               it ready for the next one.  Calls that share a workspace must
 *               be ordered (same stream); length <= 524288.
 * Three launches, each over the whole GPU: scoring (+ a per-row 4096-bin
 * score histogram), candidate gather (the bin holding the k-th score, per
 * 2048-key chunk), and exact resolve (the cut, the output offsets and the
 * indices).
 * ------------------------------------------------------------------------ */
int64_t dsa_score_topk_workspace_bytes(int64_t batch, int64_t length);

/* The two halves of dsa_score_topk, for callers that time or overlap them:
 * dsa_score_hist writes the scores and the selection's intermediate state
 * (per-chunk candidate lists, or the per-row score histogram when a
 * workgroup's chunk exceeds 8192 keys) into the workspace; dsa_select_topk
 * turns scores + that state into the top-k and leaves the workspace ready for
 * the next dsa_score_hist.  Every dsa_score_hist on a workspace must be
 * followed by a dsa_select_topk on it (same batch, length and k) before the
 * next dsa_score_hist. */
int dsa_score_hist(const void* queries, const float* weights, const void* keys,
                   const float* key_scales, float* scores, int64_t batch, int64_t length,
                   int64_t k, int32_t key_dtype, void* workspace, int64_t workspace_bytes,
                   void* stream);
int dsa_select_topk(const float* scores, int64_t batch, int64_t length, int64_t k,
                    int64_t* out_indices, float* out_values, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* Measurement variants of the two halves (no counterpart in the reference,
 * whose benchmark brackets launches with events): the half's first kernel
 * records start_event at its own start and its last kernel records
 * stop_event at its own end (hipExtLaunchKernel), so the interval is the
 * kernels' execution alone, as a profiler's kernel trace reports it.  The
 * events (hipEvent_t) are created by the caller; either may be NULL. */
int dsa_score_hist_timed(const void* queries, const float* weights, const void* keys,
                         const float* key_scales, float* scores, int64_t batch, int64_t length,
                         int64_t k, int32_t key_dtype, void* workspace, int64_t workspace_bytes,
                         void* stream, void* start_event, void* stop_event);
int dsa_select_topk_timed(const float* scores, int64_t batch, int64_t length, int64_t k,
                          int64_t* out_indices, float* out_values, void* workspace,
                          int64_t workspace_bytes, void* stream, void* start_event,
                          void* stop_event);

/* Exact top-k (stable_topk set, ascending index order, -1 padding) of score
 * rows [rows, length] fp32, spread over the whole GPU: a 4096-bin histogram
 * of every row, then the decode step's candidate gather and exact resolve.
 * For a few long rows, where dsa_topk's one workgroup per row is bound by a
 * single CU.  Replaces torch.topk(scores, k, sorted=False) on such rows
 * (scripts/benchmark_progressive_dsa.py:123-169).  The workspace is the
 * decode step's (dsa_score_topk_workspace_bytes(rows, length), zero-filled
 * before first use and left zeroed); length <= 524288, scores 16-byte aligned. */
int dsa_topk_distributed(const float* scores, int64_t rows, int64_t length, int64_t k,
                         int64_t* out_indices, float* out_values, void* workspace,
                         int64_t workspace_bytes, void* stream);

int dsa_score_topk(const void* queries, const float* weights, const void* keys,
                   const float* key_scales, float* scores, int64_t batch, int64_t length,
                   int64_t k, int32_t key_dtype, int64_t* out_indices, float* out_values,
                   void* workspace, int64_t workspace_bytes, void* stream);

/* Allocation-free variant of dsa_score_topk.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as dsa_score_topk minus the workspace, which lives in
 * a file-scope device array of DSA_NOALLOC_SCRATCH_BYTES per GPU, held from
 * module load until the process ends.  Shapes whose workspace
 * (dsa_score_topk_workspace_bytes(batch, length), about 8 bytes per key plus
 * 16 KiB per row) exceeds it are rejected with DSA_STATUS_WORKSPACE_TOO_SMALL.
 * Calls no hipMalloc/hipFree.  All calls on one GPU share that GPU's array:
 * calls ordered on one stream are safe, calls that overlap on one GPU race.
 * The pointers and the stream must belong to the current device. */
#define DSA_NOALLOC_SCRATCH_BYTES (16ll << 20)
int dsa_score_topk_noalloc(const void* queries, const float* weights, const void* keys,
                           const float* key_scales, float* scores, int64_t batch, int64_t length,
                           int64_t k, int32_t key_dtype, int64_t* out_indices, float* out_values,
                           void* stream);

/* ------------------------------------------------------------------------
 * Temporal pruning of one decode step (seeded, bounded block scan).
 * Device counterpart of the reference's replay filter: replay.py:172-222
 * (_run_filter) and replay.py:225-400 (replay_transition with a calibrated
 * absolute margin, methods static / static_hot_first / dynamic).
 *
 *   prev_block_max [batch, ceil(prev_length / block_size)] fp32: block maxima
 *               of the previous step's scores (dsa_block_max)
 *   prev_topk   [batch, k] int64: the previous step's top-k (the seeds),
 *               distinct, < prev_length
 *   gamma       [batch] fp32: absolute margin; U_b = prev max + gamma, and
 *               blocks holding keys past prev_length are never pruned
 *   block_margins [batch, ceil(prev_length / block_size)] float64 or NULL:
 *               per-block margins used instead of gamma (U_b = prev max +
 *               margin_b), e.g. the certified ones of dsa_certified_margins
 *               (gamma may then be NULL)
 *   scan_order  0 address, 1 previous-hot (blocks of the seeds first, then
 *               larger U, then address), 2 larger U then address
 *   wave        0: threshold fixed at the seed minimum (static); W > 0: the
 *               threshold becomes the k-th largest evaluated score after
 *               every W blocks of the scan (W = 1 is the reference's dynamic
 *               filter).  With DSA_AMD_TEMPORAL_PATH=launch (the
 *               sequential path) k + wave * block_size <= 8192.
 *   scores      [batch, length] fp32 out: evaluated keys' scores, else -inf
 *   evaluated_blocks [batch, ceil(length / block_size)] bytes out: 1 = kept
 *   out_topk    [batch, k] int64 out: stable top-k of the evaluated keys, in
 *               ascending index order
 *   qk_scored   [batch] int32 out: keys scored (seeds + kept blocks, once each)
 *   waits_given_up [batch] int32 out, or NULL: workgroups of the fused static
 *               launch (below) whose bounded wait for the row's seed minima
 *               ran out (other work held the CUs it needed for ~4 s).  Such a
 *               workgroup keeps every block of its chunk, so the row's kept
 *               blocks, qk_scored and top-k are a superset of the filter's;
 *               0 means the decisions are exactly the filter's.  Always 0 on
 *               the other paths, which do not wait.
 *   keys        [batch, key_stride, 128]: the first `length` rows of each
 *               sequence are scored (a KV cache with spare capacity needs no
 *               copy); fp8 key_scales are [batch, ceil(key_stride / 128)]
 *   length <= 131072 and at most 2048 blocks, block_size in {16, 32, 64,
 *   128}, k <= 4096; keys as in dsa_full_scores (bf16/fp16, or fp8 with
 *   key_scales).
 *   workspace   dsa_temporal_workspace_bytes(batch, length, k, block_size)
 *               bytes, 256-byte aligned, shared by the temporal, approximate
 *               and verifier steps; its first 32 KiB must be zero before its
 *               first use (the static step's generation-stamped exchange
 *               slots, which no later call misreads); calls that share it
 *               must be ordered (one stream).
 * A static step (wave 0) loads only the seeds and the kept blocks: when its
 * shape fits the decode step's candidate-list plan and its workgroups fit on
 * the device at once it is one scoring launch plus the list select.  A
 * dynamic step (wave > 0) runs in rounds that split the scan at group
 * boundaries (DSA_AMD_TEMPORAL_ROUNDS: fractions of the groups, default 0.25,
 * or 0.1,0.3 from 64K keys): each round scores every block of its positions
 * whose bound clears the threshold at the round's start, over the whole GPU,
 * then replays the scan's decisions exactly in one workgroup per row; blocks
 * scored there and then pruned are reported by dsa_temporal_keys_loaded.
 * DSA_AMD_TEMPORAL_PATH=launch in the environment keeps every step on the
 * sequential launch paths (per-wave block and refresh launches, or the
 * persistent per-row scan), which load only the blocks they keep.
 * ------------------------------------------------------------------------ */
int64_t dsa_temporal_workspace_bytes(int64_t batch, int64_t length, int64_t k, int32_t block_size);

/* Key rows the last dynamic temporal step on `workspace` loaded, per row
 * (int32 [batch], device memory, written on `stream`): the seeds plus every
 * key of the blocks its rounds scored, a superset of the keys it reports in
 * qk_scored.  Defined after a dynamic step (wave > 0) on the default path;
 * the other paths load the keys they score.  No counterpart in the reference,
 * whose replay (replay.py:369-371) prices bytes from the keys scored: this is
 * the measured side of that figure. */
int dsa_temporal_keys_loaded(const void* workspace, int64_t batch, int64_t length, int64_t k, int32_t block_size,
                             int32_t* out, void* stream);

int dsa_temporal_step(const void* queries, const float* weights, const void* keys, int64_t key_stride,
                      const float* key_scales, const float* prev_block_max, int64_t prev_length,
                      const int64_t* prev_topk,
                      const float* gamma, const double* block_margins, float* scores, uint8_t* evaluated_blocks,
                      int64_t* out_topk,
                      int32_t* qk_scored, int32_t* waits_given_up, int64_t batch, int64_t length, int64_t k,
                      int32_t block_size,
                      int32_t scan_order, int32_t wave, int32_t key_dtype, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Own-trajectory pruned decode step (approx.py:129-364 replay_step with
 * history_mode="own"; policy fields approx.py:15-39 ApproxPolicy).
 *
 * The per-block metadata of the policy lives on the device, one row per
 * sequence with a fixed capacity (state_stride blocks):
 *   last_max, ema, volatility  fp32  [batch, state_stride]
 *   age, cold_streak           int16 [batch, state_stride]
 * It describes the first ceil(prev_length / block_size) blocks; blocks past
 * those are read as the reference's extension (-inf, -inf, 0, 0, 1).
 *
 * dsa_approx_step scores the seeds (prev_topk, the previous approximate
 * top-k), then scans blocks in the policy's order.  A block is forced when
 * full_refresh is set, it holds keys the previous step did not have, it lies
 * in the recent window, its age reached age_cap (>= 0), or its cold streak is
 * below cold_streak.  Any other block is skipped iff
 *   risk = last_max + gamma + age_slope * age                    (risk_model 0)
 *   risk = ema + volatility_lambda * volatility + gamma + age_slope * age (1)
 * is below the threshold in force (float64 arithmetic, as the reference).
 * wave = 0 keeps the seed threshold (static policy); wave >= 1 refreshes it to
 * the k-th largest evaluated score after every `wave` blocks of the scan
 * (wave = 1 is the reference's per-block refresh).
 * Outputs are those of dsa_temporal_step (out_topk is the approximate top-k in
 * ascending index order).  On return, the metadata of every block of the
 * current length has been advanced in place: refreshed blocks take the
 * current block max (EMA and volatility updated with ema_alpha, age 0),
 * others keep stale values with age + 1 (saturating at 32767); the cold
 * streak is 0 for blocks holding an approximate top-k key, else + 1.
 * gamma_rows (nullable) overrides policy->gamma per sequence.
 * history_mode="teacher" needs the dense step and is not a device path;
 * order "oracle_current" reads the current scores and is rejected.
 * Limits as dsa_temporal_step; state_stride >= ceil(length / block_size).
 * ------------------------------------------------------------------------ */
#define DSA_RISK_LAST_MAX 0
#define DSA_RISK_EMA 1
#define DSA_ORDER_ADDRESS 0
#define DSA_ORDER_PREVIOUS_MAX 1 /* also "predicted_risk" */
#define DSA_ORDER_BUCKET 2
#define DSA_ORDER_CURRENT_MAX 3 /* "oracle_current": replay over recorded rows only */
#define DSA_HISTORY_OWN 0       /* approx.py history_mode "own": the state follows the step's own top-k */
#define DSA_HISTORY_TEACHER 1   /* "teacher": seeds and state follow the dense trace (replay only) */

typedef struct dsa_approx_policy {
  double gamma;
  double age_slope;
  double ema_alpha;
  double volatility_lambda;
  int32_t risk_model;    /* DSA_RISK_* */
  int32_t order;         /* DSA_ORDER_* */
  int32_t buckets;       /* bucket count of DSA_ORDER_BUCKET ("bucket8" -> 8) */
  int32_t cold_streak;
  int32_t age_cap;       /* < 0: no cap */
  int32_t recent_window; /* keys; 0: none */
  int32_t full_refresh;  /* policy "full", refresh interval or fallback hit */
  int32_t history;       /* DSA_HISTORY_OWN, or DSA_HISTORY_TEACHER (replay over recorded rows only) */
} dsa_approx_policy;

int dsa_approx_step(const void* queries, const float* weights, const void* keys, int64_t key_stride,
                    const float* key_scales, const dsa_approx_policy* policy, const double* gamma_rows,
                    int64_t prev_length, const int64_t* prev_topk, float* last_max, float* ema,
                    float* volatility, int16_t* age, int16_t* cold_streak, int64_t state_stride,
                    float* scores, uint8_t* evaluated_blocks, int64_t* out_topk, int32_t* qk_scored,
                    int64_t batch, int64_t length, int64_t k, int32_t block_size, int32_t wave,
                    int32_t key_dtype, void* workspace, int64_t workspace_bytes, void* stream);

/* One step replayed over recorded score rows (approx.py:129-364
 * replay_step): row r's scores come from current_scores [batch][score_stride]
 * instead of being computed from keys.  The order DSA_ORDER_CURRENT_MAX (the
 * reference's "oracle_current") visits blocks by larger current_block_max
 * [batch][blocks] (fp32, nullable otherwise), then lower address.
 * History (policy->history, approx.py:143-158,270-280):
 *   DSA_HISTORY_OWN: prev_topk is the previous step's own top-k and the
 *     state is updated for the refreshed blocks only;
 *   DSA_HISTORY_TEACHER: prev_topk is the previous step's dense top-k, and
 *     every block's state is reset from the dense row (last max = EMA = the
 *     block's maximum, volatility 0, age 0), with the cold streak restarting
 *     at the blocks of teacher_topk [batch][k], the current step's dense
 *     top-k (required in this mode, nullable otherwise).
 * Other arguments, outputs and limits as dsa_approx_step. */
int dsa_approx_replay_step(const float* current_scores, int64_t score_stride, const float* current_block_max,
                           const dsa_approx_policy* policy, const double* gamma_rows, int64_t prev_length,
                           const int64_t* prev_topk, const int64_t* teacher_topk, float* last_max,
                           float* ema, float* volatility, int16_t* age, int16_t* cold_streak, int64_t state_stride,
                           float* scores, uint8_t* evaluated_blocks, int64_t* out_topk, int32_t* qk_scored,
                           int64_t batch, int64_t length, int64_t k, int32_t block_size, int32_t wave, void* workspace,
                           int64_t workspace_bytes, void* stream);

/* initialize_state (approx.py:112-126) from dense score rows [batch, length]
 * (row stride score_stride) and their top-k (any order): last_max = ema =
 * block max, volatility = 0, age = 0, cold_streak = 0 for blocks holding a
 * top-k key, else 1. */
int dsa_approx_init_state(const float* scores, int64_t score_stride, const int64_t* topk, float* last_max,
                          float* ema, float* volatility, int16_t* age, int16_t* cold_streak,
                          int64_t state_stride, int64_t batch, int64_t length, int64_t k, int32_t block_size,
                          void* stream);

/* The filter of dsa_temporal_step replayed over recorded scores
 * (replay.py:172-222 run_filter inside replay_transition :225-400): the
 * scores of row r are read from current_scores [batch][score_stride] instead
 * of being computed from keys (score_stride 0: every row reads the same
 * scores), gamma is float64 per sequence (the reference's gamma_sigma *
 * sigma), and scan_order_out [batch][blocks] (nullable) receives the scan
 * order.  scan_order 3 visits blocks by larger order_key [batch][blocks]
 * (fp32), then lower address: the reference's "oracle_current" order with the
 * current block maxima as the key.  Its "oracle" method is that order with
 * the current maxima also as prev_block_max, gamma 0 and
 * prev_length = length.  Other arguments, outputs and limits as
 * dsa_temporal_step. */
int dsa_temporal_replay_step(const float* current_scores, int64_t score_stride, const float* prev_block_max,
                             int64_t prev_length, const int64_t* prev_topk, const double* gamma,
                             const float* order_key, float* scores, uint8_t* evaluated_blocks,
                             int32_t* scan_order_out, int64_t* out_topk, int32_t* qk_scored, int64_t batch,
                             int64_t length, int64_t k, int32_t block_size, int32_t scan_order, int32_t wave,
                             void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Two-path verifier step (verifier.py:173-392 verifier_step with
 * apply_rescue_to_state :103-170; the reference replays it offline over
 * recorded dense and verifier score rows, here it is a live decode step).
 *
 * The own-trajectory temporal scan of dsa_approx_step, then a verifier score
 * of every key the scan left unscored ("cold"):
 *   DSA_VERIFIER_HEAD: sum over spec->width selected heads (head_ids [width],
 *     or [batch][head_id_stride] per sequence, e.g. dynamic_head_indices)
 *     of w_h relu(q_h . k) over the full key rows;
 *   DSA_VERIFIER_DIM: all 64 heads over spec->width sketch dims: query_sketch
 *     [batch][64][width] bf16 against key_sketch [batch][sketch_stride][width]
 *     (int8 codes scaled by spec->sketch_scale and rounded to bf16, or bf16
 *     values), as written by dsa_dim_sketch.
 * Cold blocks are ranked by their largest cold verifier score (larger first,
 * lower block id on ties; ranking [batch][blocks] lists them, -1 after, and
 * is nullable); the first min(cold, ceil(rescue_fraction * cold)) are rescued
 * (spec->promotion 0), or every cold block whose score is >= the float32
 * promotion_threshold (1).  Rescued blocks' cold keys are scored in full;
 * out_topk is the stable top-k of every scored key (ascending index).  The
 * state is then advanced as by dsa_approx_step with rescued blocks updated
 * like refreshed ones and the cold streak restarted from the final top-k.
 * Outputs: scores (dense score of every scored key, -inf elsewhere),
 * verifier_scores (nullable; cold keys, -inf elsewhere), block_scores and
 * cold_count (cold keys per block), evaluated_blocks (temporal refreshes),
 * rescued_blocks, qk_scored (temporal exact keys), counts [batch][4] = cold
 * keys, cold blocks, rescued blocks, rescued cold keys.
 * Limits as dsa_approx_step; the dim path takes bf16 queries.
 * ------------------------------------------------------------------------ */
#define DSA_VERIFIER_HEAD 0
#define DSA_VERIFIER_DIM 1

typedef struct dsa_verifier_spec {
  int32_t path;         /* DSA_VERIFIER_* */
  int32_t width;        /* head path: 1..64 heads; dim path: multiple of 8 in [8, 128] */
  int32_t promotion;    /* 0: global budget (rescue_fraction), 1: fixed threshold */
  int32_t sketch_codes; /* dim path: 1 = int8 codes, 0 = bf16 values */
  double rescue_fraction;
  float promotion_threshold;
  float sketch_scale;
} dsa_verifier_spec;

int dsa_verifier_step(const void* queries, const float* weights, const void* keys, int64_t key_stride,
                      const float* key_scales, const dsa_approx_policy* policy, const double* gamma_rows,
                      int64_t prev_length, const int64_t* prev_topk, float* last_max, float* ema,
                      float* volatility, int16_t* age, int16_t* cold_streak, int64_t state_stride,
                      const dsa_verifier_spec* spec, const int32_t* head_ids, int64_t head_id_stride,
                      const void* query_sketch, const void* key_sketch, int64_t sketch_stride, float* scores,
                      float* verifier_scores, float* block_scores, uint8_t* cold_count, uint8_t* evaluated_blocks,
                      uint8_t* rescued_blocks, int32_t* ranking, int64_t* out_topk, int32_t* qk_scored,
                      int32_t* counts, int64_t batch, int64_t length, int64_t k, int32_t block_size, int32_t wave,
                      int32_t key_dtype, void* workspace, int64_t workspace_bytes, void* stream);

/* The verifier step replayed over recorded rows (verifier.py:173-392 as
 * replay_verifier_trace :395-432 drives it): the dense scores of row r come
 * from current_scores [batch][score_stride] and the verifier scores of its
 * cold keys from recorded_verifier_scores [batch][verifier_stride] instead of
 * being computed from keys.  Other arguments, outputs and limits as
 * dsa_verifier_step (spec->path and the sketch fields are not used). */
int dsa_verifier_replay_step(const float* current_scores, int64_t score_stride,
                             const float* recorded_verifier_scores, int64_t verifier_stride,
                             const dsa_approx_policy* policy, const double* gamma_rows, int64_t prev_length,
                             const int64_t* prev_topk, float* last_max, float* ema, float* volatility, int16_t* age,
                             int16_t* cold_streak, int64_t state_stride, const dsa_verifier_spec* spec, float* scores,
                             float* verifier_scores, float* block_scores, uint8_t* cold_count,
                             uint8_t* evaluated_blocks, uint8_t* rescued_blocks, int32_t* ranking, int64_t* out_topk,
                             int32_t* qk_scored, int32_t* counts, int64_t batch, int64_t length, int64_t k,
                             int32_t block_size, int32_t wave, void* workspace, int64_t workspace_bytes, void* stream);

/* Dimension sketch of rows x [rows][dim] (verifier_scoring.py:9-41, 95-139):
 * the normalized Walsh-Hadamard transform over dim (a power of two <= 128;
 * when rotate != 0), each butterfly sum and the final multiply by dim^-0.5
 * rounded to dtype (F32 / F16 / BF16), then the dims listed in dims [width]
 * (NULL: the first width), then, when bits is 2, 4 or 8, symmetric
 * quantization with limit 2^(bits-1) - 1: code = clamp(rint(v / scale)).
 * out [rows][width]: int8 codes (out_codes != 0) or values in dtype
 * (code * scale rounded to dtype when quantized). */
int dsa_dim_sketch(const void* x, int64_t rows, int32_t dim, int32_t dtype, const int32_t* dims, int32_t width,
                   int32_t rotate, int32_t bits, float scale, void* out, int32_t out_codes, void* stream);

/* max |x| over n values (fake_symmetric_quantize's tensor scale,
 * verifier_scoring.py:37-38), written to *out as fp32. */
int dsa_abs_max(const void* x, int64_t n, int32_t dtype, float* out, void* stream);

/* Elementwise symmetric fake quantization (verifier_scoring.py:29-41):
 * codes (nullable) = clamp(rint(x / scale), +-(2^(bits-1) - 1)); values
 * (nullable) = code * scale rounded to dtype. */
int dsa_fake_quantize(const void* x, int64_t n, int32_t dtype, int32_t bits, float scale, void* values,
                      int8_t* codes, void* stream);

/* All-head sketch scores (score_dim_sparse, verifier_scoring.py:95-139, after
 * the sketches): out[q][key] = sum_h w[q][h] relu(qs[q][h] . ks[key]) for
 * query sketches [queries][heads][width] bf16 (heads <= 64) and key sketches
 * [keys][width] (int8 codes scaled by sketch_scale and rounded to bf16, or
 * bf16 values); fp32 dot products. */
int dsa_sketch_scores(const void* query_sketch, const float* weights, int64_t queries, int32_t heads,
                      const void* key_sketch, int32_t sketch_codes, float sketch_scale, int32_t width, int64_t keys,
                      float* out, void* stream);

/* ------------------------------------------------------------------------
 * Per-block maxima of score rows (replay.py:149-150 _block_max,
 * approx.py:53-55): out[r, b] = max(scores[r, b*bs : min(len, (b+1)*bs)]).
 * block_size is any positive value.
 * ------------------------------------------------------------------------ */
int dsa_block_max(const float* scores, int64_t rows, int64_t length, int64_t row_stride,
                  int32_t block_size, float* out, void* stream);

/* Per-block maximum key L2 norm (certified.py:51-62 block_key_norms) for keys
 * [tokens, heads, dim] (heads = 1 for the shared-key layout):
 * out[b, h] = max over tokens of the block of ||keys[t, h, :]||, float64
 * (sums of squares in float64, as the reference computes them). */
int dsa_block_key_norms(const void* keys, int64_t tokens, int64_t heads, int64_t dim,
                        int32_t block_size, int32_t key_dtype, double* out, void* stream);

/* Certified temporal radius (certified.py:18-48 temporal_score_radius):
 * out[b] = sum_h block_key_norm[b, h] * (|w_now-w_prev|_h ||q_prev,h|| +
 * |w_now|_h ||q_now,h - q_prev,h||), everything float64 (q: [heads, dim],
 * w: [heads], norms: [blocks, heads]).  The result is scaled by (1 + 2^-36)
 * so that it never falls below the reference's float64 value; requires
 * heads <= 1024 and dim + heads <= 8188. */
int dsa_temporal_score_radius(const double* q_now, const double* q_prev, const double* w_now,
                              const double* w_prev, const double* block_key_norm, int64_t blocks,
                              int64_t heads, int64_t dim, double* out, void* stream);

/* Certified per-block margins of a temporal step over a shared-key cache
 * (the reference's radius, certified.py:18-48, with every head's block norm
 * equal to the block's largest key norm), plus an allowance for the fp32
 * rounding of both steps' scores, so that with the previous step's dense
 * block maxima, U_b = prev max + margin_b bounds every current score of
 * block b as the scoring kernels compute it: a step pruning with these
 * margins keeps every key of the dense top-k.  q_now, q_prev [batch, 64, 128]
 * and keys [batch, key_stride, 128] in key_dtype (bf16/fp16), or fp8 e4m3fn
 * keys with key_scales [batch, ceil(key_stride / 128)] fp32 and bf16 queries
 * (a key's norm is then scale * ||k8||, the key the scoring kernel scores);
 * w_now, w_prev [batch, 64] fp32; margins [batch, ceil(prev_length /
 * block_size)] float64 over the first prev_length keys, block_size <= 4096;
 * queries and keys 16-byte aligned.  Computed in float64. */
int dsa_certified_margins(const void* q_now, const void* q_prev, const float* w_now, const float* w_prev,
                          const void* keys, const float* key_scales, int64_t key_stride, int64_t batch,
                          int64_t prev_length, int32_t block_size, int32_t key_dtype, double* margins, void* stream);

/* ------------------------------------------------------------------------
 * Sidecar encoder epilogues (sidecar.py:10-88).  The projections wq / wk /
 * weights_proj run in dsa_project_rows / dsa_project_rows_pair (a decode
 * step) or dsa_project_gemm (below); these entry points run everything after
 * them in one pass per row.  dtype codes: DSA_DTYPE_F32
 * or DSA_DTYPE_BF16; arithmetic follows torch's per-op rounding in that dtype.
 * ------------------------------------------------------------------------ */

/* apply_noninterleaved_rope (sidecar.py:10-28) on the first rope_dim dims of
 * every head: x, out [tokens][heads][dim] (dim even, <= 256), positions [tokens]
 * (one position per token, shared by its heads), inv_freq_i = theta^(-i/half),
 * pairs (i, i + half) rotated by position * inv_freq_i. */
int dsa_rope(const void* x, void* out, const int64_t* positions, int64_t tokens, int32_t heads,
             int32_t dim, int32_t rope_dim, float theta, int32_t dtype, void* stream);

/* Decode-step projections (sidecar.py:74-88: wq / wk on bf16 hidden,
 * weights_proj on hidden.float()) for 1..16 tokens, weight-streaming:
 * out[t][n] = sum_k hidden[t][k] * weight[n][k] with hidden bf16
 * [tokens][hidden_stride], weight [features][kdim] row-major (a Linear's
 * weight) and fp32 accumulation.  weight_dtype DSA_DTYPE_BF16: MFMA, features
 * a multiple of 16, out bf16 (rounded once); DSA_DTYPE_F32: fp32 FMAs, out
 * fp32.  kdim a multiple of 32. */
int dsa_project_rows(const void* hidden, int64_t hidden_stride, int64_t tokens, const void* weight,
                     int32_t weight_dtype, int64_t features, int64_t kdim, void* out, int64_t out_stride, void* stream);

/* encode_queries' two projections of one hidden batch (sidecar.py:78-79:
 * wq(hidden) and weights_proj(hidden.float())) in one launch: out_bf16 as
 * dsa_project_rows with a bf16 weight [features_bf16][kdim], out_f32 as
 * dsa_project_rows with an fp32 weight [features_f32][kdim]; the outputs are
 * identical to the two separate calls.  The reference computes them as two
 * Linear calls; the pairing saves a launch per decode step. */
int dsa_project_rows_pair(const void* hidden, int64_t hidden_stride, int64_t tokens, int64_t kdim,
                          const void* weight_bf16, int64_t features_bf16, void* out_bf16, int64_t out_bf16_stride,
                          const float* weight_f32, int64_t features_f32, float* out_f32, int64_t out_f32_stride,
                          void* stream);

/* The sidecar's projections for batches of tokens (sidecar.py:55-58 wq /
 * wk / weights_proj as used by encode_keys / encode_queries, :74-88), on
 * MFMA: out[t][f] = sum_k hidden[t][k] * weight[f][k].  The reference's
 * nn.Linear calls; dsa_project_rows serves a decode step of at most 16
 * tokens, this entry point any token count.
 *   weight_dtype DSA_DTYPE_BF16: hidden bf16, fp32 accumulation, out bf16
 *     (rounded once).  With positions (int64 [tokens]) the output stage also
 *     applies encode_queries' RoPE (sidecar.py:10-28, 81-82) to every
 *     128-feature head: dims 0..63 rotated, dim d with d + 32, by
 *     position * theta^(-d / 32), with cos / sin and every product and sum
 *     rounded to bf16 as the encoder epilogues round them.  That needs
 *     features a multiple of 256 and dsa_project_gemm_workspace_bytes(tokens)
 *     bytes of workspace (the per-token rotation table); out_scale must be 1.
 *   weight_dtype DSA_DTYPE_F32: hidden bf16 (widened exactly) or fp32, out
 *     fp32 = (hidden . weight) * out_scale, one fp32 product: weights_proj on
 *     hidden.float() times (heads * head_dim)^-0.5 in one pass.
 * kdim a multiple of 8, features a multiple of 4,
 * hidden_stride a multiple of 8 and out_stride of 4 elements; pointers
 * 16-byte aligned; each of hidden, weight and out below 2 GiB. */
int64_t dsa_project_gemm_workspace_bytes(int64_t tokens);
int dsa_project_gemm(const void* hidden, int32_t hidden_dtype, int64_t hidden_stride, int64_t tokens, int64_t kdim,
                     const void* weight, int32_t weight_dtype, int64_t features, void* out, int64_t out_stride,
                     float out_scale, const int64_t* positions, float theta, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* encode_keys after wk (sidecar.py:74-76 and 67-72): LayerNorm over dim
 * (fp32 weight/bias, biased variance, eps), then RoPE on the first rope_dim
 * dims, written to out row out_rows[t] (or t when out_rows is NULL) so that a
 * decode step appends straight into its key cache; a token whose row is
 * outside [0, out_row_limit) is not written.  proj [tokens] rows of
 * proj_row_stride elements (proj_dtype), out rows of out_row_stride elements
 * (out_dtype). */
int dsa_encode_keys_epilogue(const void* proj, int32_t proj_dtype, int64_t proj_row_stride,
                             const float* ln_weight, const float* ln_bias, float ln_eps,
                             const int64_t* positions, int32_t rope_dim, float theta, void* out,
                             int32_t out_dtype, int64_t out_row_stride, const int64_t* out_rows,
                             int64_t out_row_limit, int64_t tokens, int32_t dim, void* stream);

/* encode_queries after wq / weights_proj (sidecar.py:78-88): RoPE on every
 * head of proj [tokens][heads][dim] (dtype) into out, and
 * out_weights = proj_weights * weight_scale (fp32 [tokens][heads]; the
 * reference's scale is (heads * dim)^-0.5). */
int dsa_encode_queries_epilogue(const void* proj, const float* proj_weights, const int64_t* positions,
                                int32_t rope_dim, float theta, float weight_scale, void* out,
                                float* out_weights, int64_t tokens, int32_t heads, int32_t dim,
                                int32_t dtype, void* stream);

/* ------------------------------------------------------------------------
 * Measurement utility (no counterpart in the reference; it serves the
 * roofline's measured peak): one launch that only reads `bytes` of device
 * memory with the decode scoring kernel's grid shape and load pattern
 * (`workgroups` workgroups of 4 waves, 64-key units of 256-byte rows, two
 * units in flight per wave).  bytes must split into whole 16 KiB units per
 * workgroup; sink is 256 floats that are practically never written.  When
 * start_event / stop_event (hipEvent_t, nullable) are given the kernel records
 * them at its own start and end, like the *_timed entry points.
 * ------------------------------------------------------------------------ */
int dsa_stream_read(const void* data, int64_t bytes, int32_t workgroups, float* sink, void* stream,
                    void* start_event, void* stop_event);

#ifdef __cplusplus
}
#endif

#endif /* DSA_AMD_H */
