/*
 * dsa_capi.h -- C ABI of the MI355X (gfx950) DSA operator library, libdsa_hip.so.
 *
 * Every entry point takes plain device pointers, 64-bit sizes and a HIP
 * stream (passed as void*), launches only on that stream, never
 * synchronises, and returns a status code.  Arguments are validated by
 * HIP-free host code before any launch, so every error path can be exercised
 * without a GPU.  The caller owns all memory: outputs and the workspace are
 * allocated by the caller; `*_workspace_size` reports how many workspace
 * bytes a call needs (a two-phase pattern like the aclnn
 * GetWorkspaceSize/execute pair used by the reference's CANN baselines,
 * sfa_grad_cann.py:40-55).
 *
 * Tensor conventions (row-major, contiguous):
 *   rows  R  = B*S1 (query layout BSND) or T1 (query layout TND)
 *   query [R, N1, D], query_rope [R, N1, Dr], sparse_indices [R, K] int32
 *   key / key_rope  [KV, D] / [KV, Dr] with KV = B*S2 (BSND), T2 (TND) or
 *                   blocks*page_size (PA_BSND, with block_table [B, max_blocks])
 *   softmax_max / softmax_sum [R, N1] fp32 (the reference's [B,1,S1,N1] or
 *                   [1,T1,N1] tensors, which have the same memory order).
 * actual_seq_q / actual_seq_kv are int32 device arrays of B entries: per-batch
 * lengths for BSND and PA_BSND (NULL = full length), cumulative lengths for
 * TND (required), exactly as the reference's Python API receives them.
 */
#ifndef DSA_CAPI_H
#define DSA_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define DSA_OK 0
#define DSA_ERR_INVALID 1     /* bad argument: the reference raises ValueError */
#define DSA_ERR_UNSUPPORTED 2 /* configuration outside the supported set (ValueError) */
#define DSA_ERR_HIP 3         /* HIP runtime error (RuntimeError) */
#define DSA_ERR_WORKSPACE 4   /* workspace missing or smaller than *_workspace_size */

/* element types */
#define DSA_DTYPE_BF16 0
#define DSA_DTYPE_FP16 1
#define DSA_DTYPE_FP32 2

/* layouts */
#define DSA_LAYOUT_BSND 0
#define DSA_LAYOUT_TND 1
#define DSA_LAYOUT_PA_BSND 2

/* Message of the last failed call on this thread ("" if none). */
const char* dsa_last_error(void);

/* Library ABI version (bumped on any signature change). */
int dsa_abi_version(void);

/*
 * Test hook, no counterpart in the reference: flags that route calls through
 * code paths normal sizes do not reach, so that tests can run them at small
 * shapes.  Bit 0 (DSA_TEST_FORCE_GLOBAL_GATHER): the kernels gather key rows
 * with 64-bit global addresses, the path key tensors of 2 GiB or more take,
 * instead of 32-bit buffer offsets.  Process-wide; 0 in normal use.
 */
#define DSA_TEST_FORCE_GLOBAL_GATHER 1
/* Bit 1: dsa_sfa_bwd plans its row chunks for a 64 KiB workspace budget (so
 * that small problems run several chunks); set it around both the
 * workspace query and the call. */
#define DSA_TEST_SMALL_BWD_CHUNKS 2
/* Bit 2: dsa_kl_bwd / dsa_kl_bwd_ex take their generic path (the one for
 * index shapes outside the fused row kernel) at every shape. */
#define DSA_TEST_KL_GENERIC 4
/* Bit 3: D = 512 forwards run the 128-head workgroup kernel without the
 * column-split P.V product (the D < 512 kernel) instead of the column-split
 * kernels; set it around both the workspace query and the call. */
#define DSA_TEST_FWD_WIDE 8
/* Bit 4: dsa_li_fwd / dsa_li_fwd_paged run the scores and the top-k as two
 * launches even where one launch does both. */
#define DSA_TEST_LI_UNFUSED 16
/* Bit 5: the indexer's scores of two query rows per batch (S1 = 2) run the
 * one-row kernel (each row streams its keys) instead of the two-row one. */
#define DSA_TEST_LI_NO_PAIR 32
void dsa_set_test_flags(int32_t flags);

/*
 * Calibration hook, no counterpart in the reference: one launch of a
 * streaming-read kernel over `bytes` bytes of `buffer` (16-byte aligned,
 * a multiple of 16), each byte read once with plain or, when `nontemporal`
 * is set, non-temporal 16-byte loads.  Timed by the caller (events around
 * the launch on `stream`), it gives the read rate that HBM-bound kernels of
 * this library can reach on the device.  `sink` may be NULL (a word the
 * kernel writes only to keep its loads).  Status codes as below.
 */
int dsa_calib_stream_read(const void* buffer, size_t bytes, int32_t nontemporal, uint32_t* sink, void* stream);

/*
 * Sparse flash attention forward, MLA-absorb (value = key[..., :D]), MQA (N2 = 1).
 * Replaces the reference core `_sfa_core` (sparse_flash_attention_triton.py:445-477)
 * and the host-side layout normalisation around it (551-611): TND rows,
 * PA_BSND block_table paging and block-wise indices (sparse_block_size > 1)
 * are handled inside the kernel.
 *   D in {128, 256, 512}, d_rope = 64, 1 <= N1 <= 128, dtype BF16 or FP16,
 *   sparse_mode 0 (full) or 3 (rightDownCausal).
 * pre_tokens / next_tokens (the reference's arguments of those names, which
 * it accepts only at their default INT64_MAX, 531-532) select a band: token
 * t of query row s1 is visible iff diag - pre_tokens <= t <= diag +
 * next_tokens, diag = s1 in mode 0 and act_kv - act_q + s1 in mode 3 (the
 * band of the Ascend FlashAttention operators).  INT64_MAX on a side leaves
 * it open; negative values are allowed.
 * Writes attention_out [R, N1, D]; when return_lse != 0 also softmax_max /
 * softmax_sum [R, N1] (entries of rows without a visible token are 0).  With
 * return_lse == 0, softmax_max and softmax_sum, when both are given, receive
 * zeros (the reference's outputs when the statistics are not requested), so
 * the caller needs no fill of its own; NULL leaves them unwritten.
 */
int dsa_sfa_fwd(const void* query, const void* query_rope, const void* key,
                const void* key_rope, const int32_t* sparse_indices,
                void* attention_out, float* softmax_max, float* softmax_sum,
                const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                const int32_t* block_table, int64_t batch, int64_t s1, int64_t s2,
                int64_t n1, int64_t d, int64_t d_rope, int64_t sparse_count,
                int64_t q_rows, int64_t kv_rows, int64_t max_blocks,
                int64_t page_size, int32_t sparse_block_size, int32_t sparse_mode,
                int64_t pre_tokens, int64_t next_tokens,
                int32_t layout_query, int32_t layout_kv, int32_t dtype,
                float scale_value, int32_t return_lse, void* workspace,
                size_t workspace_bytes, void* stream);

/* Workspace bytes dsa_sfa_fwd needs for these sizes on the current device:
 * the split partials of rows split into token ranges, which happens when
 * there are fewer rows than CUs and, at d = 512, when a row's positions
 * (sparse_count * sparse_block_size) exceed one 2048-entry index list; 0
 * when no row is split. */
size_t dsa_sfa_fwd_workspace_size(int64_t q_rows, int64_t n1, int64_t d,
                                  int64_t sparse_count, int32_t sparse_block_size);

/*
 * dsa_sfa_fwd without a workspace argument, and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops or harnesses
 * that forbid hipMalloc).  Arguments and results are dsa_sfa_fwd's; the
 * split partials go to a fixed 64 MiB device array inside the library (one
 * per GPU, held until the process ends), whose address is looked up on the
 * first call on each device (make one eager call on a device before
 * capturing this entry point into a HIP graph).  Rows longer than one index
 * list whose split partials would exceed 64 MiB run one split per row
 * through the chunked kernel instead; sizes whose workspace still exceeds
 * 64 MiB are rejected with DSA_ERR_UNSUPPORTED (on a 256-CU MI355X no
 * supported shape needs more than about 51 MB).  The array is shared by
 * every call on a GPU: calls that overlap on one device (concurrent streams
 * or threads) race and must be serialised by the caller.
 */
int dsa_sfa_fwd_noalloc(const void* query, const void* query_rope, const void* key,
                        const void* key_rope, const int32_t* sparse_indices,
                        void* attention_out, float* softmax_max, float* softmax_sum,
                        const int32_t* actual_seq_q, const int32_t* actual_seq_kv,
                        const int32_t* block_table, int64_t batch, int64_t s1, int64_t s2,
                        int64_t n1, int64_t d, int64_t d_rope, int64_t sparse_count,
                        int64_t q_rows, int64_t kv_rows, int64_t max_blocks,
                        int64_t page_size, int32_t sparse_block_size, int32_t sparse_mode,
                        int64_t pre_tokens, int64_t next_tokens,
                        int32_t layout_query, int32_t layout_kv, int32_t dtype,
                        float scale_value, int32_t return_lse, void* stream);

/*
 * Sparse flash attention backward, MLA-absorb, MQA.  Replaces the reference
 * core `_sfa_grad_core` (sparse_flash_attention_grad_triton.py:334-376) and
 * the layout handling around it (451-531): TND rows and block-wise indices
 * are resolved in the kernel.  layout applies to query and key alike (BSND
 * or TND), as in the reference.  pre_tokens / next_tokens select the same
 * band as in dsa_sfa_fwd (the reference rejects values other than INT64_MAX,
 * 428-429).  Inputs as dsa_sfa_fwd plus d_out and out
 * [R, N1, D] and the forward's softmax_max / softmax_sum [R, N1] fp32
 * (natural-log units).  Writes d_query [R, N1, D], d_query_rope [R, N1, 64]
 * in the query dtype and d_key / d_value [KV, D], d_key_rope [KV, 64] in the
 * key dtype.  d_key (through the scores) and d_value (through P.dO) are
 * separate, as in the reference; a caller sharing key and value sums them.
 * d_value may be NULL: d_key then receives dk + dv, summed in fp32 before
 * the cast (MLA absorb, value = key[..., :D]: the gradient of the shared
 * latent, which the reference's bprop recipe forms as dk + dv, 30-71).
 * Every output is deterministic (bit-identical between runs): the dK / dV
 * contributions of each (query row, token) are summed over all heads and
 * reduced per key token in integer fixed point, where the reference
 * scatter-adds with fp32 atomics (277-300) and rejects deterministic mode
 * (434-435).  The workspace (dsa_sfa_bwd_workspace_size) holds the
 * per-slot dS / P, the per-token records and their buckets; rows are
 * processed in chunks that keep it within about 24 GiB.
 */
int dsa_sfa_bwd(const void* query, const void* query_rope, const void* key, const void* key_rope,
                const int32_t* sparse_indices, const void* d_out, const void* out,
                const float* softmax_max, const float* softmax_sum, const int32_t* actual_seq_q,
                const int32_t* actual_seq_kv, void* d_query, void* d_query_rope, void* d_key,
                void* d_key_rope, void* d_value, int64_t batch, int64_t s1, int64_t s2, int64_t n1,
                int64_t d, int64_t d_rope, int64_t sparse_count, int64_t q_rows, int64_t kv_rows,
                int32_t sparse_block_size, int32_t sparse_mode, int64_t pre_tokens,
                int64_t next_tokens, int32_t layout, int32_t dtype, float scale_value,
                void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of dsa_sfa_bwd for these sizes; merge_kv != 0 when
 * d_value will be NULL (dk + dv in one output). */
size_t dsa_sfa_bwd_workspace_size(int64_t q_rows, int64_t kv_rows, int64_t n1, int64_t d,
                                  int64_t sparse_count, int32_t sparse_block_size, int32_t merge_kv);

/*
 * Sparse lightning-indexer KL-loss backward.  Replaces the reference core
 * `_sparse_lightning_indexer_grad_kl_loss_core`
 * (sparse_lightning_indexer_grad_kl_loss_triton.py:355-464), i.e. its gather
 * (39-71), fused KL / dQi / dW kernel (74-263), dKi scatter (266-317) and
 * cast (320-327).  BSND only, N2 = Nidx2 = 1, sparse_mode 3 (the API guards,
 * 534-538).  query [B,S1,N1,D], key [B,S2,1,D], query_rope [B,S1,N1,d_rope]
 * and key_rope [B,S2,1,d_rope] (d_rope 0 = no rope, both NULL),
 * query_index [B,S1,Nidx1,d_idx], key_index [B,S2,1,d_idx], weights
 * [B,S1,Nidx1] (dtype weights_dtype), sparse_indices [B,S1,1,topK],
 * softmax_max / softmax_sum [B,1,S1,N1] fp32, actual_seq_qlen /
 * actual_seq_klen [B] (NULL = full lengths).  Writes d_query_index (query
 * index dtype), d_key_index (key index dtype), d_weights (weights dtype)
 * and loss[1] fp32 (sum over rows).  dKi is reduced in a fixed-point sum
 * (no floating-point atomics; the parts of long tokens meet in int64
 * atomics, whose order does not matter), so every output is deterministic.
 * The workspace (dsa_kl_bwd_workspace_size) holds rows * topK * d_idx fp16 slot
 * contributions (scaled by a per-row power of two), the token buckets and
 * kv_rows * d_idx int64 accumulators.  query/key/rope/index tensors share
 * one dtype (bf16 or fp16); D in {128, 256, 512}; N1 <= 128; d_idx a
 * multiple of 8 up to 256; Nidx1 <= 128; topK up to 2^20 with rows * topK
 * < 2^31.  d_idx = 128, Nidx1 <= 64 and topK <= 7168 run one fused row
 * kernel; other shapes a generic path with the same outputs.
 */
int dsa_kl_bwd(const void* query, const void* key, const void* query_rope, const void* key_rope,
               const void* query_index, const void* key_index, const void* weights,
               const int32_t* sparse_indices, const float* softmax_max, const float* softmax_sum,
               const int32_t* actual_seq_qlen, const int32_t* actual_seq_klen, void* d_query_index,
               void* d_key_index, void* d_weights, float* loss, int64_t batch, int64_t s1, int64_t s2,
               int64_t n1, int64_t d, int64_t d_rope, int64_t n_idx, int64_t d_idx, int64_t sparse_count,
               int32_t dtype, int32_t weights_dtype, float scale_value, void* workspace,
               size_t workspace_bytes, void* stream);

/* Workspace bytes of dsa_kl_bwd. */
size_t dsa_kl_bwd_workspace_size(int64_t batch, int64_t s1, int64_t s2, int64_t sparse_count,
                                 int64_t d_idx);

/*
 * dsa_kl_bwd over packed (TND) rows and a paged key cache.  The reference
 * rejects every layout but BSND (sparse_lightning_indexer_grad_kl_loss_triton.py:
 * 534-535); this entry point extends the same computation:
 *   layout_query BSND: query [B*S1, N1, D] rows; TND: [T1 = q_rows, N1, D]
 *     with cumulative actual_seq_qlen [B] (required).
 *   layout_key BSND: key / key_rope / key_index [B*S2, 1, X]; TND:
 *     [T2 = kv_rows, 1, X] with cumulative actual_seq_klen (needs a TND
 *     query); PA_BSND: caches [kv_rows = blocks * page_size, 1, X] addressed
 *     through block_table [B, max_blocks] (int32, -1 = no page), with
 *     per-batch actual_seq_klen (required).
 * Row semantics are dsa_kl_bwd's: row (b, s1) is active when s1 < its query
 * length and covers the first n = min(topK, max(ak - aq + s1 + 1, 0)) slots;
 * token ids are clamped to [0, L) with L = S2 (BSND), the batch's key length
 * (TND) or max_blocks * page_size (PA_BSND).  A token in a -1 page reads as a
 * zero key row and receives no gradient.  d_key_index has the key_index
 * shape and holds the sum over every slot that targets a key row (shared
 * pages included); rows no slot targets are zero.  s1 is read for a BSND
 * query only, s2 for a BSND key only.
 */
int dsa_kl_bwd_ex(const void* query, const void* key, const void* query_rope, const void* key_rope,
                  const void* query_index, const void* key_index, const void* weights,
                  const int32_t* sparse_indices, const float* softmax_max, const float* softmax_sum,
                  const int32_t* actual_seq_qlen, const int32_t* actual_seq_klen, const int32_t* block_table,
                  void* d_query_index, void* d_key_index, void* d_weights, float* loss, int64_t batch,
                  int64_t s1, int64_t s2, int64_t n1, int64_t d, int64_t d_rope, int64_t n_idx, int64_t d_idx,
                  int64_t sparse_count, int64_t q_rows, int64_t kv_rows, int64_t max_blocks, int64_t page_size,
                  int32_t layout_query, int32_t layout_key, int32_t dtype, int32_t weights_dtype,
                  float scale_value, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of dsa_kl_bwd_ex. */
size_t dsa_kl_bwd_ex_workspace_size(int64_t q_rows, int64_t kv_rows, int64_t sparse_count, int64_t d_idx);

/*
 * Dense lightning-indexer softmax LSE (the dense warm-up stage).  Replaces
 * the reference core `_dense_index_stats_core` and its kernel
 * `_dense_indexer_stats_kernel` (dense_loss_backward_triton.py:129-177,
 * 405-432).  BSND: query_index [B,S1,Nidx1,d_idx], key_index [B,S2,1,d_idx],
 * weights [B,S1,Nidx1] (weights_dtype), actual_seq_qlen / actual_seq_klen
 * [B] per-batch lengths (NULL = full).  For a row (b, s1) with s1 < act_q
 * over its visible keys t < min(max(act_k - act_q + s1 + 1, 0), S2):
 * I[t] = sum_g w_g ReLU(qi_g . ki_t), softmax_max_index = max I and
 * softmax_sum_index = sum exp(I - max) (fp32 [B*S1]); -inf / 0 for a row with
 * no visible key.  d_idx in {128, 256, 512}, Nidx1 <= 128.  No workspace.
 */
int dsa_dense_li_softmax_lse(const void* query_index, const void* key_index, const void* weights,
                             const int32_t* actual_seq_qlen, const int32_t* actual_seq_klen,
                             float* softmax_max_index, float* softmax_sum_index, int64_t batch, int64_t s1,
                             int64_t s2, int64_t n_idx, int64_t d_idx, int32_t dtype, int32_t weights_dtype,
                             void* stream);

/*
 * Dense lightning-indexer KL-loss backward (the dense warm-up stage).
 * Replaces `_dense_loss_backward_core` and `_dense_loss_backward_with_index_core`
 * (dense_loss_backward_triton.py:435-655) with their kernels (129-397).
 * query [B,S1,N1,D], key [B,S2,N2,D] (N1 % N2 == 0, GQA), query_rope /
 * key_rope [..,64] or NULL with d_rope = 0, query_index / key_index /
 * weights as dsa_dense_li_softmax_lse, softmax_max / softmax_sum [B,N2,S1,G]
 * fp32 (G = N1/N2).  softmax_max_index / softmax_sum_index: the index LSE
 * ([B*S1] fp32) as given, or both NULL to compute it.  Writes d_query_index,
 * d_key_index (index dtype), d_weights (weights dtype) and loss[1] (sum over
 * rows).  dKeyIndex is reduced without atomics, so every output is
 * deterministic.  D in {128, 256, 512}, N1 <= 128.  The workspace
 * (dsa_dense_kl_bwd_workspace_size) holds the [B*S1, S2] fp32 index-score /
 * dI rows and the dKeyIndex partial sums.
 */
int dsa_dense_kl_bwd(const void* query, const void* key, const void* query_rope, const void* key_rope,
                     const void* query_index, const void* key_index, const void* weights,
                     const float* softmax_max, const float* softmax_sum, const float* softmax_max_index,
                     const float* softmax_sum_index, const int32_t* actual_seq_qlen,
                     const int32_t* actual_seq_klen, void* d_query_index, void* d_key_index, void* d_weights,
                     float* loss, int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t n2, int64_t d,
                     int64_t d_rope, int64_t n_idx, int64_t d_idx, int32_t dtype, int32_t weights_dtype,
                     float scale_value, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of dsa_dense_kl_bwd. */
size_t dsa_dense_kl_bwd_workspace_size(int64_t batch, int64_t s1, int64_t s2, int64_t d_idx);

/*
 * Lightning indexer: scores + stable top-k.  Replaces the reference core
 * `_lightning_indexer_score_core` (lightning_indexer_triton.py:382-413) and the
 * top-k after it (`_stable_topk`, 339-357, called at 539), with the stable
 * order the readme specifies (readme.md:63-69): score descending, index
 * ascending on ties, -inf entries and padding reported as index -1.
 *   query [R1, N1, D] (R1 = B*S1 BSND or T1 TND), key [R2, N2, D] (R2 = B*S2
 *   BSND or T2 TND), weights [R1, N1] (weights_dtype BF16 / FP16 / FP32),
 *   D up to 256 with 16-byte rows (a multiple of 8; of 4 for FP32), N1 % N2
 *   == 0, N1/N2 <= 128, dtype BF16, FP16 or FP32 (FP32 products in full fp32),
 *   sparse_mode 0 or 3.  With a TND query both length arrays are cumulative
 *   (as the reference converts both, 500-506); a TND key needs a TND query.
 *   For a TND key, s2 is the largest per-batch key length (the width of the
 *   score rows).
 * Writes sparse_indices [R1, N2, K] int32 and, when return_value != 0,
 * sparse_values [R1, N2, K] in the query dtype (-inf where the index is -1).
 * With return_value == 0, a sparse_values buffer that is given receives
 * zeros (the reference's values when they are not requested), so the caller
 * needs no fill of its own; NULL leaves it unwritten.
 * The workspace holds the fp32 scores [R1*N2, s2].  K <= 16384.
 */
int dsa_li_fwd(const void* query, const void* key, const void* weights,
               const int32_t* actual_seq_q, const int32_t* actual_seq_k,
               int32_t* sparse_indices, void* sparse_values, int64_t batch, int64_t s1,
               int64_t s2, int64_t n1, int64_t n2, int64_t d, int64_t sparse_count,
               int64_t q_rows, int64_t k_rows, int32_t sparse_mode, int32_t layout_query,
               int32_t layout_key, int32_t dtype, int32_t weights_dtype, int32_t return_value,
               void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of dsa_li_fwd: the fp32 score rows, q_rows * n2 * s2 * 4. */
size_t dsa_li_fwd_workspace_size(int64_t q_rows, int64_t n2, int64_t s2);

/*
 * Indexer scores only (the first stage of dsa_li_fwd; the reference's
 * `_lightning_indexer_score_core`, lightning_indexer_triton.py:382-413):
 * scores [R1*N2, s2] fp32, -inf where masked.  Arguments as dsa_li_fwd.
 */
int dsa_li_scores(const void* query, const void* key, const void* weights,
                  const int32_t* actual_seq_q, const int32_t* actual_seq_k, float* scores,
                  int64_t batch, int64_t s1, int64_t s2, int64_t n1, int64_t n2, int64_t d,
                  int64_t q_rows, int64_t k_rows, int32_t sparse_mode, int32_t layout_query,
                  int32_t layout_key, int32_t dtype, int32_t weights_dtype, void* stream);

/*
 * Stable top-k of fp32 score rows (the second stage of dsa_li_fwd; replaces
 * `_stable_topk`, lightning_indexer_triton.py:339-357): scores [rows, s2] ->
 * indices [rows, K] int32 and, if values != NULL, values [rows, K] fp32.
 * Bit-exact on given scores; K <= 16384; K > s2 pads with -1 / -inf.
 */
int dsa_li_topk_from_scores(const float* scores, int64_t rows, int64_t s2, int64_t sparse_count,
                            int32_t* indices, float* values, void* stream);

/*
 * Lightning indexer over a paged key cache (PA_BSND).  The reference rejects
 * a block_table (lightning_indexer_triton.py:497-498); this entry point is
 * its extension to the paged indexer-key cache of decode, with the paging
 * semantics of the reference's SFA de-paging (sparse_flash_attention_triton.py
 * :382-403): key s2 of batch b is row block_table[b, s2 / page_size] *
 * page_size + s2 % page_size of key_cache [num_blocks, page_size, N2, D], and a
 * -1 (or out-of-range) block reads as a zero key row (score 0 while visible).
 * actual_seq_k holds per-batch key lengths (required); the score rows are
 * max_blocks * page_size wide.  Query, weights, outputs and workspace
 * (dsa_li_fwd_workspace_size(q_rows, n2, max_blocks * page_size)) as
 * dsa_li_fwd; layout_query BSND or TND (cumulative actual_seq_q).
 */
int dsa_li_fwd_paged(const void* query, const void* key_cache, const void* weights,
                     const int32_t* actual_seq_q, const int32_t* actual_seq_k,
                     const int32_t* block_table, int32_t* sparse_indices, void* sparse_values,
                     int64_t batch, int64_t s1, int64_t n1, int64_t n2, int64_t d,
                     int64_t sparse_count, int64_t q_rows, int64_t num_blocks, int64_t page_size,
                     int64_t max_blocks, int32_t sparse_mode, int32_t layout_query, int32_t dtype,
                     int32_t weights_dtype, int32_t return_value, void* workspace,
                     size_t workspace_bytes, void* stream);

/* Scores only of dsa_li_fwd_paged: scores [R1*N2, max_blocks * page_size] fp32. */
int dsa_li_scores_paged(const void* query, const void* key_cache, const void* weights,
                        const int32_t* actual_seq_q, const int32_t* actual_seq_k,
                        const int32_t* block_table, float* scores, int64_t batch, int64_t s1,
                        int64_t n1, int64_t n2, int64_t d, int64_t q_rows, int64_t num_blocks,
                        int64_t page_size, int64_t max_blocks, int32_t sparse_mode,
                        int32_t layout_query, int32_t dtype, int32_t weights_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_CAPI_H */
