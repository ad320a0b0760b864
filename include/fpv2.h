/*
 * fpv2.h — C ABI of libfpv2_hip.so, the MI355X (gfx950) implementation of
 * FlashPrefill V2 block-sparse prefill attention.
 *
 * Every entry point takes device pointers, sizes, element strides and a
 * hipStream_t (passed as void* so this header needs no HIP include).  Work is
 * enqueued on that stream; nothing synchronises the host and nothing is
 * allocated: the caller owns every input, output and workspace buffer.
 * Return value: FPV2_OK (0) or a negative fpv2_status; fpv2_last_error()
 * then describes the failure (thread-local string).
 *
 * Layouts (row-major, element strides; the last dimension is contiguous):
 *   q        [Hq,  Lq, D]  query heads, head h uses KV head h / (Hq / Hkv)
 *   k, v     [Hkv, Lk, D]
 *   pooled   [Hkv, Nb, D]  rows and D contiguous, any head stride (a pooled
 *                          cache with spare block capacity is used in place),
 *                          Nb = ceil(rows / block_k)
 *   lists    [Hkv, Nt, Nb] int32 contiguous, Nt = padded_query_length / tile_q
 *   counts   [Hkv, Nt]     int32 contiguous
 *   selected [Hkv, Nt, Nb] uint8 (0/1) contiguous
 * Padding is never materialised: rows at or beyond the valid lengths are
 * treated as zeros on input and are never read.
 */
#ifndef FPV2_H_
#define FPV2_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FPV2_ABI_VERSION 3

typedef enum fpv2_status {
  FPV2_OK = 0,
  FPV2_ERR_ARGUMENT = -1,    /* shape / length / pointer inconsistency     */
  FPV2_ERR_UNSUPPORTED = -2, /* dtype, head_dim or size outside the kernels */
  FPV2_ERR_LAUNCH = -3       /* hipLaunchKernel / hipGetLastError failure   */
} fpv2_status;

typedef enum fpv2_dtype {
  FPV2_F32 = 0,
  FPV2_F16 = 1,
  FPV2_BF16 = 2
} fpv2_dtype;

/* Largest key-block count the fused scoring kernel keeps in LDS. */
#define FPV2_MAX_BLOCKS 8192

/* Selection parameters: the fields of FPV2Config plus the call geometry.
 * Mirrors fpv2/selection.py:30-43 (FPV2Config) and the arguments of
 * block_scores_and_select, selection.py:109-117. */
typedef struct fpv2_select_params {
  int64_t query_heads;         /* Hq                                         */
  int64_t kv_heads;            /* Hkv, divides Hq                            */
  int64_t head_dim;            /* D                                          */
  int64_t padded_query_length; /* Nt * tile_q                                */
  int64_t query_length;        /* valid query rows, (0, padded]              */
  int64_t num_blocks;          /* Nb                                         */
  int64_t key_length;          /* valid keys (pruned-list eligibility)       */
  int64_t offset;              /* absolute key position of query row 0       */
  int64_t block_k;
  int64_t tile_q;
  int64_t sink_tokens;
  int64_t window_tokens;
  int64_t last_n_blocks;
  float scale;
  float alpha;
  int64_t q_head_stride; /* elements between query heads               */
  int64_t q_row_stride;  /* elements between query positions           */
  int64_t pooled_head_stride; /* elements between KV heads of pooled_k,
                                 >= num_blocks * head_dim                 */
} fpv2_select_params;

/* Attention parameters.  Mirrors the argument list of sparse_attention,
 * fpv2/kernel.py:441-459, and the int32 params block it builds at
 * kernel.py:528-548. */
typedef struct fpv2_attn_params {
  int64_t query_heads;
  int64_t kv_heads;
  int64_t head_dim;
  int64_t padded_query_length; /* Nt * tile_q (indexes the block lists)      */
  int64_t query_length;        /* valid query rows                           */
  int64_t out_rows;            /* rows of `out` to write, [query_length,
                                  padded]; rows >= query_length get zeros    */
  int64_t key_length;          /* valid keys                                 */
  int64_t num_blocks;          /* Nb                                         */
  int64_t offset;
  int64_t block_k;
  int64_t tile_q;
  int32_t mean_correction;     /* 0/1: append pooled entries of pruned blocks */
  double scale;                /* scale*log2(e) is formed in double and
                                  rounded once, as kernel.py:546-548        */
  int64_t q_head_stride, q_row_stride;
  int64_t k_head_stride, k_row_stride;
  int64_t v_head_stride, v_row_stride;
  int64_t o_head_stride, o_row_stride;
  int64_t pooled_head_stride; /* elements between KV heads of pooled_k and
                                 pooled_v, >= num_blocks * head_dim        */
} fpv2_attn_params;

/* ABI version (FPV2_ABI_VERSION) and the last error of this thread. */
int fpv2_abi_version(void);
const char* fpv2_last_error(void);

/*
 * Mean-pool `rows` of x[batch, rows, D] into out[batch, num_blocks, D]
 * (rows and D contiguous, out_batch_stride elements between batches), block
 * b averaging rows [b*block_size, (b+1)*block_size); rows >= valid_rows count
 * as zeros.  The mean is computed in float64 and rounded once to the output
 * dtype (= input dtype).  Pooling a range of blocks of a longer sequence is
 * the same call with x and out advanced to the first block.
 * Replaces pool_blocks, fpv2/selection.py:68-80.
 */
int fpv2_pool_blocks(const void* x, void* out, int dtype, int64_t batch,
                     int64_t valid_rows, int64_t num_blocks, int64_t head_dim,
                     int64_t block_size, int64_t batch_stride,
                     int64_t row_stride, int64_t out_batch_stride, void* stream);

/*
 * Pool K and V of one attention layer in a single launch (the two
 * pool_blocks calls of fpv2/patch.py:137-138).  k and v share geometry and
 * strides; pooled_k / pooled_v are [kv_heads, num_blocks, D] with
 * pooled_head_stride elements between heads.
 */
int fpv2_pool_kv(const void* k, const void* v, void* pooled_k, void* pooled_v,
                 int dtype, int64_t kv_heads, int64_t valid_rows,
                 int64_t num_blocks, int64_t head_dim, int64_t block_size,
                 int64_t head_stride, int64_t row_stride,
                 int64_t pooled_head_stride, void* stream);

/*
 * Pooled-QK scoring and block selection, one workgroup per
 * (KV head, query tile); replaces block_scores_and_select,
 * fpv2/selection.py:109-201, fused with compact_block_indices,
 * fpv2/kernel.py:141-184.
 * q_dtype / k_dtype: both FPV2_BF16 or both FPV2_F16 (MFMA path) or both
 * FPV2_F32.  Outputs are optional (NULL skips them):
 *   selected   [Hkv, Nt, Nb] uint8
 *   scores     [Hkv, G, padded_query_length, Nb] float32, raw scale*q.k
 *   lists      selected_ids / selected_counts / pruned_ids / pruned_counts;
 *              give all four or none.
 * num_blocks must not exceed FPV2_MAX_BLOCKS.
 */
int fpv2_score_select(const void* q, const void* pooled_k, int dtype,
                      const fpv2_select_params* params, uint8_t* selected,
                      float* scores, int32_t* selected_ids,
                      int32_t* selected_counts, int32_t* pruned_ids,
                      int32_t* pruned_counts, void* stream);

/*
 * Compact a selection mask into padded ascending block lists:
 * selected_ids = selected blocks ascending, then unselected ascending
 * (a stable argsort of -mask); pruned = ~selected & (min(block_end,
 * key_length) <= tile_first); counts = row sums.
 * Replaces compact_block_indices, fpv2/kernel.py:141-184.
 */
int fpv2_compact_block_indices(const uint8_t* selected, int64_t kv_heads,
                               int64_t num_tiles, int64_t num_blocks,
                               int64_t tile_q, int64_t block_k, int64_t offset,
                               int64_t key_length, int32_t* selected_ids,
                               int32_t* selected_counts, int32_t* pruned_ids,
                               int32_t* pruned_counts, void* stream);

/*
 * Block-sparse FlashAttention-2 forward with pooled mean correction.
 * Replaces the fpv2_sparse_attention Metal kernel and its dispatch,
 * fpv2/kernel.py:187-438 and :441-590.  q, k, v, pooled_k, pooled_v and
 * out share dtype (FPV2_BF16 or FPV2_F16); head_dim in {64, 96, 128, 256}.
 * Ids are clipped to [0, Nb-1] and counts to [0, Nb] as at kernel.py:555-558.
 */
int fpv2_sparse_attention(const void* q, const void* k, const void* v,
                          const void* pooled_k, const void* pooled_v,
                          const int32_t* selected_ids,
                          const int32_t* selected_counts,
                          const int32_t* pruned_ids,
                          const int32_t* pruned_counts, void* out, int dtype,
                          const fpv2_attn_params* params, void* stream);

/*
 * Workspace bytes fpv2_sparse_attention_split needs (0 when split_tiles is
 * 0), or a negative fpv2_status.  The segments of a split tile cover
 * seg_steps 32-key sub-tiles each, counted over the longest walk a split
 * tile can have: every block that starts at or before the last query row,
 * plus ceil(Nb / 32) correction sub-tiles with mean_correction.
 * Workspace: [Hkv * split_tiles * ceil(G * tile_q / 128)] items x segments
 * x 128 rows of (D float32 partial outputs, then (m, l) float32 pairs).
 * No counterpart in the reference: its kernel runs a query tile in one
 * threadgroup (fpv2/kernel.py:248-325).
 */
int64_t fpv2_sparse_attention_split_workspace_bytes(const fpv2_attn_params* params,
                                                    int64_t split_tiles,
                                                    int64_t seg_steps);

/*
 * fpv2_sparse_attention with the last split_tiles query tiles of the call
 * split by key range: each runs as consecutive segments of seg_steps
 * sub-tiles of its walk in separate workgroups, whose unnormalised partials
 * (O, row sum, scale) a second kernel merges into out.  Meant for the dense
 * tail (the last last_n_blocks tiles select every visible block,
 * fpv2/selection.py:191-195), which otherwise walks the whole key range in
 * one workgroup.  The result equals fpv2_sparse_attention's up to float32
 * summation order.  workspace: at least
 * fpv2_sparse_attention_split_workspace_bytes bytes, 16-byte aligned, owned
 * by the caller (no contents are kept between calls); calls that share a
 * workspace on different streams race.  No counterpart in the reference
 * (see above).
 */
int fpv2_sparse_attention_split(const void* q, const void* k, const void* v,
                                const void* pooled_k, const void* pooled_v,
                                const int32_t* selected_ids,
                                const int32_t* selected_counts,
                                const int32_t* pruned_ids,
                                const int32_t* pruned_counts, void* out, int dtype,
                                const fpv2_attn_params* params, int64_t split_tiles,
                                int64_t seg_steps, void* workspace,
                                int64_t workspace_bytes, void* stream);

/* Size of the device scratch array of fpv2_sparse_attention_split_static. */
#define FPV2_SPLIT_SCRATCH_BYTES (64LL << 20)

/*
 * fpv2_sparse_attention_split without a workspace argument and without any
 * allocation: the partials live in a file-scope device array of
 * FPV2_SPLIT_SCRATCH_BYTES, one copy per GPU, kept until the process ends
 * (its address is taken once per device, on the first call with that
 * device current).  A split needing more scratch than that
 * (fpv2_sparse_attention_split_workspace_bytes) fails with
 * FPV2_ERR_UNSUPPORTED before any launch.  Every partial the merge reads is
 * written by the same call, so nothing needs clearing; but all calls on one
 * GPU share the array, so calls that overlap on one GPU (other streams,
 * other threads) race.  No counterpart in the reference; it is for callers
 * that cannot allocate device memory (code under graph capture, serving
 * loops with a fixed memory plan).
 */
int fpv2_sparse_attention_split_static(const void* q, const void* k, const void* v,
                                       const void* pooled_k, const void* pooled_v,
                                       const int32_t* selected_ids,
                                       const int32_t* selected_counts,
                                       const int32_t* pruned_ids,
                                       const int32_t* pruned_counts, void* out, int dtype,
                                       const fpv2_attn_params* params, int64_t split_tiles,
                                       int64_t seg_steps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FPV2_H_ */
