/*
 * kvc.h — C ABI of the MI355X (gfx950) paged KV-cache library, libkvc.so.
 *
 * Every entry point takes plain device/host pointers, sizes and strides and an
 * explicit hipStream_t (passed as void*), returns an int status (KVC_OK == 0),
 * and never allocates device memory: buffers (caches, tables, workspace,
 * staging, pinned host memory) are owned by the caller.  A failed call leaves
 * a human-readable reason in kvc_last_error() (thread-local).
 *
 * Cache layout ("NHD", one tensor per layer for K and one for V):
 *     cache[num_blocks][block_size][num_kv_heads][head_dim]
 * with an arbitrary block stride (so a [num_blocks, 2, block_size, H, D]
 * combined tensor can be passed as two views) and a token stride inside a
 * block.  The heads of one token must be contiguous (head stride == head_dim).
 * A slot is   block_id * block_size + offset_in_block.
 *
 * Reference interfaces (file:line in aojsd/GPU_Offloading) each entry point
 * replaces are cited beside it.  Strides are in ELEMENTS unless the name ends
 * in _bytes.
 */
#ifndef KVC_H_
#define KVC_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum kvc_status {
  KVC_OK = 0,
  KVC_ERR_INVALID_ARG = 1,   /* null pointer, negative size, bad stride   */
  KVC_ERR_UNSUPPORTED = 2,   /* shape/dtype combination not compiled      */
  KVC_ERR_ALIGNMENT = 3,     /* pointer or stride breaks vector alignment */
  KVC_ERR_WORKSPACE = 4,     /* workspace / staging buffer too small      */
  KVC_ERR_HIP = 5            /* a HIP runtime call or launch failed       */
};

/* Library version (major*10000 + minor*100 + patch). */
int kvc_version(void);
/* Static description of a status code. */
const char* kvc_status_string(int status);
/* Detail of the last failed call on this thread ("" if none). */
const char* kvc_last_error(void);

/* ------------------------------------------------------------------------
 * (a5) KV append — slot_mapping scatter.
 * Replaces vLLM _C reshape_and_cache_flash as called at
 *   src/MoE/moe_engine.py:2059-2062 and :2344-2347
 *   (PyTorch twin with identical semantics: moe_engine.py:2196-2198).
 * For every token i < num_tokens with 0 <= slot_mapping[i] < num_blocks*block_size:
 *   key_cache[slot/bs][slot%bs][:][:]   = key[i][:][:]
 *   value_cache[slot/bs][slot%bs][:][:] = value[i][:][:]
 * A negative slot is padding and is skipped (moe_engine.py:3539-3540); an
 * out-of-range slot is also skipped and counted in *oob_count when that
 * device pointer is non-null (the count is accumulated, not reset).
 * Pure byte copy: elem_bytes is the element size (2 for bf16/fp16).
 * ---------------------------------------------------------------------- */
int kvc_reshape_and_cache_flash(
    const void* key, const void* value,
    void* key_cache, void* value_cache,
    const int64_t* slot_mapping,
    int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int64_t num_blocks, int32_t elem_bytes,
    int64_t key_token_stride, int64_t value_token_stride,
    int64_t cache_block_stride, int64_t cache_token_stride,
    int32_t* oob_count, void* stream);

/* ------------------------------------------------------------------------
 * Block-table gather into contiguous [tokens, num_kv_heads, head_dim].
 * New API (the reference engine has no gather; its closed form is
 * cache[bt[seq, :nb]].flatten(0,1)[:len], cf. the un-permute in
 * src/dense/scratch_examples/vllm_paged_attn.py:161-190).
 * Sequence b contributes tokens [seq_starts[b], seq_starts[b] + len_b) of its
 * logical KV (len_b = cu_seq_lens[b+1] - cu_seq_lens[b]) to output rows
 * [cu_seq_lens[b], cu_seq_lens[b+1]).  seq_starts may be null (all zero).
 * max_seq_len bounds every len_b (host-side value, sizes the grid; rows past
 * it are not written).  block_table_width is the number of entries per
 * block-table row.  Rows whose position falls outside the row or whose entry is
 * outside [0, num_blocks) are zero-filled and counted in *oob_count when
 * non-null.  out_rows is the number of rows out_key and out_value hold: output
 * rows outside [0, out_rows) (a cu_seq_lens larger than the outputs) are not
 * written and are counted in *oob_count.
 * ---------------------------------------------------------------------- */
int kvc_gather_kv(
    const void* key_cache, const void* value_cache,
    const int32_t* block_table, int64_t block_table_row_stride,
    int32_t block_table_width,
    const int32_t* cu_seq_lens, const int32_t* seq_starts,
    int32_t batch, int32_t max_seq_len,
    int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int64_t num_blocks, int32_t elem_bytes,
    int64_t cache_block_stride, int64_t cache_token_stride,
    void* out_key, void* out_value, int64_t out_token_stride, int64_t out_rows,
    int32_t* oob_count, void* stream);

/* ------------------------------------------------------------------------
 * (a6/a7/a8) Paged GQA decode attention (bf16 in/out, fp32 accumulate).
 * Replaces FlashInfer BatchDecodeWithPagedKVCacheWrapper.plan/run as called at
 *   src/MoE/moe_engine.py:1352-1358, :1949-1955 (plan) and :3907-3909 (run).
 * Request b attends over the pages indices[indptr[b] .. indptr[b+1]) where
 * the final page holds last_page_len[b] tokens (1..page_size):
 *   out[b][hq] = softmax_t(sm_scale * q[b][hq] . K[t][hq/group]) . V[t][hq/group]
 * group = num_qo_heads / num_kv_heads.  Optional lse[b][hq] receives the
 * natural-log log-sum-exp of the scaled logits (-inf for an empty request).
 *
 * kvc_decode_plan is host-only (no device access), like FlashInfer plan(),
 * which also reads a host indptr.  It cuts the batch's flattened page list
 * into num_segments segments per group of heads_per_group KV heads (by
 * default one per workgroup the GPU holds at once; num_segments_hint > 0
 * forces the count), balanced in pages plus switches between requests (at
 * most 128 pages each), and writes the plan image into plan_host:
 *   [0, 4*num_segments)          (first piece, end piece, first slot, pages)
 *   [pieces_offset, +8*pieces)   (request, first slot, end slot, partial or -1,
 *                                 request's last slot, its tokens, 0, 0)
 *   [nparts_offset, +batch)      pieces per request
 * last_page_len_host (tokens in each request's final page) is copied into
 * the pieces so that the kernel needs no dependent load at a piece switch.
 * (plan_ints int32 in total; kvc_decode_plan_ints gives the size for a
 * segment count).  If plan_capacity is too small it fills schedule->plan_ints
 * and returns KVC_ERR_WORKSPACE.  The caller copies the image to the device
 * and passes it to kvc_batch_decode_run.  Pieces of one request are merged
 * with the log-sum-exp rule of src/dense/offload_kv_attn.py:24-39;
 * kvc_decode_workspace_bytes sizes the fp32 partials.
 * ---------------------------------------------------------------------- */
typedef struct kvc_decode_schedule {
  int32_t batch;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_size;
  int32_t num_segments;     /* segments per group of KV heads              */
  int32_t num_head_groups;  /* ceil(num_kv_heads / heads_per_group)        */
  int32_t num_pieces;
  int32_t pieces_offset;    /* int32 offsets inside the plan image         */
  int32_t nparts_offset;
  int32_t max_partitions;   /* max pieces of one request                   */
  int32_t total_pages;      /* indptr[batch]                               */
  int32_t num_empty;        /* requests with no pages (output zero)        */
  int32_t heads_per_group;  /* KV heads one workgroup streams together     */
  int64_t plan_ints;        /* int32 entries of the plan image             */
  int64_t workspace_bytes;  /* bytes kvc_batch_decode_run will use         */
  int32_t append_pieces;    /* most leading pieces of a segment that reach
                               a request end (fused append supports <= 4)  */
  int32_t small_batch;      /* 1: one workgroup per (request, KV head), its
                               waves splitting the pages (see below)       */
} kvc_decode_schedule;

int64_t kvc_decode_plan_ints(int32_t batch, int32_t num_segments);

int kvc_decode_plan(const int32_t* indptr_host, const int32_t* last_page_len_host,
                    int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                    int32_t head_dim, int32_t page_size,
                    int32_t num_segments_hint, int32_t num_cus,
                    kvc_decode_schedule* schedule, int32_t* plan_host,
                    int64_t plan_capacity);

int64_t kvc_decode_workspace_bytes(int32_t batch, int32_t num_qo_heads,
                                   int32_t head_dim, int32_t max_partitions);

/* plan: the device copy (16-byte aligned) of the image kvc_decode_plan wrote.
 * The kernels take every request's page span and last-page length from the
 * plan image (kvc_decode_plan copies them from the host indptr and
 * last_page_len); the device indptr and last_page_len arguments are accepted
 * for symmetry with FlashInfer's run() and are not read (they may be null).
 * So lengths changed on the device after kvc_decode_plan are not seen: plan
 * again, as FlashInfer requires after every change of the lengths.  The page
 * ids themselves (indices) are read on the device at run time. */
int kvc_batch_decode_run(
    const kvc_decode_schedule* schedule, const int32_t* plan,
    const void* q, int64_t q_batch_stride,
    const void* key_cache, const void* value_cache,
    int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t num_blocks,
    const int32_t* indptr, const int32_t* indices, int64_t num_indices,
    const int32_t* last_page_len,
    float sm_scale,
    void* workspace, int64_t workspace_bytes,
    void* out, int64_t out_batch_stride, float* lse, void* stream);

/* Allocation-free decode run.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation).  Same arguments and
 * results as kvc_batch_decode_run without the workspace: the split-K
 * partials live in a device array of the library (KVC_NOALLOC_SCRATCH_BYTES
 * bytes, one per GPU, held until the process ends).  The call allocates
 * nothing.  A schedule whose workspace_bytes exceed the array is refused with
 * KVC_ERR_WORKSPACE.  The stream must belong to the current device (its first
 * call on a device looks up that device's copy of the array).  All calls on
 * one GPU share the array: calls that overlap on one GPU (other streams,
 * other threads) race on it, so serialize them. */
#define KVC_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)

int kvc_batch_decode_run_noalloc(
    const kvc_decode_schedule* schedule, const int32_t* plan,
    const void* q, int64_t q_batch_stride,
    const void* key_cache, const void* value_cache,
    int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t num_blocks,
    const int32_t* indptr, const int32_t* indices, int64_t num_indices,
    const int32_t* last_page_len,
    float sm_scale,
    void* out, int64_t out_batch_stride, float* lse, void* stream);

/* Fused append + decode for a pure-decode step.  No single counterpart in
 * the reference: it does, in one launch, what the engine does with
 * reshape_and_cache_flash of the step's tokens (moe_engine.py:2344-2347)
 * followed by the decode run (:3907-3909).  Row b of new_key / new_value
 * ([batch][num_kv_heads][head_dim], new_*_stride elements between rows) is
 * written to the cache as request b's last token -- page
 * indices[indptr[b+1]-1], offset last_page_len[b]-1, i.e. the slot the step's
 * slot mapping gives it -- and attended with the rest of the request.
 * Requests with no pages append nothing.  The cache and the output equal
 * those of the two separate calls bit for bit.  Needs head_dim 128, a
 * multiple of 8 KV heads, group <= 4 and schedule->append_pieces <= 4;
 * otherwise KVC_ERR_UNSUPPORTED (the caller then makes the two calls). */
int kvc_batch_decode_append_run(
    const kvc_decode_schedule* schedule, const int32_t* plan,
    const void* q, int64_t q_batch_stride,
    void* key_cache, void* value_cache,
    int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t num_blocks, const int32_t* indptr, const int32_t* indices,
    int64_t num_indices, const int32_t* last_page_len,
    const void* new_key, int64_t new_key_stride,
    const void* new_value, int64_t new_value_stride, float sm_scale,
    void* workspace, int64_t workspace_bytes, void* out,
    int64_t out_batch_stride, float* lse, void* stream);

/* ------------------------------------------------------------------------
 * (f2) Paged-KV prefill attention: multi-token queries over the paged cache
 * (bf16 in/out, fp32 accumulate, MFMA).  Replaces FlashInfer
 * BatchPrefillWithPagedKVCacheWrapper.plan/run as called for continuation
 * prefills at src/MoE/moe_engine.py:1733-1751, :3710-3727 (plan) and
 * :3939-3941 (run).
 * Request b's queries are rows qo_indptr[b] .. qo_indptr[b+1] of q (q_len
 * tokens) and its keys the kv_len tokens of pages
 * indices[kv_indptr[b] .. kv_indptr[b+1]) (the final page holding
 * last_page_len[b] tokens).  Query i (0-based in the request) sees key j when
 * j <= i + kv_len - q_len (causal, aligned to the end of the cache, as
 * FlashInfer) or always (causal = 0):
 *   out[qo_indptr[b]+i][hq] = softmax_j(sm_scale q.K[j][hq/group]) . V[j][hq/group]
 * A query that sees no key gets 0 (lse -inf).  Optional lse[row][hq] is the
 * natural-log log-sum-exp of the scaled logits.
 *
 * kvc_prefill_plan is host-only: it cuts every request's queries into tiles
 * of tile_tokens tokens (256 query rows = tile_tokens x group heads), makes
 * one work unit per (tile, KV head) and deals the units to
 * W = min(256, num_items * num_kv_heads) workgroups, one per CU, by list
 * scheduling (longest tiles first, cost = key tiles + 2, workgroup w on XCD
 * w % 8).  The plan image is the workgroups' table, W pairs
 * (first unit, units) padded to a multiple of 4 int32, then
 * num_items * num_kv_heads unit records of 8 int32 in workgroup order:
 *   (KV head, first query, q_len, kv_len, qo_indptr[b], kv_indptr[b],
 *    64-key tiles to visit, pages)
 * If plan_capacity is too small it fills schedule->plan_ints and returns
 * KVC_ERR_WORKSPACE.  The caller copies the image (16-byte aligned) to the
 * device for kvc_batch_prefill_run.  head_dim 128, page_size 16,
 * group 1/2/4/8.
 * ---------------------------------------------------------------------- */
typedef struct kvc_prefill_schedule {
  int32_t batch;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_size;
  int32_t causal;
  int32_t tile_tokens;      /* query tokens per work unit                  */
  int32_t num_items;        /* query tiles (work units per KV head)        */
  int32_t total_q;          /* qo_indptr[batch]                            */
  int32_t max_key_tiles;    /* most 64-key tiles one unit visits           */
  int64_t plan_ints;        /* int32 entries of the plan image             */
} kvc_prefill_schedule;

int kvc_prefill_plan(const int32_t* qo_indptr_host, const int32_t* kv_indptr_host,
                     const int32_t* last_page_len_host, int32_t batch,
                     int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                     int32_t page_size, int32_t causal,
                     kvc_prefill_schedule* schedule, int32_t* plan_host,
                     int64_t plan_capacity);

/* q/out: [total_q][num_qo_heads][head_dim] with a token stride (elements).
 * q, out, the caches and the plan 16-byte aligned, every stride a multiple
 * of 8 elements (KVC_ERR_ALIGNMENT otherwise).  The cache's block stride
 * must stay under 4 GiB (2^31 elements) and a block's 16 tokens under
 * 2 GiB: KVC_ERR_INVALID_ARG otherwise. */
int kvc_batch_prefill_run(
    const kvc_prefill_schedule* schedule, const int32_t* plan,
    const void* q, int64_t q_token_stride,
    const void* key_cache, const void* value_cache,
    int64_t cache_block_stride, int64_t cache_token_stride,
    int64_t num_blocks, const int32_t* indices, int64_t num_indices,
    float sm_scale, void* out, int64_t out_token_stride, float* lse, void* stream);

/* ------------------------------------------------------------------------
 * (f3) vLLM's x-packed paged layout (src/dense/include/paged_transformer.py:85-92):
 *   key_cache   [num_blocks][H][head_size/x][block_size][x]   x = 16 B / element
 *   value_cache [num_blocks][H][head_size][block_size]
 * Strides are in elements; the innermost three (two) dimensions are packed,
 * block and head strides are parameters (the same for K and V).
 * Supported: 2-byte elements (x = 8), head_size 128, block_size 16.
 *
 * kvc_reshape_and_cache_xpacked replaces vLLM _C reshape_and_cache as called
 * at paged_transformer.py:290-294: for every token i with slot s >= 0,
 *   key_cache[s/16][h][d/8][s%16][d%8] = key[i][h][d]
 *   value_cache[s/16][h][d][s%16]      = value[i][h][d]
 * (bit copies; slot < 0 skipped; slot >= num_blocks*16 skipped and counted
 * in the optional *oob_count).
 * ---------------------------------------------------------------------- */
enum { KVC_DTYPE_FP16 = 0, KVC_DTYPE_BF16 = 1 };

int kvc_reshape_and_cache_xpacked(
    const void* key, const void* value, void* key_cache, void* value_cache,
    const int64_t* slot_mapping, int64_t num_tokens, int32_t num_heads, int32_t head_size,
    int32_t block_size, int32_t x, int64_t num_blocks, int64_t key_token_stride,
    int64_t value_token_stride, int64_t cache_block_stride, int64_t cache_head_stride,
    int32_t* oob_count, void* stream);

/* Decode attention over the x-packed layout; replaces vLLM _C
 * paged_attention_v1 / paged_attention_v2 as called at
 * paged_transformer.py:325-332 and scratch_examples/vllm_paged_attn.py:274-288:
 *   out[b][hq] = softmax_t(scale q[b][hq].K[t][hq/group]) . V[t][hq/group]
 * over the seq_lens[b] tokens of block_tables[b][...], group =
 * num_heads / num_kv_heads (1/2/4/8), fp32 accumulation, p rounded to the
 * cache dtype before the value product (as vLLM's kernel).  out is
 * [num_seqs][num_heads][head_size] (packed).  v2 splits every sequence into
 * 512-token partitions and leaves vLLM's scratch: max_logits[b][hq][p] (max
 * scaled logit), exp_sums[b][hq][p] (sum of exp(logit - max)) and
 * tmp_out[b][hq][p][:] (the partition's normalised output), each with
 * max_num_partitions >= ceil(max_seq_len / 512) entries per (b, hq), then
 * combines them.  max_seq_len must bound every seq_lens[b]. */
int kvc_paged_attention_v1(
    void* out, const void* query, int64_t q_stride, const void* key_cache,
    const void* value_cache, int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_size, float scale, const int32_t* block_tables, int64_t block_table_stride,
    int32_t max_blocks_per_seq, const int32_t* seq_lens, int32_t block_size,
    int32_t max_seq_len, int64_t num_blocks, int32_t dtype, int64_t kv_block_stride,
    int64_t kv_head_stride, void* stream);

int kvc_paged_attention_v2(
    void* out, float* exp_sums, float* max_logits, void* tmp_out, int32_t max_num_partitions,
    const void* query, int64_t q_stride, const void* key_cache, const void* value_cache,
    int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads, int32_t head_size, float scale,
    const int32_t* block_tables, int64_t block_table_stride, int32_t max_blocks_per_seq,
    const int32_t* seq_lens, int32_t block_size, int32_t max_seq_len, int64_t num_blocks,
    int32_t dtype, int64_t kv_block_stride, int64_t kv_head_stride, void* stream);

/* ------------------------------------------------------------------------
 * (a8) Merge two attention states, fp32 math:
 *   lse = logaddexp(lse1, lse2); out = out1*e^(lse1-lse) + out2*e^(lse2-lse)
 * Restates src/dense/offload_kv_attn.py:24-39 on the device.  out* are bf16
 * [n, head_dim] rows, lse* fp32 [n] natural log.  out may alias out1 or out2;
 * lse (nullable) must not alias lse1 or lse2.
 * ---------------------------------------------------------------------- */
int kvc_merge_attention_states(const void* out1, const float* lse1,
                               const void* out2, const float* lse2,
                               int64_t n, int32_t head_dim,
                               void* out, float* lse, void* stream);

/* ------------------------------------------------------------------------
 * (a10) KV block eviction / restore.  New API; precedents are
 * kv_snapshot/kv_restore (src/MoE/moe_engine.py:4163-4183) and the pinned
 * H2D/D2H side-stream pipeline (src/dense/include/paged_offload_transformer.py:
 * 111-134, 394-418).
 * staging layout: [n][2][block_bytes]  (K block then V block), where
 * block_bytes = block_size * num_kv_heads * head_dim * elem_bytes and a block
 * occupies block_bytes contiguous bytes at cache + id * cache_block_stride_bytes.
 * Ids outside [0, num_blocks) are skipped and counted in *oob_count.
 * ---------------------------------------------------------------------- */
int kvc_gather_blocks(const void* key_cache, const void* value_cache,
                      int64_t cache_block_stride_bytes, int64_t block_bytes,
                      int64_t num_blocks, const int32_t* block_ids,
                      int64_t n, void* staging, int32_t* oob_count,
                      void* stream);

int kvc_scatter_blocks(const void* staging, const int32_t* block_ids,
                       int64_t n, void* key_cache, void* value_cache,
                       int64_t cache_block_stride_bytes, int64_t block_bytes,
                       int64_t num_blocks, int32_t* oob_count, void* stream);

/* Swap out: gather the n blocks to the device staging buffer then
 * hipMemcpyAsync them to host_dst ([n][2][block_bytes], pinned host memory),
 * in chunks of at most staging_bytes, all on `stream`.  Swap in is the
 * reverse (H2D into staging, then scatter into dst block ids).  Both return as
 * soon as the work is enqueued.  The copies are the bottleneck (the gathers
 * and scatters run at HBM speed, ~1% of the copy time): with 64 MiB of staging
 * a swap runs at the host link's rate (55 GB/s each way measured on MI355X
 * for 512 MiB); smaller staging costs a fixed overhead per chunk (47-49 GB/s
 * at 8 MiB).  Run them on a side stream to overlap other work. */
int kvc_swap_out(const void* key_cache, const void* value_cache,
                 int64_t cache_block_stride_bytes, int64_t block_bytes,
                 int64_t num_blocks, const int32_t* block_ids, int64_t n,
                 void* staging, int64_t staging_bytes, void* host_dst,
                 int32_t* oob_count, void* stream);

int kvc_swap_in(const void* host_src, const int32_t* block_ids, int64_t n,
                void* key_cache, void* value_cache,
                int64_t cache_block_stride_bytes, int64_t block_bytes,
                int64_t num_blocks, void* staging, int64_t staging_bytes,
                int32_t* oob_count, void* stream);

/* ------------------------------------------------------------------------
 * (f1) Step-setup metadata on the device.
 * kvc_compute_slot_mapping replaces vLLM prepare_pos_seq_lens +
 * _compute_slot_mappings_kernel as called at src/MoE/moe_engine.py:3514-3541
 * (eager twins :1308-1316, :2677-2695).  Request r (seq id seq_ids[r]) owns
 * tokens [query_start_loc[r], query_start_loc[r+1]); token i of it sits at
 * position num_computed[seq_ids[r]] + (i - query_start_loc[r]) and its slot is
 *   block_table[seq, pos / block_size] * block_size + pos % block_size.
 * An unallocated entry (-1) yields a negative slot, which the append skips,
 * exactly as the reference formula does.  Token slots [num_tokens,
 * num_tokens_padded) are set to -1 (PAD) and their positions to 0; tokens whose
 * seq id is outside [0, block_table_rows) or whose page is outside the row
 * also get slot -1.  positions may be null.
 *
 * kvc_copy_page_indices replaces _copy_page_indices_kernel + the row
 * index_select at moe_engine.py:1937-1946: for request r (block-table row
 * seq_ids[r], or r when seq_ids is null)
 *   indices[indptr[r] + j] = block_table[row][j],  j < indptr[r+1]-indptr[r].
 * Entries at or past indices_capacity (the buffer's length) are not written.
 * ---------------------------------------------------------------------- */
int kvc_compute_slot_mapping(
    const int32_t* block_table, int64_t block_table_row_stride,
    int32_t block_table_rows, int32_t max_pages_per_seq,
    const int32_t* seq_ids, const int32_t* query_start_loc,
    const int32_t* num_computed, int32_t num_reqs,
    int32_t num_tokens, int32_t num_tokens_padded, int32_t block_size,
    int64_t* slot_mapping, int32_t* positions, void* stream);

int kvc_copy_page_indices(const int32_t* block_table,
                          int64_t block_table_row_stride,
                          int32_t block_table_rows,
                          const int32_t* seq_ids, const int32_t* indptr,
                          int32_t num_reqs, int32_t max_pages_per_req,
                          int32_t* indices, int64_t indices_capacity, void* stream);

/* kvc_stage_from_host replaces the pinned-buffer .copy_(..., non_blocking=True)
 * uploads of the step metadata at src/MoE/moe_engine.py:3493-3494, 3506-3507
 * with one kernel on `stream`:
 *   dev[i] = host[i]  for i in [0, head) and [tail_begin, tail_end)   (int32)
 * read from the pinned image when the kernel runs, so `host` must stay
 * unchanged until then (wait for an event recorded after this call).  `host`
 * must be pinned host memory (hipHostMalloc, torch pin_memory) and both
 * buffers 16-byte aligned; tail_begin is a multiple of 4 and
 * 0 <= head <= tail_begin <= tail_end.  The upload runs on the compute queue:
 * a hipMemcpyAsync of pinned memory goes to a copy engine, which the compute
 * queue then waits for. */
int kvc_stage_from_host(const int32_t* host, int32_t* dev, int64_t head,
                        int64_t tail_begin, int64_t tail_end, void* stream);

/* kvc_decode_step_setup is the engine's whole pure-decode step setup in one
 * launch: the pinned uploads (src/MoE/moe_engine.py:3493-3494, 3506-3507),
 * the block-table writes the scheduler made since the last step, vLLM's
 * prepare_pos_seq_lens + _compute_slot_mappings_kernel for one new token per
 * request (:3514-3541), the device lengths (:3554-3556) and the page-index
 * flatten of FlashInfer's plan (:1937-1946).  From the pinned int32
 * host_image (layout below, offsets in int32 units):
 *   dev_image[i] = host_image[i] for i in [0, plan_ints) and
 *                  [tail_begin, tail_end)  (the decode plan and the fields);
 *   block_table[p / max_pages_per_seq][p % max_pages_per_seq] = bt_val[k]
 *       for the distinct int64 flat positions p = bt_pos[k], k < num_bt_writes
 *       (positions outside the table are skipped);
 *   seq_lens[i] = lens_after[i], i < max_seqs;
 *   slot_mapping[r] = block_table[ids[r]][pos / bs] * bs + pos % bs with
 *       pos = positions[r] (the new token's position), r < num_reqs, and -1
 *       for r in [num_reqs, num_slots) and for rows or pages outside the table;
 *   indices[indptr[r] + j] = block_table[ids[r]][j], j < indptr[r+1]-indptr[r]
 *       (entries at or past indices_capacity are not written),
 * every read of the table seeing the step's writes.  The fields are read
 * from the image when the kernel runs: keep host_image unchanged until an
 * event recorded after this call has completed.  host_image must be pinned
 * (hipHostMalloc, torch pin_memory), both images 16-byte aligned, the
 * block-table rows contiguous (flat positions count max_pages_per_seq per
 * row).  Every field must lie in [tail_begin, tail_end). */
typedef struct kvc_decode_step_layout {
  int64_t plan_ints;    /* [0, plan_ints): the decode plan image            */
  int64_t tail_begin;   /* [tail_begin, tail_end): the step's fields,       */
  int64_t tail_end;     /*   tail_begin a multiple of 4                     */
  int64_t ids;          /* int32[num_reqs]: block-table row of request r    */
  int64_t positions;    /* int32[num_reqs]: position of its new token       */
  int64_t indptr;       /* int32[num_reqs + 1]: page offsets                */
  int64_t lens_after;   /* int32[max_seqs]: every row's length after it     */
  int64_t bt_pos;       /* int64[num_bt_writes] (even offset): flat positions */
  int64_t bt_val;       /* int32[num_bt_writes]: page ids written there     */
  int32_t num_reqs;
  int32_t num_bt_writes;
  int32_t max_seqs;
  int32_t block_size;
} kvc_decode_step_layout;

int kvc_decode_step_setup(const int32_t* host_image, int32_t* dev_image,
                          const kvc_decode_step_layout* layout,
                          int32_t* block_table, int64_t block_table_row_stride,
                          int32_t block_table_rows, int32_t max_pages_per_seq,
                          int32_t* seq_lens, int64_t* slot_mapping, int32_t num_slots,
                          int32_t* indices, int64_t indices_capacity, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVC_H_ */
