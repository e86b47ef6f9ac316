/*
 * tv_attn.h -- C ABI of the MI355X (gfx950) attention hot path for tinyvllm.
 *
 * The reference (jonirajala/tinyvllm) has no FFI: its hot path is three Python
 * functions over tinygrad tensors.  Each entry point below replaces one of them
 * and is bound from Python with ctypes (tinyvllm_amd/_lib.py).
 *
 * Conventions
 *  - All pointers are device pointers (HIP), except where noted.  Buffers are
 *    owned by the caller; no entry point allocates or frees memory.
 *  - `stream` is a hipStream_t (NULL = default stream).  Work is enqueued
 *    asynchronously; device faults surface at the next synchronisation.
 *  - dtype codes: TV_F32 = 0, TV_F16 = 1, TV_BF16 = 2.
 *  - Return value 0 = success; otherwise a TV_E* code and tv_last_error()
 *    returns a message (thread-local, valid until the next call on the thread).
 *  - Layouts are dense row-major unless a stride argument says otherwise:
 *      queries      [num_seqs, 1, num_heads, head_dim]
 *      k/v cache    [num_blocks, block_size, num_kv_heads, head_dim]
 *      block_tables [num_seqs, block_table_stride] int32, zero padded
 *      context_lens [num_seqs] int32
 *      prefill q    [q_len, num_heads, head_dim]      (token stride q_stride)
 *      prefill k/v  [kv_len, num_kv_heads, head_dim]  (token stride k/v_stride)
 */
#ifndef TV_ATTN_H
#define TV_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TV_F32 0
#define TV_F16 1
#define TV_BF16 2

#define TV_OK 0
#define TV_EINVAL 1       /* bad argument (shape, dtype, pointer, size) */
#define TV_EUNSUPPORTED 2 /* valid but not implemented for this shape */
#define TV_EHIP 3         /* HIP runtime error at launch */

/* ABI version of this header (bumped on any signature change). */
int tv_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* tv_last_error(void);

/*
 * Workspace (bytes) needed by tv_paged_decode for the split-context partials:
 * num_seqs * num_heads * ceil(max_blocks*block_size / partition_size)
 * * (head_dim + 2) floats.  When every sequence fits one partition and
 * 32 <= num_seqs <= 1024 it is num_seqs + 1 ints (rounded up to 256 bytes) for
 * a longest-first schedule of the sequences, which tv_paged_decode uses when
 * the caller provides it and skips otherwise; else 0.  Host-only computation.
 */
size_t tv_paged_decode_workspace_bytes(int num_seqs, int num_heads, int head_dim,
                                       int max_blocks, int block_size, int partition_size);

/*
 * Partition size (tokens) for tv_paged_decode on the current device: the whole
 * context (max_blocks*block_size rounded up to 16) when the batch gives at
 * least 4 (sequence, KV head) work-groups per CU; otherwise the context split
 * into as many partitions as make a full-width batch's work-groups fill the
 * GPU's resident work-groups once (occupancy x CUs), rounded up to 16 tokens
 * and at least 64.  No counterpart in the reference (which never splits);
 * queries the device.  Returns 0 on bad arguments (see tv_last_error).
 */
int tv_paged_decode_partition_size(int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                                   int max_blocks, int block_size, int dtype);

/*
 * Paged decode attention.  Replaces paged_decode_attention(...)
 * (tinyvllm/model/llama.py:97-144).
 *   out[b,0,h,:] = softmax_j((q[b,0,h,:] . K[j]) * scale) V[j]
 * over positions j < min(context_lens[b], max_blocks*block_size) of sequence b,
 * where position j lives in block block_tables[b, j / block_size] at row
 * j % block_size, and query head h reads KV head h / (num_heads/num_kv_heads).
 * max_blocks (<= block_table_stride) is the number of table columns used
 * (block_table_stride 0: every sequence reads row 0, e.g. the query rows of one
 * prompt chunk over that sequence's table); the
 * reference's optional max_context_len maps to
 * max_blocks = min(ceil(max_context_len/block_size), block_table_stride).
 * context_lens[b] <= 0 reproduces the reference's all-masked softmax over the
 * whole gathered width.  A block id outside [0, num_blocks) yields NaN outputs
 * for that sequence.
 * partition_size: tokens per work-group (multiple of 16, > 0).  Sequences longer
 * than one partition are split (flash-decoding) and merged by a second kernel;
 * that needs `workspace` of tv_paged_decode_workspace_bytes(...) bytes (for an
 * unsplit launch the workspace is optional and only holds the schedule).
 * q, caches and out share `dtype`; out may instead be TV_F32 (out_dtype).
 */
int tv_paged_decode(void* out, const void* queries, const void* k_cache, const void* v_cache,
                    const int32_t* block_tables, const int32_t* context_lens,
                    int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                    int block_size, int num_blocks, int block_table_stride, int max_blocks,
                    float scale, int dtype, int out_dtype, int partition_size,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * tv_paged_decode without a workspace argument: the split-context partials and
 * the longest-first schedule live in a scratch array that the library holds on
 * each device (16 MiB, allocated with the code object, kept until the process
 * ends).  No counterpart in the reference; for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Arguments and results are those of tv_paged_decode
 * with workspace = that scratch.  A launch whose tv_paged_decode_workspace_bytes
 * exceeds 16 MiB fails with TV_EINVAL.  Allocates nothing; the first call on a
 * device looks the scratch address up once, so make that call eagerly before
 * capturing later calls into a graph.  All calls on one device share the
 * scratch: calls that overlap on one device (different streams, or host
 * threads) race and must be serialised by the caller.
 */
int tv_paged_decode_noalloc(void* out, const void* queries, const void* k_cache, const void* v_cache,
                            const int32_t* block_tables, const int32_t* context_lens,
                            int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                            int block_size, int num_blocks, int block_table_stride, int max_blocks,
                            float scale, int dtype, int out_dtype, int partition_size, void* stream);

/*
 * Prefill attention over one prompt.  Replaces flash_prefill_attention(...)
 * (tinyvllm/model/llama.py:58-94) with the batch dimension (always 1 there)
 * removed.  causal != 0 excludes key j for query i when j > i (top-left
 * aligned, llama.py:86-90).  head_dim_v may differ from head_dim (generic
 * kernel); fp16/bf16 with head_dim in {64,128}, head_dim_v == head_dim and
 * 16-byte aligned rows run on MFMA.  Strides are in elements between
 * consecutive tokens.
 * chunk_tiles: key tiles (of 64) per work unit; long causal rows are split into
 * chunks processed by separate work-groups and merged by a second kernel, which
 * needs `workspace` of tv_flash_prefill_workspace_bytes(...) bytes (0 = no
 * split).  chunk_tiles <= 0 picks a size from the shape: no chunks, except
 * causal head_dim-128 prompts of 2048+ rows whose 128-row query tiles leave at
 * least a quarter of the current device's resident work-group slots free
 * (few heads, e.g. a head-sharded model): their longer tiles run as two key
 * halves merged by a second kernel (the size then depends on the device);
 * that split is optional -- with workspace NULL such a prompt runs unsplit.
 * The workspace must be 16-byte aligned.
 */
size_t tv_flash_prefill_workspace_bytes(int q_len, int kv_len, int num_heads, int head_dim, int head_dim_v,
                                        int causal, int dtype, int chunk_tiles);

int tv_flash_prefill(void* out, const void* q, const void* k, const void* v,
                     int q_len, int kv_len, int num_heads, int num_kv_heads,
                     int head_dim, int head_dim_v,
                     int64_t q_stride, int64_t k_stride, int64_t v_stride, int64_t out_stride,
                     int causal, float scale, int dtype, int out_dtype,
                     int chunk_tiles, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Several prompts in one launch.  No counterpart in the reference, whose engine
 * prefills one sequence per call (engine.py:125-132, llama.py:65-67 asserts
 * batch 1); each prompt is attended exactly as tv_flash_prefill attends it.
 * Prompt z owns rows cu_seqlens_q[z] .. cu_seqlens_q[z+1] of q / out and rows
 * cu_seqlens_k[z] .. cu_seqlens_k[z+1] of k / v (device int32 arrays of
 * num_seqs + 1 entries).  seq_order (device int32 [num_seqs], may be NULL) is
 * the order in which prompts are dispatched -- longest first balances the
 * launch.  max_q_len / max_kv_len must bound every prompt's lengths (rows past
 * max_q_len are not computed); total_q is the sum of query lengths (kernel
 * shape choice only).  fp16 / bf16, head_dim 64 or 128, 16-byte aligned rows
 * (TV_EUNSUPPORTED otherwise); no workspace.
 */
int tv_flash_prefill_varlen(void* out, const void* q, const void* k, const void* v,
                            const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, const int32_t* seq_order,
                            int num_seqs, int max_q_len, int max_kv_len, int64_t total_q,
                            int num_heads, int num_kv_heads, int head_dim,
                            int64_t q_stride, int64_t k_stride, int64_t v_stride, int64_t out_stride,
                            int causal, float scale, int dtype, int out_dtype, void* stream);

/*
 * Prefill attention of one prompt chunk whose keys and values are read from the
 * paged cache.  No counterpart in the reference, whose prefill at start_pos > 0
 * attends within the chunk only (llama.py:184); chunked prefill over the cached
 * prefix is on its roadmap (ROADMAP.md:75-99).  Query row i (q [q_len,
 * num_heads, head_dim], token stride q_stride) sits at position start_pos + i
 * and attends keys 0 .. start_pos + q_len - 1 of the sequence -- with causal,
 * keys j <= start_pos + i -- where key j is row j % block_size of block
 * block_table[j / block_size] of k_cache / v_cache [num_blocks, block_size,
 * num_kv_heads, head_dim] (the chunk's own K/V must already be written).
 * Equal to the last q_len rows of tv_flash_prefill over the whole sequence.
 * fp16 / bf16, head_dim 64 or 128, block_size a power of two, at most 4096
 * table entries (TV_EUNSUPPORTED otherwise).  block_table holds at least
 * ceil((start_pos + q_len) / block_size) entries.  A block id outside
 * [0, num_blocks) is never dereferenced: the rows of every 64-row query tile
 * whose keys include that block come out NaN in every head.
 */
int tv_flash_prefill_paged(void* out, const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* block_table, int num_blocks, int block_size, int q_len, int start_pos,
                           int num_heads, int num_kv_heads, int head_dim, int64_t q_stride, int64_t out_stride,
                           int causal, float scale, int dtype, int out_dtype, void* stream);

/*
 * Fused K/V cache write from a slot mapping.  Replaces the per-chunk
 * KVCache.write_kv loop (tinyvllm/core/kv_cache.py:34-38 called from
 * llama.py:199-209 and llama.py:381-386) with one launch:
 *   k_cache[slot / block_size, slot % block_size] = k[t]   (likewise v)
 * for slot = slot_mapping[t], t < num_tokens.  Negative slots are skipped.
 * k/v rows are num_kv_heads*head_dim contiguous elements; k_stride/v_stride are
 * the element distances between consecutive tokens.  err_count (device
 * uint32, may be NULL) is incremented once per token whose slot is past the
 * cache; such tokens are skipped.
 */
int tv_reshape_and_cache(void* k_cache, void* v_cache, const void* k, const void* v,
                         const int32_t* slot_mapping, int num_tokens,
                         int num_kv_heads, int head_dim, int block_size, int num_blocks,
                         int64_t k_stride, int64_t v_stride, int dtype,
                         uint32_t* err_count, void* stream);

/*
 * KVCache.write_kv(layer_idx, block_id, start_offset, k, v)
 * (tinyvllm/core/kv_cache.py:34-38): tokens t < num_tokens go to
 * [block_id, start_offset + t].  Arguments are validated on the host
 * (block_id in range, start_offset + num_tokens <= block_size).
 */
int tv_write_kv(void* k_cache, void* v_cache, const void* k, const void* v,
                int block_id, int start_offset, int num_tokens,
                int num_kv_heads, int head_dim, int block_size, int num_blocks,
                int64_t k_stride, int64_t v_stride, int dtype, void* stream);

/*
 * KVCache.read_kv_blocks(layer_idx, block_ids, context_len)
 * (tinyvllm/core/kv_cache.py:40-55): gathers the first context_len rows of the
 * listed blocks into k_out/v_out [context_len, num_kv_heads, head_dim].
 * block_ids is a device int32 array of num_block_ids entries;
 * context_len <= num_block_ids*block_size.  Ids outside the cache read as 0.
 */
int tv_read_kv_blocks(void* k_out, void* v_out, const void* k_cache, const void* v_cache,
                      const int32_t* block_ids, int num_block_ids, int context_len,
                      int num_kv_heads, int head_dim, int block_size, int num_blocks,
                      int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TV_ATTN_H */
