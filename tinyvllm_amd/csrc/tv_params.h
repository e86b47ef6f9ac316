// Launch parameter blocks shared by the kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>

namespace tv {

// Prefill attention (flash_prefill.hip).
struct PrefillParams {
  void* out;
  const void* q;
  const void* k;
  const void* v;
  int q_len;
  int kv_len;
  int num_heads;
  int num_kv_heads;
  int head_dim;
  int head_dim_v;
  long long q_stride;    // elements between consecutive tokens
  long long k_stride;
  long long v_stride;
  long long out_stride;
  int causal;
  float scale;
  int out_dtype;
  int xcd_remap;         // 1: place the heads of a KV group on one XCD
  int chunk_tiles;       // key tiles per work unit (long causal rows are split)
  int max_chunks;        // largest number of key chunks of one query tile
  float* part_o;         // [Hq, nqt, max_chunks, 64, head_dim] chunk outputs (split tiles only)
  float* part_ml;        // [Hq, nqt, max_chunks, 64, 2] chunk (max, sum)
  // Several prompts per launch (null: one prompt).  Prompt z's tokens are rows
  // cu_q[z] .. cu_q[z+1] of q / out and cu_k[z] .. cu_k[z+1] of k / v; grid.z
  // runs over seq_order (prompt ids, longest first) when it is set.
  const int* cu_q;
  const int* cu_k;
  const int* seq_order;
  // Keys and values in a paged cache (null: k / v are contiguous rows).  Key
  // j of the prompt is cache row kv_table[j >> kv_bs_log2] * 2^kv_bs_log2 +
  // (j & (2^kv_bs_log2 - 1)); k / v point at the cache base, k_stride /
  // v_stride are the cache row strides (num_kv_heads * head_dim).
  const int* kv_table;
  int kv_bs_log2;
  int kv_num_blocks;     // ids outside [0, kv_num_blocks) make the head's outputs NaN
  // Absolute position of query row 0: causal rows see keys j <= i + q_pos_offset
  // (0: top-left aligned, the reference's prompt; start_pos: a chunk after a
  // cached prefix).
  int q_pos_offset;
  // 128-row kernel: 1 deals query tiles longest first (grids with more
  // work-groups than are resident at once), 0 zig-zag (prefill_rows_kernel).
  int longest_first;
  // 128-row kernel, one causal prompt: query tiles rows_split .. nqt - 1 run
  // as two work-groups over the two halves of their keys (rows_split_unit,
  // tv_paged_keys.h); both halves' normalised rows go to split_o, their
  // (max, sum) to split_ml, and prefill_rows_merge_kernel combines them into
  // out.  rows_split >= nqt: no split.
  int rows_split;
  void* split_o;         // [Hq, nqt - rows_split, 2 halves, 128, head_dim], fp32 or fp16
  float* split_ml;       // [Hq, nqt - rows_split, 2 halves, 128, 2]
};

// Cache write from a slot mapping or a base slot (kv_cache.hip).
struct KVWriteParams {
  void* k_cache;
  void* v_cache;
  const void* k;
  const void* v;
  const int* slots;      // may be null
  int base_slot;
  int num_tokens;
  int row_vecs;          // vectors per cache row (Hkv*D*elem / W)
  long long k_stride;    // vectors between consecutive input tokens
  long long v_stride;
  long long num_slots;   // num_blocks * block_size
  unsigned* err_count;   // may be null
};

// Cache gather for read_kv_blocks (kv_cache.hip).
struct KVGatherParams {
  void* k_out;
  void* v_out;
  const void* k_cache;
  const void* v_cache;
  const int* block_ids;
  int context_len;
  int block_size;
  int row_vecs;
  int num_blocks;
};

bool prefill_uses_mfma(const PrefillParams& p, int dtype);
size_t prefill_workspace_bytes(const PrefillParams& p, int dtype);
int launch_flash_prefill(const PrefillParams& p, int dtype, void* workspace, size_t workspace_bytes,
                         hipStream_t stream);
size_t prefill_rows_workspace_bytes(const PrefillParams& p, int dtype);
bool launch_prefill_rows(const PrefillParams& p, int dtype, int num_seqs, int max_q_len, void* workspace,
                         hipStream_t stream);
int launch_flash_prefill_paged(const PrefillParams& p, int dtype, hipStream_t stream);
int launch_flash_prefill_varlen(const PrefillParams& p, int num_seqs, int max_q_len, int max_kv_len,
                                long long total_q, int dtype, hipStream_t stream);
void launch_kv_write(const KVWriteParams& p, int vec_bytes, hipStream_t stream);
void launch_kv_gather(const KVGatherParams& p, int vec_bytes, hipStream_t stream);

}  // namespace tv
