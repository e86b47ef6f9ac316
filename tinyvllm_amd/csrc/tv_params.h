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

int launch_flash_prefill(const PrefillParams& p, int dtype, bool allow_mfma, hipStream_t stream);
void launch_kv_write(const KVWriteParams& p, int vec_bytes, hipStream_t stream);
void launch_kv_gather(const KVGatherParams& p, int vec_bytes, hipStream_t stream);

}  // namespace tv
