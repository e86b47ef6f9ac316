// Launch parameter blocks of the dense decode-step kernels (dense.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tv {

enum LinearEpilogue : int { kEpiPartial = 0, kEpiSwiglu = 1, kEpiLogits = 2 };

constexpr int kLinBM = 64;    // rows of A (tokens) per work-group
constexpr int kLinBN = 64;    // rows of W (output features) per work-group, 16 per wave
constexpr int kLinKC = 256;   // K elements per LDS chunk at 16-bit types (512 bytes; 128 at fp32)

// Y = A W^T over the K range of one split; grid (splits, ceil(N/64), ceil(M/64)).
struct LinearParams {
  const void* a;          // [M, K] at row stride lda
  const void* w;          // [N, K] dense
  int M, N, K;
  long long lda;
  int k_split;            // K elements per split (multiple of 32)
  float* part;            // partial: [splits, M, N]
  void* out;              // swiglu: T [M, N/2]; logits: float [M, N] (may be null)
  long long ldo;
  unsigned long long* keys;   // logits: [ceil(N/64), M] argmax keys (may be null)
};

// x = emb[tokens] or x += sum of partials; xh = T(rmsnorm(x) * weight).
struct NormParams {
  float* x;               // [M, dim] residual stream
  void* xh;               // [M, dim] normalised copy in T
  const float* part;      // [splits, M, dim] or null
  int splits;
  const void* emb;        // [vocab, dim] T or null
  const int* tokens;      // [M] when emb is set
  int vocab;
  const float* weight;    // [dim]
  int M, dim;
  float eps;
};

// Sum the QKV split partials, rotate q and k, store q and write k/v.
struct QKVParams {
  void* q;                // [M, Hq*D] T
  void* k_out;            // [M, Hkv*D] T or null
  void* v_out;            // [M, Hkv*D] T or null
  void* k_cache;          // [NB, bs, Hkv, D] T or null
  void* v_cache;
  const float* part;      // [splits, M, (Hq+2Hkv)*D]
  int splits;
  const int* positions;   // [M] or null (then pos_base + m)
  int pos_base;
  const float* rope;      // [rope_len, D/2, 2] (cos, sin)
  int rope_len;
  const int* block_tables;   // row of token m: block_tables + m * bt_row_step
  long long bt_row_step;
  int bt_width;
  int block_size, num_blocks;
  int M, Hq, Hkv, D;
  int* slots;             // [M] slot written per row (-1: none) or null
  unsigned* err_count;    // rows whose slot was outside the cache, or null
};

// Greedy token from the per-work-group argmax keys; advance positions.
struct AdvanceParams {
  const unsigned long long* keys;   // [nparts, M]
  int nparts, M;
  int* tokens;            // [M] out
  int* positions;         // [M] or null: += 1
  int* context_lens;      // [M] or null: += 1
  int* history;           // [M, history_len] or null: history[m, pos + 1] = token
  int history_len;
};

// Decode-step attention fused with the q|k|v split sum, RoPE and the K/V write
// (step_attn.hip); grid (Hkv, B).
struct StepAttnParams {
  void* out;              // [B, Hq, D] T
  const float* part;      // [splits, B, (Hq+2Hkv)*D] q|k|v projection partials
  int splits;
  const int* positions;   // [B]
  const int* context_lens;   // [B]
  const float* rope;      // [rope_len, D/2, 2]
  int rope_len;
  void* k_cache;          // [NB, bs, Hkv, D] T
  void* v_cache;
  const int* block_tables;   // [B, bt_stride]
  int bt_stride, max_blocks;
  int block_size, num_blocks;
  int B, Hq, Hkv;
  float scale;
  int write_before;       // 1: k/v written before attention; 0: after (the reference's order)
};

bool step_attn_supported(int head_dim, int group, int block_size);
void launch_step_attn(const StepAttnParams& p, int head_dim, int dtype, hipStream_t s);

void launch_linear(const LinearParams& p, int epilogue, int dtype, hipStream_t s);
void launch_norm(const NormParams& p, int dtype, hipStream_t s);
void launch_qkv_rope(const QKVParams& p, int dtype, hipStream_t s);
void launch_rope_table(float* table, int max_pos, int head_dim, float theta, hipStream_t s);
void launch_advance(const AdvanceParams& p, hipStream_t s);
// out[i] = base + i, i < n
void launch_iota(int* out, int n, int base, hipStream_t s);

}  // namespace tv
