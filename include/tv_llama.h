/*
 * tv_llama.h -- C ABI of the batched decode step of a LLaMA-architecture model
 * (TinyLlama-1.1B shape) on MI355X (gfx950), built around the attention entry
 * points of tv_attn.h.
 *
 * The reference (jonirajala/tinyvllm) runs the step as one TinyJit-compiled
 * tinygrad function (Llama.create_jit_decode, tinyvllm/model/llama.py:290-344)
 * called from Llama.decode (llama.py:346-388), and greedy sampling in
 * sample_tokens (tinyvllm/core/sampling.py:131-134).  Here the step is a fixed
 * sequence of HIP kernels launched by tv_llama_decode_step on one stream, with
 * every per-step input (tokens, positions, context lengths, block tables) in
 * device memory, so the whole step can be captured once into a HIP graph
 * (tv_llama_graph_*) and replayed without host work.
 *
 * Conventions are those of tv_attn.h (device pointers, caller-owned buffers,
 * stream = hipStream_t, return 0 or a TV_E* code with tv_last_error()).
 * dtype is TV_F16, TV_BF16 or TV_F32 (the reference's default model dtype,
 * weights.py:32) for everything in this header: the products run on MFMA
 * (v_mfma_f32_16x16x32 for 16-bit types, v_mfma_f32_16x16x4_f32 for fp32).
 * Norm weights and the RoPE table are float32.
 */
#ifndef TV_LLAMA_H
#define TV_LLAMA_H

#include <stddef.h>
#include <stdint.h>

#include "tv_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define TV_EPI_PARTIAL 0 /* out: float [splits, M, N] per-split partial sums */
#define TV_EPI_SWIGLU 1  /* out: T [M, N/2] silu(w1 x) * (w3 x), rows of W interleaved by four */
#define TV_EPI_LOGITS 2  /* out: float [M, N] (may be NULL) + per-work-group argmax keys */

/*
 * K elements per split that tv_llama_decode_step uses for an M x N x K product
 * (a multiple of 32; >= K means one split).  Host-only.
 */
int tv_linear_k_split(int M, int N, int K);

/*
 * Y = A W^T, A [M, K] (row stride lda elements), W [N, K] dense, both of dtype.
 * Replaces tinygrad Linear(bias=False) calls (llama.py:150-153, 214-216, 254).
 * Requires K % 32 == 0, N % 4 == 0, k_split % 32 == 0, 16-byte aligned A/W rows.
 *  TV_EPI_PARTIAL: out float [ceil(K/k_split), M, N].
 *  TV_EPI_SWIGLU:  W rows 4j, 4j+1 are w1 rows 2j, 2j+1 and rows 4j+2, 4j+3 the
 *                  w3 rows 2j, 2j+1; out T [M, N/2] at row stride ldo
 *                  (llama.py:220-221).  Needs k_split >= K.
 *  TV_EPI_LOGITS:  out float [M, N] at row stride ldo (may be NULL); keys
 *                  uint64 [ceil(N/64), M] (argmax keys consumed by
 *                  tv_argmax_advance).  Needs k_split >= K.
 */
int tv_linear(void* out, const void* a, const void* w, int M, int N, int K, int64_t lda, int64_t ldo,
              int k_split, int epilogue, uint64_t* keys, int dtype, void* stream);

/*
 * Residual stream update and RMSNorm (llama.py:14-23, 336-338):
 *   if emb:   x[m] = emb[tokens[m]]                 (tok_embeddings, llama.py:311)
 *   if part:  x[m] += sum_s part[s, m]              (h = h + out, llama.py:337-338)
 *   xh[m] = dtype(x[m] * rsqrt(mean(x[m]^2) + eps) * weight)
 * x float [M, dim]; part float [splits, M, dim] or NULL; weight float [dim].
 */
int tv_rms_norm_residual(float* x, void* xh, const float* part, int splits, const void* emb,
                         const int32_t* tokens, int vocab, const float* weight, int M, int dim, float eps,
                         int dtype, void* stream);

/*
 * RoPE table float [max_pos, head_dim/2, 2] of (cos, sin)(p * theta^(-2i/head_dim))
 * (precompute_freqs_cis, llama.py:26-31).
 */
int tv_rope_table(float* table, int max_pos, int head_dim, float theta, void* stream);

/*
 * q/k/v of M tokens from the fused projection's split partials
 * part float [splits, M, (Hq + 2 Hkv) * D]: rotate q and k (apply_rope,
 * llama.py:34-55) at position positions[m] (or pos_base + m when positions is
 * NULL), store q [M, Hq*D], optionally k/v [M, Hkv*D], and, when the caches are
 * given, write k/v into slot block_tables[m * bt_row_step + pos / block_size] *
 * block_size + pos % block_size of the [num_blocks, block_size, Hkv, D] caches
 * (llama.py:188-209, 381-386).  Rows whose slot falls outside the table or the
 * cache are not written; they are counted in err_count and get slot -1 in slots.
 */
int tv_qkv_rope_cache(void* q, void* k_out, void* v_out, void* k_cache, void* v_cache, const float* part,
                      int splits, const int32_t* positions, int pos_base, const float* rope, int rope_len,
                      const int32_t* block_tables, int64_t bt_row_step, int bt_width, int block_size,
                      int num_blocks, int M, int n_heads, int n_kv_heads, int head_dim, int dtype, int32_t* slots,
                      uint32_t* err_count, void* stream);

/*
 * Greedy sampling from TV_EPI_LOGITS keys (sampling.py:131-134): tokens[m] =
 * argmax (first maximum).  When positions is given, history[m, positions[m]+1]
 * = token (if inside history_len) and positions[m] += 1; when context_lens is
 * given, context_lens[m] += 1.
 */
int tv_argmax_advance(int32_t* tokens, int32_t* positions, int32_t* context_lens, int32_t* history,
                      int history_len, const uint64_t* keys, int nparts, int M, void* stream);

/* ---- model-level step ------------------------------------------------------ */

/* Weights in device memory; per-layer fields are host arrays of n_layers device pointers. */
typedef struct tv_llama_model {
  int n_layers, dim, n_heads, n_kv_heads, head_dim, hidden_dim, vocab_size;
  int dtype;
  float norm_eps;
  const void* tok_embeddings;          /* [vocab, dim] */
  const void* const* wqkv;             /* [(Hq + 2 Hkv) * D, dim]: wq, wk, wv rows */
  const void* const* wo;               /* [dim, Hq * D] */
  const void* const* w13;              /* [2 * hidden, dim], interleaved as for TV_EPI_SWIGLU */
  const void* const* w2;               /* [dim, hidden] */
  const float* const* attention_norm;  /* [dim] */
  const float* const* ffn_norm;        /* [dim] */
  const float* norm;                   /* [dim] */
  const void* output;                  /* [vocab, dim] */
  const float* rope;                   /* tv_rope_table output */
  int rope_len;
} tv_llama_model;

/* Paged K/V caches: host arrays of n_layers device pointers [num_blocks, block_size, Hkv, D]. */
typedef struct tv_llama_cache {
  void* const* k_caches;
  void* const* v_caches;
  int num_blocks, block_size;
} tv_llama_cache;

typedef struct tv_llama_decode_args {
  int batch;
  int32_t* tokens;              /* [B] token of this step; replaced by the sampled token */
  int32_t* positions;           /* [B] its position (RoPE, cache slot); advanced by one */
  int32_t* context_lens;        /* [B] tokens attended to; advanced by one */
  const int32_t* block_tables;  /* [B, bt_stride] */
  int bt_stride, max_blocks;    /* table row stride; columns attended (<= bt_stride) */
  int partition_size;           /* split-context partition (multiple of 16) */
  int write_before_attend;      /* 1: cache write, then attention; 0: the reference order */
  float* logits;                /* [B, vocab] or NULL */
  int32_t* history;             /* [B, history_len] or NULL: history[b, pos + 1] = sampled token */
  int history_len;
  void* workspace;
  size_t workspace_bytes;
} tv_llama_decode_args;

/* Workspace of tv_llama_decode_step.  Host-only. */
size_t tv_llama_decode_workspace_bytes(const tv_llama_model* model, int batch, int max_blocks, int block_size,
                                       int partition_size);

/*
 * One batched decode step (Llama.decode + the JIT body, llama.py:290-388, and
 * greedy sampling): embedding, n_layers x (RMSNorm, fused QKV product, RoPE,
 * K/V cache write, paged attention, output product, residual, RMSNorm, SwiGLU
 * MLP, residual), final RMSNorm, LM head and argmax.
 * write_before_attend = 1 writes the step's K/V before attention, so a context
 * length of position + 1 includes the token itself; 0 keeps the reference's
 * order (attention first, llama.py:378-386).
 */
int tv_llama_decode_step(const tv_llama_model* model, const tv_llama_cache* cache, const tv_llama_decode_args* args,
                         void* stream);

/* Capture tv_llama_decode_step on `stream` (not the NULL stream) into an executable HIP graph. */
int tv_llama_graph_create(const tv_llama_model* model, const tv_llama_cache* cache,
                          const tv_llama_decode_args* args, void* stream, void** graph);
int tv_llama_graph_launch(void* graph, void* stream);
int tv_llama_graph_destroy(void* graph);

typedef struct tv_llama_prefill_args {
  int num_tokens;
  const int32_t* tokens;        /* [num_tokens] */
  int start_pos;
  const int32_t* block_table;   /* this sequence's table row: bt_width entries covering */
  int bt_width;                 /* positions 0 .. start_pos + num_tokens - 1 (TV_EINVAL otherwise) */
  float* logits;                /* [num_tokens, vocab], or [1, vocab] with logits_last_only, or NULL */
  int logits_last_only;
  int32_t* next_token;          /* [1] greedy token after the last position, or NULL */
  void* workspace;
  size_t workspace_bytes;
  /* 0: the reference's prefill, attending within this chunk only (llama.py:184;
   * a chunk at start_pos > 0 ignores the cached prefix).  1: each token attends
   * to every cached position up to its own (chunked prefill; no reference
   * counterpart), through the paged cache after the chunk's K/V are written. */
  int attend_prefix;
} tv_llama_prefill_args;

/* Workspace of tv_llama_prefill.  Host-only. */
size_t tv_llama_prefill_workspace_bytes(const tv_llama_model* model, int num_tokens);

/*
 * Prompt pass of one sequence (Llama.prefill, llama.py:264-285): the same
 * layers over num_tokens positions start_pos.., K/V written into the cache,
 * attention causal over this chunk only (llama.py:184).
 */
int tv_llama_prefill(const tv_llama_model* model, const tv_llama_cache* cache, const tv_llama_prefill_args* args,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TV_LLAMA_H */
