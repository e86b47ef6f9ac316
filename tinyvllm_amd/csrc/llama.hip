// C ABI of the dense decode-step kernels and the decode / prefill drivers
// (declared in include/tv_llama.h).
//
// tv_llama_decode_step launches, per layer, 8 kernels (+1 split-context merge
// when the attention is partitioned) on one stream:
//   linear(partial)  xh -> fused q|k|v projection, K split across work-groups
//   qkv_rope         split sum, RoPE, q store, K/V cache write
//   paged_decode     attention over the paged cache (tv_paged_decode)
//   linear(partial)  attention output projection
//   norm             x += projection; xh = RMSNorm(x) * ffn_norm
//   linear(swiglu)   silu(w1 xh) * (w3 xh), one pass over the interleaved w1|w3
//   linear(partial)  down projection
//   norm             x += projection; xh = RMSNorm(x) * next norm weight
// then linear(logits) with the argmax keys and the sampling/advance kernel.
// Every pointer the kernels read comes from the argument structs, so the
// sequence can be captured into a HIP graph once and replayed.
#include <algorithm>
#include <cmath>

#include "../../include/tv_llama.h"
#include "tv_dense.h"
#include "tv_error.h"

namespace {

using tv::check_launch;
using tv::fail;
using tv::ok;

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
long long round_up(long long x, long long a) { return (x + a - 1) / a * a; }

bool step_dtype(int d) { return d == TV_F16 || d == TV_BF16 || d == TV_F32; }
size_t elem_bytes(int d) { return d == TV_F32 ? 4 : 2; }
bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int splits_of(int K, int k_split) { return (K + k_split - 1) / k_split; }

// Carves 256-byte aligned regions out of one workspace.
struct Carver {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t at = off;
    off = align_up(off + bytes, 256);
    return at;
  }
};

struct StepLayout {
  int ks_qkv, ks_o, ks_2;
  size_t part, q, attn, x, xh, h, keys, kst, vst, slots, attn_ws, attn_ws_bytes, total;
};

int validate_model(const tv_llama_model* m, const char* who) {
  if (!m) return fail(TV_EINVAL, "%s: null model", who);
  if (!step_dtype(m->dtype)) return fail(TV_EUNSUPPORTED, "%s: dtype %d (float32 / float16 / bfloat16)", who, m->dtype);
  if (m->n_layers <= 0 || m->dim <= 0 || m->n_heads <= 0 || m->n_kv_heads <= 0 || m->head_dim <= 0 ||
      m->hidden_dim <= 0 || m->vocab_size <= 0 || m->n_heads % m->n_kv_heads != 0)
    return fail(TV_EINVAL, "%s: bad model shape", who);
  if (m->dim % 32 || (m->n_heads * m->head_dim) % 32 || m->hidden_dim % 32)
    return fail(TV_EUNSUPPORTED, "%s: dim, n_heads*head_dim and hidden_dim must be multiples of 32", who);
  if (m->dim > 8192) return fail(TV_EUNSUPPORTED, "%s: dim %d above 8192", who, m->dim);
  if (m->head_dim % 2 || m->vocab_size % 4)
    return fail(TV_EUNSUPPORTED, "%s: head_dim must be even and vocab_size a multiple of 4", who);
  if (!m->tok_embeddings || !m->wqkv || !m->wo || !m->w13 || !m->w2 || !m->attention_norm || !m->ffn_norm ||
      !m->norm || !m->output || !m->rope || m->rope_len <= 0)
    return fail(TV_EINVAL, "%s: null weight pointer", who);
  for (int l = 0; l < m->n_layers; ++l)
    if (!m->wqkv[l] || !m->wo[l] || !m->w13[l] || !m->w2[l] || !m->attention_norm[l] || !m->ffn_norm[l])
      return fail(TV_EINVAL, "%s: null weight pointer in layer %d", who, l);
  return TV_OK;
}

int qkv_width(const tv_llama_model* m) { return (m->n_heads + 2 * m->n_kv_heads) * m->head_dim; }

StepLayout step_layout(const tv_llama_model* m, int B, int max_blocks, int block_size, int partition_size,
                       bool decode) {
  StepLayout L{};
  const int qd = m->n_heads * m->head_dim;
  const int kd = m->n_kv_heads * m->head_dim;
  const int nqkv = qkv_width(m);
  L.ks_qkv = tv_linear_k_split(B, nqkv, m->dim);
  L.ks_o = tv_linear_k_split(B, m->dim, qd);
  L.ks_2 = tv_linear_k_split(B, m->dim, m->hidden_dim);
  const size_t part_floats = std::max({(size_t)splits_of(m->dim, L.ks_qkv) * nqkv, (size_t)splits_of(qd, L.ks_o) * m->dim,
                                       (size_t)splits_of(m->hidden_dim, L.ks_2) * m->dim}) * (size_t)B;
  const size_t es = elem_bytes(m->dtype);
  Carver c;
  L.part = c.take(part_floats * 4);
  L.q = c.take((size_t)B * qd * es);
  L.attn = c.take((size_t)B * qd * es);
  L.x = c.take((size_t)B * m->dim * 4);
  L.xh = c.take((size_t)B * m->dim * es);
  L.h = c.take((size_t)B * m->hidden_dim * es);
  L.keys = c.take((size_t)((m->vocab_size + tv::kLinBN - 1) / tv::kLinBN) * B * 8);
  L.kst = c.take((size_t)B * kd * es);
  L.vst = c.take((size_t)B * kd * es);
  L.slots = c.take((size_t)B * 4);
  // prefill: room for a prefix-attending chunk's unsplit paged-decode launch
  // (its only workspace is the schedule of B + 1 ints)
  L.attn_ws_bytes = decode ? tv_paged_decode_workspace_bytes(B, m->n_heads, m->head_dim, max_blocks, block_size,
                                                             partition_size)
                           : align_up((size_t)(B + 1) * 4, 256);
  L.attn_ws = c.take(L.attn_ws_bytes);
  L.total = c.off;
  return L;
}

template <typename P> P* at(void* base, size_t off) {
  return reinterpret_cast<P*>(reinterpret_cast<char*>(base) + off);
}

void linear(const void* a, const void* w, int M, int N, int K, long long lda, int k_split, int epi, void* out,
            long long ldo, unsigned long long* keys, int dtype, hipStream_t s) {
  tv::LinearParams p{};
  p.a = a;
  p.w = w;
  p.M = M;
  p.N = N;
  p.K = K;
  p.lda = lda;
  p.k_split = k_split;
  p.part = epi == tv::kEpiPartial ? reinterpret_cast<float*>(out) : nullptr;
  p.out = epi == tv::kEpiPartial ? nullptr : out;
  p.ldo = ldo;
  p.keys = keys;
  tv::launch_linear(p, epi, dtype, s);
}

void norm(float* x, void* xh, const float* part, int splits, const void* emb, const int* tokens, int vocab,
          const float* weight, int M, int dim, float eps, int dtype, hipStream_t s) {
  tv::NormParams p{};
  p.x = x;
  p.xh = xh;
  p.part = part;
  p.splits = splits;
  p.emb = emb;
  p.tokens = tokens;
  p.vocab = vocab;
  p.weight = weight;
  p.M = M;
  p.dim = dim;
  p.eps = eps;
  tv::launch_norm(p, dtype, s);
}

// The layers after the embedding: the part of the step shared by decode and prefill.
struct LayerIO {
  int M;
  float* x;
  void* xh;
  float* part;
  void* q;
  void* attn;
  void* h;
  // attention: decode uses the paged cache, prefill the staged chunk
  bool decode;
  const tv_llama_decode_args* dargs;
  const tv_llama_prefill_args* pargs;
  void* kst;
  void* vst;
  int* slots;
  void* attn_ws;
  size_t attn_ws_bytes;
  int ks_qkv, ks_o, ks_2;
};

// Split sum + RoPE + K/V write + attention of one decode layer in one kernel.
int attend_fused(const tv_llama_model* m, const tv_llama_cache* c, const LayerIO& io, int l, hipStream_t s) {
  const int dt = m->dtype;
  const float scale = 1.0f / std::sqrt((float)m->head_dim);
  const int M = io.M;
  const tv_llama_decode_args* a = io.dargs;
  tv::StepAttnParams sp{};
  sp.out = io.attn;
  sp.part = io.part;
  sp.splits = splits_of(m->dim, io.ks_qkv);
  sp.positions = a->positions;
  sp.context_lens = a->context_lens;
  sp.rope = m->rope;
  sp.rope_len = m->rope_len;
  sp.k_cache = c->k_caches[l];
  sp.v_cache = c->v_caches[l];
  sp.block_tables = a->block_tables;
  sp.bt_stride = a->bt_stride;
  sp.max_blocks = a->max_blocks;
  sp.block_size = c->block_size;
  sp.num_blocks = c->num_blocks;
  sp.B = M;
  sp.Hq = m->n_heads;
  sp.Hkv = m->n_kv_heads;
  sp.scale = scale;
  sp.write_before = a->write_before_attend ? 1 : 0;
  tv::launch_step_attn(sp, m->head_dim, dt, s);
  return check_launch("step_attn");
}

// The same without the fused kernel: qkv_rope, then tv_paged_decode (decode)
// or tv_flash_prefill (prefill).  In the reference's order the decode stages
// k/v with their slots and writes them after attention.
int attend_unfused(const tv_llama_model* m, const tv_llama_cache* c, const LayerIO& io, int l, hipStream_t s) {
  const int dt = m->dtype;
  const int qd = m->n_heads * m->head_dim;
  const int kd = m->n_kv_heads * m->head_dim;
  const float scale = 1.0f / std::sqrt((float)m->head_dim);
  const int M = io.M;
  tv::QKVParams qp{};
  qp.q = io.q;
  qp.part = io.part;
  qp.splits = splits_of(m->dim, io.ks_qkv);
  qp.rope = m->rope;
  qp.rope_len = m->rope_len;
  qp.block_size = c->block_size;
  qp.num_blocks = c->num_blocks;
  qp.M = M;
  qp.Hq = m->n_heads;
  qp.Hkv = m->n_kv_heads;
  qp.D = m->head_dim;
  if (io.decode) {
    const tv_llama_decode_args* a = io.dargs;
    qp.positions = a->positions;
    qp.block_tables = a->block_tables;
    qp.bt_row_step = a->bt_stride;
    qp.bt_width = a->bt_stride;
    if (a->write_before_attend) {
      qp.k_cache = c->k_caches[l];
      qp.v_cache = c->v_caches[l];
    } else {
      // reference order: stage k/v and their slots now, write them after attention
      qp.k_out = io.kst;
      qp.v_out = io.vst;
      qp.slots = io.slots;
    }
  } else {
    const tv_llama_prefill_args* a = io.pargs;
    qp.pos_base = a->start_pos;
    qp.block_tables = a->block_table;
    qp.bt_row_step = 0;
    qp.bt_width = a->bt_width;
    qp.k_out = io.kst;
    qp.v_out = io.vst;
    qp.k_cache = c->k_caches[l];
    qp.v_cache = c->v_caches[l];
  }
  tv::launch_qkv_rope(qp, dt, s);
  int rc = check_launch("qkv_rope");
  if (rc != TV_OK) return rc;

  if (io.decode) {
    const tv_llama_decode_args* a = io.dargs;
    rc = tv_paged_decode(io.attn, io.q, c->k_caches[l], c->v_caches[l], a->block_tables, a->context_lens,
                         a->batch, m->n_heads, m->n_kv_heads, m->head_dim, c->block_size, c->num_blocks,
                         a->bt_stride, a->max_blocks, scale, dt, dt, a->partition_size, io.attn_ws,
                         io.attn_ws_bytes, s);
    if (rc != TV_OK) return rc;
    if (!a->write_before_attend) {
      // Llama.decode writes k/v at get_slot() after the JIT call (llama.py:381-386)
      rc = tv_reshape_and_cache(c->k_caches[l], c->v_caches[l], io.kst, io.vst, io.slots, M, m->n_kv_heads,
                                m->head_dim, c->block_size, c->num_blocks, kd, kd, dt, nullptr, s);
      if (rc != TV_OK) return rc;
    }
  } else if (io.pargs->attend_prefix && io.pargs->start_pos > 0) {
    // chunked prefill over the cached prefix: the chunk's k/v are in the cache
    // now, so the chunk attends keys 0 .. start_pos + M - 1 through the
    // sequence's table (MFMA tiles, causal at offset start_pos)
    const tv_llama_prefill_args* a = io.pargs;
    rc = tv_flash_prefill_paged(io.attn, io.q, c->k_caches[l], c->v_caches[l], a->block_table, c->num_blocks,
                                c->block_size, M, a->start_pos, m->n_heads, m->n_kv_heads, m->head_dim, qd, qd, 1,
                                scale, dt, dt, s);
    if (rc == TV_EUNSUPPORTED) {
      // fp32 models, odd head sizes or block sizes: row i is a paged decode of
      // context start_pos + i + 1 over the sequence's one table row (stride 0)
      const int width = a->bt_width * c->block_size;
      rc = tv_paged_decode(io.attn, io.q, c->k_caches[l], c->v_caches[l], a->block_table, io.slots, M, m->n_heads,
                           m->n_kv_heads, m->head_dim, c->block_size, c->num_blocks, 0, a->bt_width, scale, dt, dt,
                           (width + 15) / 16 * 16, io.attn_ws, io.attn_ws_bytes, s);
    }
    if (rc != TV_OK) return rc;
  } else {
    rc = tv_flash_prefill(io.attn, io.q, io.kst, io.vst, M, M, m->n_heads, m->n_kv_heads, m->head_dim,
                          m->head_dim, qd, kd, kd, qd, 1, scale, dt, dt, 0, nullptr, 0, s);
    if (rc != TV_OK) return rc;
  }
  return TV_OK;
}

int run_layers(const tv_llama_model* m, const tv_llama_cache* c, const LayerIO& io, hipStream_t s) {
  const int dt = m->dtype;
  const int qd = m->n_heads * m->head_dim;
  const int nqkv = qkv_width(m);
  const int M = io.M;
  // the fused step attention runs on 16-bit MFMA; fp32 models take qkv_rope + tv_paged_decode
  const bool fused_attn = io.decode && dt != TV_F32 &&
                          tv::step_attn_supported(m->head_dim, m->n_heads / m->n_kv_heads, c->block_size);
  for (int l = 0; l < m->n_layers; ++l) {
    linear(io.xh, m->wqkv[l], M, nqkv, m->dim, m->dim, io.ks_qkv, tv::kEpiPartial, io.part, 0, nullptr, dt, s);
    int rc = fused_attn ? attend_fused(m, c, io, l, s) : attend_unfused(m, c, io, l, s);
    if (rc != TV_OK) return rc;

    linear(io.attn, m->wo[l], M, m->dim, qd, qd, io.ks_o, tv::kEpiPartial, io.part, 0, nullptr, dt, s);
    norm(io.x, io.xh, io.part, splits_of(qd, io.ks_o), nullptr, nullptr, 0, m->ffn_norm[l], M, m->dim, m->norm_eps,
         dt, s);
    linear(io.xh, m->w13[l], M, 2 * m->hidden_dim, m->dim, m->dim, m->dim, tv::kEpiSwiglu, io.h, m->hidden_dim,
           nullptr, dt, s);
    linear(io.h, m->w2[l], M, m->dim, m->hidden_dim, m->hidden_dim, io.ks_2, tv::kEpiPartial, io.part, 0, nullptr,
           dt, s);
    const float* next_w = l + 1 < m->n_layers ? m->attention_norm[l + 1] : m->norm;
    norm(io.x, io.xh, io.part, splits_of(m->hidden_dim, io.ks_2), nullptr, nullptr, 0, next_w, M, m->dim,
         m->norm_eps, dt, s);
    rc = check_launch("layer");
    if (rc != TV_OK) return rc;
  }
  return TV_OK;
}

// Work-groups a skinny product aims for when it splits K.
constexpr long long kLinearTargetWorkGroups = 192;

}  // namespace

extern "C" {

int tv_linear_k_split(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 32;
  const long long full = round_up(K, 32);
  const long long tiles = ((N + tv::kLinBN - 1) / tv::kLinBN) * (long long)((M + tv::kLinBM - 1) / tv::kLinBM);
  // About three work-groups per four CUs: more splits add partials that the
  // consumer (norm or step attention) reads back, and on the TinyLlama step
  // 192 beat 128, 160, 224 and 256 (1.53 vs 1.55-1.59 ms).
  const long long target = kLinearTargetWorkGroups;
  if (tiles >= target / 2) return (int)full;
  const long long want = (target + tiles - 1) / tiles;
  const long long per = (K + want - 1) / want;
  // whole LDS chunks: a partial chunk still streams the chunk's full width of W
  const long long ks = per >= tv::kLinKC ? (per + tv::kLinKC / 2) / tv::kLinKC * tv::kLinKC : round_up(per, 32);
  return (int)std::min(full, std::max(ks, 32LL));
}

int tv_linear(void* out, const void* a, const void* w, int M, int N, int K, int64_t lda, int64_t ldo, int k_split,
              int epilogue, uint64_t* keys, int dtype, void* stream) {
  if (!a || !w || (!out && epilogue != TV_EPI_LOGITS)) return fail(TV_EINVAL, "tv_linear: null pointer argument");
  if (!step_dtype(dtype)) return fail(TV_EUNSUPPORTED, "tv_linear: dtype %d (float32 / float16 / bfloat16)", dtype);
  if (M <= 0 || N <= 0 || K <= 0) return fail(TV_EINVAL, "tv_linear: bad shape %d x %d x %d", M, N, K);
  if (K % 32 || N % 4) return fail(TV_EUNSUPPORTED, "tv_linear: K %% 32 and N %% 4 must be 0 (K=%d, N=%d)", K, N);
  if (lda < K) return fail(TV_EINVAL, "tv_linear: lda %lld < K %d", (long long)lda, K);
  if (!aligned16(a) || !aligned16(w) || lda % 8) return fail(TV_EINVAL, "tv_linear: A/W rows must be 16-byte aligned");
  if (k_split <= 0 || k_split % 32) return fail(TV_EINVAL, "tv_linear: k_split %d must be a positive multiple of 32", k_split);
  if (epilogue < TV_EPI_PARTIAL || epilogue > TV_EPI_LOGITS) return fail(TV_EINVAL, "tv_linear: bad epilogue %d", epilogue);
  if (epilogue != TV_EPI_PARTIAL && k_split < K)
    return fail(TV_EINVAL, "tv_linear: the swiglu / logits epilogues need one split (k_split >= K)");
  if (epilogue == TV_EPI_SWIGLU && (ldo < N / 2 || (uintptr_t)out % 4))
    return fail(TV_EINVAL, "tv_linear: swiglu output row stride %lld < N/2", (long long)ldo);
  if (epilogue == TV_EPI_LOGITS && out && (ldo < N || ldo % 4 || !aligned16(out)))
    return fail(TV_EINVAL, "tv_linear: logits output needs ldo >= N, ldo %% 4 == 0, 16-byte alignment");
  if (epilogue == TV_EPI_PARTIAL && !aligned16(out)) return fail(TV_EINVAL, "tv_linear: partials must be 16-byte aligned");
  const long long splits = splits_of(K, k_split);
  if ((N + tv::kLinBN - 1) / tv::kLinBN > 65535 || (M + tv::kLinBM - 1) / tv::kLinBM > 65535)
    return fail(TV_EINVAL, "tv_linear: grid too large");
  linear(a, w, M, N, K, lda, k_split, epilogue, out, ldo, reinterpret_cast<unsigned long long*>(keys), dtype,
         reinterpret_cast<hipStream_t>(stream));
  return check_launch("tv_linear");
}

int tv_rms_norm_residual(float* x, void* xh, const float* part, int splits, const void* emb, const int32_t* tokens,
                         int vocab, const float* weight, int M, int dim, float eps, int dtype, void* stream) {
  if (!x || !xh || !weight || (emb && !tokens)) return fail(TV_EINVAL, "tv_rms_norm_residual: null pointer argument");
  if (!step_dtype(dtype)) return fail(TV_EUNSUPPORTED, "tv_rms_norm_residual: dtype %d (float32 / float16 / bfloat16)", dtype);
  if (M <= 0 || dim <= 0 || dim % 4 || (part && splits <= 0) || (emb && vocab <= 0))
    return fail(TV_EINVAL, "tv_rms_norm_residual: bad shape (M=%d, dim=%d, splits=%d)", M, dim, splits);
  if (dim > 8192) return fail(TV_EUNSUPPORTED, "tv_rms_norm_residual: dim %d above 8192", dim);
  if (!aligned16(x) || !aligned16(weight) || (part && !aligned16(part)) || (uintptr_t)xh % 8 ||
      (emb && (uintptr_t)emb % 8))
    return fail(TV_EINVAL, "tv_rms_norm_residual: misaligned buffer");
  norm(x, xh, part, part ? splits : 0, emb, tokens, vocab, weight, M, dim, eps, dtype,
       reinterpret_cast<hipStream_t>(stream));
  return check_launch("tv_rms_norm_residual");
}

int tv_rope_table(float* table, int max_pos, int head_dim, float theta, void* stream) {
  if (!table || max_pos <= 0 || head_dim <= 0 || head_dim % 2 || !(theta > 0.0f))
    return fail(TV_EINVAL, "tv_rope_table: bad arguments");
  tv::launch_rope_table(table, max_pos, head_dim, theta, reinterpret_cast<hipStream_t>(stream));
  return check_launch("tv_rope_table");
}

int tv_qkv_rope_cache(void* q, void* k_out, void* v_out, void* k_cache, void* v_cache, const float* part, int splits,
                      const int32_t* positions, int pos_base, const float* rope, int rope_len,
                      const int32_t* block_tables, int64_t bt_row_step, int bt_width, int block_size, int num_blocks,
                      int M, int n_heads, int n_kv_heads, int head_dim, int dtype, int32_t* slots,
                      uint32_t* err_count, void* stream) {
  if (!q || !part || !rope) return fail(TV_EINVAL, "tv_qkv_rope_cache: null pointer argument");
  if (!step_dtype(dtype)) return fail(TV_EUNSUPPORTED, "tv_qkv_rope_cache: dtype %d (float32 / float16 / bfloat16)", dtype);
  if (M <= 0 || splits <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 || rope_len <= 0)
    return fail(TV_EINVAL, "tv_qkv_rope_cache: bad shape");
  if (!k_cache != !v_cache) return fail(TV_EINVAL, "tv_qkv_rope_cache: give both caches or neither");
  if (k_cache && (!block_tables || block_size <= 0 || num_blocks <= 0 || bt_width <= 0 || bt_row_step < 0))
    return fail(TV_EINVAL, "tv_qkv_rope_cache: bad cache geometry");
  if ((uintptr_t)q % 4 || (uintptr_t)part % 8 || (uintptr_t)rope % 8 || (k_out && (uintptr_t)k_out % 4) ||
      (v_out && (uintptr_t)v_out % 4) || (k_cache && ((uintptr_t)k_cache % 4 || (uintptr_t)v_cache % 4)))
    return fail(TV_EINVAL, "tv_qkv_rope_cache: misaligned buffer");
  if ((long long)M * ((n_heads + 2 * n_kv_heads) * head_dim / 2) > (long long)0x7fffffff * 256)
    return fail(TV_EINVAL, "tv_qkv_rope_cache: grid too large");
  tv::QKVParams p{};
  p.q = q;
  p.k_out = k_out;
  p.v_out = v_out;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.part = part;
  p.splits = splits;
  p.positions = positions;
  p.pos_base = pos_base;
  p.rope = rope;
  p.rope_len = rope_len;
  p.block_tables = block_tables;
  p.bt_row_step = bt_row_step;
  p.bt_width = bt_width;
  p.block_size = block_size;
  p.num_blocks = num_blocks;
  p.M = M;
  p.Hq = n_heads;
  p.Hkv = n_kv_heads;
  p.D = head_dim;
  p.slots = slots;
  p.err_count = err_count;
  tv::launch_qkv_rope(p, dtype, reinterpret_cast<hipStream_t>(stream));
  return check_launch("tv_qkv_rope_cache");
}

int tv_argmax_advance(int32_t* tokens, int32_t* positions, int32_t* context_lens, int32_t* history, int history_len,
                      const uint64_t* keys, int nparts, int M, void* stream) {
  if (!tokens || !keys) return fail(TV_EINVAL, "tv_argmax_advance: null pointer argument");
  if (M <= 0 || nparts <= 0 || (history && history_len <= 0)) return fail(TV_EINVAL, "tv_argmax_advance: bad shape");
  tv::AdvanceParams p{};
  p.keys = reinterpret_cast<const unsigned long long*>(keys);
  p.nparts = nparts;
  p.M = M;
  p.tokens = tokens;
  p.positions = positions;
  p.context_lens = context_lens;
  p.history = history;
  p.history_len = history_len;
  tv::launch_advance(p, reinterpret_cast<hipStream_t>(stream));
  return check_launch("tv_argmax_advance");
}

size_t tv_llama_decode_workspace_bytes(const tv_llama_model* model, int batch, int max_blocks, int block_size,
                                       int partition_size) {
  if (!model || batch <= 0 || max_blocks <= 0 || block_size <= 0 || partition_size <= 0) return 0;
  if (model->n_heads <= 0 || model->head_dim <= 0 || model->dim <= 0 || model->hidden_dim <= 0) return 0;
  return step_layout(model, batch, max_blocks, block_size, partition_size, true).total;
}

int tv_llama_decode_step(const tv_llama_model* m, const tv_llama_cache* c, const tv_llama_decode_args* a,
                         void* stream) {
  int rc = validate_model(m, "tv_llama_decode_step");
  if (rc != TV_OK) return rc;
  if (!c || !c->k_caches || !c->v_caches || c->num_blocks <= 0 || c->block_size <= 0)
    return fail(TV_EINVAL, "tv_llama_decode_step: bad cache");
  if (!a || a->batch <= 0 || !a->tokens || !a->positions || !a->context_lens || !a->block_tables ||
      a->bt_stride <= 0 || a->max_blocks <= 0 || a->max_blocks > a->bt_stride || a->partition_size <= 0)
    return fail(TV_EINVAL, "tv_llama_decode_step: bad decode arguments");
  if (a->history && a->history_len <= 0) return fail(TV_EINVAL, "tv_llama_decode_step: bad history_len");
  if (a->logits && !aligned16(a->logits)) return fail(TV_EINVAL, "tv_llama_decode_step: logits must be 16-byte aligned");
  const StepLayout L = step_layout(m, a->batch, a->max_blocks, c->block_size, a->partition_size, true);
  if (!a->workspace || a->workspace_bytes < L.total || !aligned16(a->workspace))
    return fail(TV_EINVAL, "tv_llama_decode_step: workspace of %zu bytes required (got %zu)", L.total,
                a->workspace_bytes);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void* ws = a->workspace;
  const int B = a->batch;
  norm(at<float>(ws, L.x), at<void>(ws, L.xh), nullptr, 0, m->tok_embeddings, a->tokens, m->vocab_size,
       m->attention_norm[0], B, m->dim, m->norm_eps, m->dtype, s);
  LayerIO io{};
  io.M = B;
  io.x = at<float>(ws, L.x);
  io.xh = at<void>(ws, L.xh);
  io.part = at<float>(ws, L.part);
  io.q = at<void>(ws, L.q);
  io.attn = at<void>(ws, L.attn);
  io.h = at<void>(ws, L.h);
  io.decode = true;
  io.dargs = a;
  io.kst = at<void>(ws, L.kst);
  io.vst = at<void>(ws, L.vst);
  io.slots = at<int>(ws, L.slots);
  io.attn_ws = L.attn_ws_bytes ? at<void>(ws, L.attn_ws) : nullptr;
  io.attn_ws_bytes = L.attn_ws_bytes;
  io.ks_qkv = L.ks_qkv;
  io.ks_o = L.ks_o;
  io.ks_2 = L.ks_2;
  rc = run_layers(m, c, io, s);
  if (rc != TV_OK) return rc;
  unsigned long long* keys = at<unsigned long long>(ws, L.keys);
  linear(io.xh, m->output, B, m->vocab_size, m->dim, m->dim, m->dim, tv::kEpiLogits, a->logits, m->vocab_size, keys,
         m->dtype, s);
  tv::AdvanceParams ap{};
  ap.keys = keys;
  ap.nparts = (m->vocab_size + tv::kLinBN - 1) / tv::kLinBN;
  ap.M = B;
  ap.tokens = a->tokens;
  ap.positions = a->positions;
  ap.context_lens = a->context_lens;
  ap.history = a->history;
  ap.history_len = a->history_len;
  tv::launch_advance(ap, s);
  return check_launch("tv_llama_decode_step");
}

int tv_llama_graph_create(const tv_llama_model* m, const tv_llama_cache* c, const tv_llama_decode_args* a,
                          void* stream, void** graph) {
  if (!graph) return fail(TV_EINVAL, "tv_llama_graph_create: null graph handle");
  *graph = nullptr;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!s) return fail(TV_EINVAL, "tv_llama_graph_create: the NULL stream cannot be captured");
  hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return fail(TV_EHIP, "tv_llama_graph_create: begin capture: %s", hipGetErrorString(e));
  const int rc = tv_llama_decode_step(m, c, a, stream);
  hipGraph_t g = nullptr;
  e = hipStreamEndCapture(s, &g);
  if (rc != TV_OK) {
    if (g) hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return fail(TV_EHIP, "tv_llama_graph_create: end capture: %s", hipGetErrorString(e));
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return fail(TV_EHIP, "tv_llama_graph_create: instantiate: %s", hipGetErrorString(e));
  *graph = exec;
  return ok();
}

int tv_llama_graph_launch(void* graph, void* stream) {
  if (!graph) return fail(TV_EINVAL, "tv_llama_graph_launch: null graph");
  const hipError_t e = hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph), reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(TV_EHIP, "tv_llama_graph_launch: %s", hipGetErrorString(e));
  return ok();
}

int tv_llama_graph_destroy(void* graph) {
  if (!graph) return ok();
  const hipError_t e = hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph));
  if (e != hipSuccess) return fail(TV_EHIP, "tv_llama_graph_destroy: %s", hipGetErrorString(e));
  return ok();
}

size_t tv_llama_prefill_workspace_bytes(const tv_llama_model* model, int num_tokens) {
  if (!model || num_tokens <= 0 || model->n_heads <= 0 || model->head_dim <= 0 || model->dim <= 0 ||
      model->hidden_dim <= 0)
    return 0;
  return step_layout(model, num_tokens, 1, 1, 1, false).total;
}

int tv_llama_prefill(const tv_llama_model* m, const tv_llama_cache* c, const tv_llama_prefill_args* a, void* stream) {
  int rc = validate_model(m, "tv_llama_prefill");
  if (rc != TV_OK) return rc;
  if (!c || !c->k_caches || !c->v_caches || c->num_blocks <= 0 || c->block_size <= 0)
    return fail(TV_EINVAL, "tv_llama_prefill: bad cache");
  if (!a || a->num_tokens <= 0 || !a->tokens || !a->block_table || a->bt_width <= 0 || a->start_pos < 0)
    return fail(TV_EINVAL, "tv_llama_prefill: bad prefill arguments");
  if (a->logits && !aligned16(a->logits)) return fail(TV_EINVAL, "tv_llama_prefill: logits must be 16-byte aligned");
  const int M = a->num_tokens;
  if ((long long)a->start_pos + M > (long long)a->bt_width * c->block_size)
    return fail(TV_EINVAL, "tv_llama_prefill: the block table covers %lld positions, the chunk ends at %lld",
                (long long)a->bt_width * c->block_size, (long long)a->start_pos + M);
  const StepLayout L = step_layout(m, M, 1, 1, 1, false);
  if (!a->workspace || a->workspace_bytes < L.total || !aligned16(a->workspace))
    return fail(TV_EINVAL, "tv_llama_prefill: workspace of %zu bytes required (got %zu)", L.total, a->workspace_bytes);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void* ws = a->workspace;
  norm(at<float>(ws, L.x), at<void>(ws, L.xh), nullptr, 0, m->tok_embeddings, a->tokens, m->vocab_size,
       m->attention_norm[0], M, m->dim, m->norm_eps, m->dtype, s);
  LayerIO io{};
  io.M = M;
  io.x = at<float>(ws, L.x);
  io.xh = at<void>(ws, L.xh);
  io.part = at<float>(ws, L.part);
  io.q = at<void>(ws, L.q);
  io.attn = at<void>(ws, L.attn);
  io.h = at<void>(ws, L.h);
  io.decode = false;
  io.pargs = a;
  io.kst = at<void>(ws, L.kst);
  io.vst = at<void>(ws, L.vst);
  io.slots = at<int>(ws, L.slots);
  io.attn_ws = at<void>(ws, L.attn_ws);
  io.attn_ws_bytes = L.attn_ws_bytes;
  io.ks_qkv = L.ks_qkv;
  io.ks_o = L.ks_o;
  io.ks_2 = L.ks_2;
  if (a->attend_prefix && a->start_pos > 0) {
    // context of chunk row i: positions 0 .. start_pos + i (held in the slots region, unused by prefill)
    tv::launch_iota(io.slots, M, a->start_pos + 1, s);
    rc = check_launch("tv_llama_prefill");
    if (rc != TV_OK) return rc;
  }
  rc = run_layers(m, c, io, s);
  if (rc != TV_OK) return rc;
  unsigned long long* keys = at<unsigned long long>(ws, L.keys);
  const size_t es = elem_bytes(m->dtype);
  const void* last = reinterpret_cast<const char*>(io.xh) + (size_t)(M - 1) * m->dim * es;
  if (a->logits) {
    if (a->logits_last_only)
      linear(last, m->output, 1, m->vocab_size, m->dim, m->dim, m->dim, tv::kEpiLogits, a->logits, m->vocab_size,
             keys, m->dtype, s);
    else
      linear(io.xh, m->output, M, m->vocab_size, m->dim, m->dim, m->dim, tv::kEpiLogits, a->logits, m->vocab_size,
             nullptr, m->dtype, s);
  }
  if (a->next_token) {
    if (!a->logits || !a->logits_last_only)
      linear(last, m->output, 1, m->vocab_size, m->dim, m->dim, m->dim, tv::kEpiLogits, nullptr, m->vocab_size, keys,
             m->dtype, s);
    tv::AdvanceParams ap{};
    ap.keys = keys;
    ap.nparts = (m->vocab_size + tv::kLinBN - 1) / tv::kLinBN;
    ap.M = 1;
    ap.tokens = a->next_token;
    tv::launch_advance(ap, s);
  }
  return check_launch("tv_llama_prefill");
}

}  // extern "C"
