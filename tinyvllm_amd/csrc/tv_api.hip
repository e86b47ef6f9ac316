// extern "C" entry points of libtvattn.so (declared in include/tv_attn.h).
// Host-side validation lives here; kernels assume validated arguments.
#include <cstdio>
#include <cstdarg>
#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <string>

#include "../../include/tv_attn.h"
#include "paged_decode_inst.h"
#include "tv_error.h"
#include "tv_device_cache.h"
#include "tv_params.h"

namespace tv {

namespace {
thread_local std::string g_err;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return TV_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TV_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

const char* last_error() { return g_err.c_str(); }

}  // namespace tv

namespace {

using tv::check_launch;
using tv::kMaxDevices;
using tv::fail;
using tv::ok;

bool valid_dtype(int d) { return d == TV_F32 || d == TV_F16 || d == TV_BF16; }
int elem_size(int d) { return d == TV_F32 ? 4 : 2; }
bool pow2(long long x) { return x > 0 && (x & (x - 1)) == 0; }
int ilog2(long long x) {
  int r = 0;
  while ((1LL << r) < x) ++r;
  return r;
}

// Whether a decode launch takes the wide work-groups (kDecodeWideWaves waves):
// unsplit, at most one (sequence, KV head) row per CU, every context within
// kDecodeWideTokens.  (Kernel shapes without a wide form, kDecodeWideOk, keep
// the 4-wave work-groups.)
bool decode_wide(int num_seqs, int rows_per_seq, long long width, int partition_size) {
  if (partition_size < width || width > tv::kDecodeWideTokens) return false;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess || cus < 1)
    return false;
  return (long long)num_seqs * rows_per_seq <= cus;
}

// Query heads of a GQA group that one decode work-group serves: the largest
// power of two <= 8 that divides the group.
constexpr int kDecodeGroupMax = 8;
int heads_per_group_chunk(int group) {
  for (int gt = kDecodeGroupMax; gt > 1; gt >>= 1)
    if (group % gt == 0) return gt;
  return 1;
}

// Largest vector width (bytes) dividing every given byte count and address.
int vec_width(std::initializer_list<long long> sizes, std::initializer_list<const void*> ptrs) {
  for (int w = 16; w > 2; w >>= 1) {
    bool ok = true;
    for (long long s : sizes) ok = ok && (s % w == 0);
    for (const void* p : ptrs) ok = ok && ((uintptr_t)p % w == 0);
    if (ok) return w;
  }
  return 2;
}

int paged_decode_impl(const char* who, void* out, const void* queries, const void* k_cache, const void* v_cache,
                      const int32_t* block_tables, const int32_t* context_lens, int num_seqs, int num_heads,
                      int num_kv_heads, int head_dim, int block_size, int num_blocks, int block_table_stride,
                      int max_blocks, float scale, int dtype, int out_dtype, int partition_size, void* workspace,
                      size_t workspace_bytes, void* stream);

// Scratch of tv_paged_decode_noalloc: the split-context partials or the
// longest-first schedule, in a file-scope device array instead of a caller's
// workspace.  Every device the library runs on holds its own copy until the
// process ends; the kernels fully write what they read back (no clearing).
constexpr size_t kDecodeScratchBytes = size_t(16) << 20;
__device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device
// (the host-side symbol is a stand-in, not a device address).
int decode_scratch(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TV_EHIP, "tv_paged_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(TV_EINVAL, "tv_paged_decode_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(TV_EHIP, "tv_paged_decode_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return TV_OK;
}

}  // namespace

extern "C" {

int tv_abi_version(void) { return 9; }

const char* tv_last_error(void) { return tv::last_error(); }

// Unsplit launches of kDecodeOrderMinSeqs .. kDecodeOrderMaxSeqs sequences run
// longest first (decode_order_kernel, paged_decode_scheduled_kernel), which
// needs num_seqs + 1 ints of workspace: KV heads per row, then the order.
static constexpr int kDecodeOrderMinSeqs = 32;
static constexpr int kDecodeOrderMaxSeqs = 1024;

size_t tv_paged_decode_workspace_bytes(int num_seqs, int num_heads, int head_dim, int max_blocks,
                                       int block_size, int partition_size) {
  if (num_seqs <= 0 || num_heads <= 0 || head_dim <= 0 || max_blocks <= 0 || block_size <= 0 ||
      partition_size <= 0)
    return 0;
  const long long width = (long long)max_blocks * block_size;
  const long long parts = (width + partition_size - 1) / partition_size;
  if (parts <= 1)
    return num_seqs >= kDecodeOrderMinSeqs && num_seqs <= kDecodeOrderMaxSeqs
               ? ((size_t)(num_seqs + 1) * sizeof(int) + 255) & ~(size_t)255
               : 0;
  return (size_t)num_seqs * num_heads * parts * (head_dim + 2) * sizeof(float);
}

int tv_paged_decode_partition_size(int num_seqs, int num_heads, int num_kv_heads, int head_dim, int max_blocks,
                                   int block_size, int dtype) {
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || max_blocks <= 0 ||
      block_size <= 0 || !valid_dtype(dtype))
    return fail(TV_EINVAL, "tv_paged_decode_partition_size: bad arguments"), 0;
  if (!(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256))
    return fail(TV_EUNSUPPORTED, "tv_paged_decode_partition_size: head_dim %d not supported", head_dim), 0;
  const long long width = (long long)max_blocks * block_size;
  const int whole = (int)((width + 15) / 16 * 16);
  const int group = num_heads / num_kv_heads;
  const int gt = heads_per_group_chunk(group);
  const long long rows = (long long)num_seqs * num_kv_heads * (group / gt);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess || cus < 1)
    return fail(TV_EHIP, "tv_paged_decode_partition_size: no device"), 0;
  if (rows >= 4LL * cus) return whole;
  if (rows <= cus && width <= tv::kDecodeWideTokens) return whole;   // one launch of wide work-groups
  const int slots = dtype == TV_F32   ? tv::decode_partitioned_slots<float>(head_dim, gt)
                    : dtype == TV_F16 ? tv::decode_partitioned_slots<_Float16>(head_dim, gt)
                                      : tv::decode_partitioned_slots<__bf16>(head_dim, gt);
  const long long parts = ((long long)slots + rows - 1) / rows;
  long long p = (width + parts - 1) / parts;
  p = (p + 15) / 16 * 16;
  if (p < 64) p = 64;
  return p < whole ? (int)p : whole;
}

int tv_paged_decode(void* out, const void* queries, const void* k_cache, const void* v_cache,
                    const int32_t* block_tables, const int32_t* context_lens, int num_seqs, int num_heads,
                    int num_kv_heads, int head_dim, int block_size, int num_blocks, int block_table_stride,
                    int max_blocks, float scale, int dtype, int out_dtype, int partition_size, void* workspace,
                    size_t workspace_bytes, void* stream) {
  return paged_decode_impl("tv_paged_decode", out, queries, k_cache, v_cache, block_tables, context_lens, num_seqs,
                           num_heads, num_kv_heads, head_dim, block_size, num_blocks, block_table_stride, max_blocks,
                           scale, dtype, out_dtype, partition_size, workspace, workspace_bytes, stream);
}

int tv_paged_decode_noalloc(void* out, const void* queries, const void* k_cache, const void* v_cache,
                            const int32_t* block_tables, const int32_t* context_lens, int num_seqs, int num_heads,
                            int num_kv_heads, int head_dim, int block_size, int num_blocks, int block_table_stride,
                            int max_blocks, float scale, int dtype, int out_dtype, int partition_size, void* stream) {
  if (num_seqs <= 0 || num_heads <= 0 || head_dim <= 0 || max_blocks <= 0 || block_size <= 0 || partition_size <= 0)
    return fail(TV_EINVAL, "tv_paged_decode_noalloc: bad shape (num_seqs=%d, num_heads=%d, head_dim=%d, "
                "max_blocks=%d, block_size=%d, partition_size=%d)", num_seqs, num_heads, head_dim, max_blocks,
                block_size, partition_size);
  const size_t need = tv_paged_decode_workspace_bytes(num_seqs, num_heads, head_dim, max_blocks, block_size,
                                                      partition_size);
  if (need > kDecodeScratchBytes)
    return fail(TV_EINVAL, "tv_paged_decode_noalloc: the launch needs %zu bytes of scratch, more than the %zu the "
                "library holds per device (use tv_paged_decode with a workspace, or larger partitions)",
                need, (size_t)kDecodeScratchBytes);
  void* scratch_ptr = nullptr;
  if (need > 0) {
    const int rc = decode_scratch(&scratch_ptr);
    if (rc != TV_OK) return rc;
  }
  return paged_decode_impl("tv_paged_decode_noalloc", out, queries, k_cache, v_cache, block_tables, context_lens,
                           num_seqs, num_heads, num_kv_heads, head_dim, block_size, num_blocks, block_table_stride,
                           max_blocks, scale, dtype, out_dtype, partition_size, scratch_ptr, need, stream);
}

}  // extern "C"

namespace {

int paged_decode_impl(const char* who, void* out, const void* queries, const void* k_cache, const void* v_cache,
                      const int32_t* block_tables, const int32_t* context_lens, int num_seqs, int num_heads,
                      int num_kv_heads, int head_dim, int block_size, int num_blocks, int block_table_stride,
                      int max_blocks, float scale, int dtype, int out_dtype, int partition_size, void* workspace,
                      size_t workspace_bytes, void* stream) {
  if (!out || !queries || !k_cache || !v_cache || !block_tables || !context_lens)
    return fail(TV_EINVAL, "%s: null pointer argument", who);
  if (!valid_dtype(dtype) || !(out_dtype == dtype || out_dtype == TV_F32))
    return fail(TV_EINVAL, "%s: bad dtype %d / out_dtype %d", who, dtype, out_dtype);
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(TV_EINVAL, "%s: bad head counts (num_seqs=%d, num_heads=%d, num_kv_heads=%d)", who,
                num_seqs, num_heads, num_kv_heads);
  if (block_size <= 0 || num_blocks <= 0 || block_table_stride < 0 || max_blocks <= 0 ||
      (block_table_stride > 0 && max_blocks > block_table_stride))
    return fail(TV_EINVAL, "%s: bad block geometry (block_size=%d, num_blocks=%d, stride=%d, max_blocks=%d)", who,
                block_size, num_blocks, block_table_stride, max_blocks);
  if ((long long)max_blocks * block_size > (1LL << 30))
    return fail(TV_EINVAL, "%s: context width too large", who);
  if (partition_size <= 0 || partition_size % 16 != 0)
    return fail(TV_EINVAL, "%s: partition_size must be a positive multiple of 16 (got %d)", who,
                partition_size);
  if (!(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256))
    return fail(TV_EUNSUPPORTED, "%s: head_dim %d not supported (16/32/64/128/256)", who, head_dim);
  if (dtype != TV_F32 && head_dim < 16)
    return fail(TV_EUNSUPPORTED, "%s: head_dim %d too small", who, head_dim);

  if ((uintptr_t)out % 16 || (uintptr_t)queries % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 ||
      (uintptr_t)block_tables % 4 || (uintptr_t)context_lens % 4)
    return fail(TV_EINVAL, "%s: queries/caches/out must be 16-byte aligned", who);

  const int group = num_heads / num_kv_heads;
  const int gt = heads_per_group_chunk(group);
  const long long width = (long long)max_blocks * block_size;
  const int max_parts = (int)((width + partition_size - 1) / partition_size);
  const size_t need = tv_paged_decode_workspace_bytes(num_seqs, num_heads, head_dim, max_blocks, block_size,
                                                      partition_size);
  if (max_parts > 1 && (!workspace || workspace_bytes < need))
    return fail(TV_EINVAL, "%s: workspace of %zu bytes required (got %zu)", who, need, workspace_bytes);
  // the longest-first schedule is optional: without room for it the launch runs in batch order
  const bool ordered = max_parts == 1 && need > 0 && workspace && workspace_bytes >= need;

  tv::DecodeParams p{};
  p.out = out;
  p.q = queries;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.block_tables = block_tables;
  p.context_lens = context_lens;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.head_chunks = group / gt;
  p.block_size = block_size;
  p.bs_log2 = pow2(block_size) ? ilog2(block_size) : -1;
  p.num_blocks = num_blocks;
  p.bt_stride = block_table_stride;
  p.max_blocks = max_blocks;
  p.scale = scale;
  p.partition_size = partition_size;
  p.max_parts = max_parts;
  p.out_dtype = out_dtype;
  if (max_parts > 1) {
    const size_t n_o = (size_t)num_seqs * num_heads * max_parts * head_dim;
    p.part_o = reinterpret_cast<float*>(workspace);
    p.part_ml = p.part_o + n_o;
  }
  if (max_parts > 65535 || num_seqs > 65535 || num_kv_heads * p.head_chunks > 65535)
    return fail(TV_EINVAL, "%s: grid too large", who);

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  p.num_seqs = num_seqs;
  bool pair = false;
  if (ordered) {
    if (dtype == TV_F32) pair = tv::decode_pair_allowed<float>(p, head_dim, gt);
    else if (dtype == TV_F16) pair = tv::decode_pair_allowed<_Float16>(p, head_dim, gt);
    else pair = tv::decode_pair_allowed<__bf16>(p, head_dim, gt);
  }
  if (ordered) {
    int* sched = reinterpret_cast<int*>(workspace);
    p.sched = sched;
    hipLaunchKernelGGL(tv::decode_order_kernel, dim3(1), dim3(1024), 0, s, context_lens, num_seqs, (int)width,
                       pair ? 1 : 0, sched);
  }
  // A small launch takes the wide work-groups; with GQA chunks of 4+ heads it
  // also serves half as many query heads per work-group when the doubled grid
  // still fits one row per CU: a wave's tile then costs half the score and P.V
  // arithmetic and the merge half the values (TinyLlama fp32 B4, ctx 17-250:
  // 9.25 -> 7.45 us; chunks of a quarter: 7.89).
  int gtw = gt;
  const bool wide = !ordered && decode_wide(num_seqs, num_kv_heads * p.head_chunks, width, partition_size);
  if (wide && gt >= 4 && decode_wide(num_seqs, num_kv_heads * (group / (gt / 2)), width, partition_size)) {
    gtw = gt / 2;
    p.head_chunks = group / gtw;
  }
  const dim3 grid(max_parts, num_kv_heads * p.head_chunks, num_seqs);
  bool launched = false;
  if (dtype == TV_F32) launched = tv::launch_paged_decode<float>(p, head_dim, gtw, pair, wide, grid, s);
  else if (dtype == TV_F16) launched = tv::launch_paged_decode<_Float16>(p, head_dim, gtw, pair, wide, grid, s);
  else launched = tv::launch_paged_decode<__bf16>(p, head_dim, gtw, pair, wide, grid, s);
  if (!launched) return fail(TV_EUNSUPPORTED, "%s: no kernel for head_dim=%d gt=%d", who, head_dim, gtw);
  int rc = check_launch(who);
  if (rc != TV_OK || max_parts <= 1) return rc;
  if (head_dim > 256) return fail(TV_EUNSUPPORTED, "%s: merge supports head_dim <= 256", who);
  hipLaunchKernelGGL(tv::paged_decode_reduce_kernel, dim3(num_heads, num_seqs), dim3(64), 0, s, p, head_dim);
  return check_launch(who);
}

}  // namespace

extern "C" {

static void prefill_params(tv::PrefillParams& p, void* out, const void* q, const void* k, const void* v, int q_len,
                           int kv_len, int num_heads, int num_kv_heads, int head_dim, int head_dim_v,
                           int64_t q_stride, int64_t k_stride, int64_t v_stride, int64_t out_stride, int causal,
                           float scale, int out_dtype, int chunk_tiles) {
  p = tv::PrefillParams{};
  p.out = out;
  p.q = q;
  p.k = k;
  p.v = v;
  p.q_len = q_len;
  p.kv_len = kv_len;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.head_dim = head_dim;
  p.head_dim_v = head_dim_v;
  p.q_stride = q_stride;
  p.k_stride = k_stride;
  p.v_stride = v_stride;
  p.out_stride = out_stride;
  p.causal = causal ? 1 : 0;
  p.scale = scale;
  p.out_dtype = out_dtype;
  if (chunk_tiles <= 0) {
    // Default: no split.  Splitting a causal row across work-groups writes an
    // fp32 partial of the whole query tile per chunk and reads it back in a
    // merge kernel; on MI355X that round trip cost more than the shorter chains
    // saved at every chunk size tried (L = 512 / 1024, 32 heads, head_dim 64).
    chunk_tiles = kv_len;   // >= the number of key tiles of any size
  }
  p.chunk_tiles = chunk_tiles;
}

size_t tv_flash_prefill_workspace_bytes(int q_len, int kv_len, int num_heads, int head_dim, int head_dim_v,
                                        int causal, int dtype, int chunk_tiles) {
  if (q_len <= 0 || kv_len <= 0 || num_heads <= 0 || head_dim <= 0 || head_dim_v <= 0 || !valid_dtype(dtype))
    return 0;
  tv::PrefillParams p;
  // dense strides and aligned placeholder addresses: the size assumes the MFMA path
  prefill_params(p, nullptr, (void*)256, (void*)256, (void*)256, q_len, kv_len, num_heads, 1, head_dim, head_dim_v,
                 (int64_t)num_heads * head_dim, head_dim, head_dim_v, (int64_t)num_heads * head_dim_v, causal, 1.0f,
                 dtype, chunk_tiles);
  return tv::prefill_workspace_bytes(p, dtype);
}

int tv_flash_prefill(void* out, const void* q, const void* k, const void* v, int q_len, int kv_len, int num_heads,
                     int num_kv_heads, int head_dim, int head_dim_v, int64_t q_stride, int64_t k_stride,
                     int64_t v_stride, int64_t out_stride, int causal, float scale, int dtype, int out_dtype,
                     int chunk_tiles, void* workspace, size_t workspace_bytes, void* stream) {
  if (!out || !q || !k || !v) return fail(TV_EINVAL, "tv_flash_prefill: null pointer argument");
  if (!valid_dtype(dtype) || !(out_dtype == dtype || out_dtype == TV_F32))
    return fail(TV_EINVAL, "tv_flash_prefill: bad dtype %d / out_dtype %d", dtype, out_dtype);
  if (q_len <= 0 || kv_len <= 0)
    return fail(TV_EINVAL, "tv_flash_prefill: empty sequence (q_len=%d, kv_len=%d)", q_len, kv_len);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(TV_EINVAL, "tv_flash_prefill: bad head counts (%d, %d)", num_heads, num_kv_heads);
  if (head_dim <= 0 || head_dim_v <= 0)
    return fail(TV_EINVAL, "tv_flash_prefill: bad head dims (%d, %d)", head_dim, head_dim_v);
  if (q_stride < (int64_t)num_heads * head_dim || k_stride < (int64_t)num_kv_heads * head_dim ||
      v_stride < (int64_t)num_kv_heads * head_dim_v || out_stride < (int64_t)num_heads * head_dim_v)
    return fail(TV_EINVAL, "tv_flash_prefill: token stride smaller than a token row");
  if (q_len > 65535 * 64 || num_heads > 65535)
    return fail(TV_EINVAL, "tv_flash_prefill: grid too large");
  if ((uintptr_t)workspace % 16 != 0) return fail(TV_EINVAL, "tv_flash_prefill: workspace must be 16-byte aligned");
  tv::PrefillParams p;
  prefill_params(p, out, q, k, v, q_len, kv_len, num_heads, num_kv_heads, head_dim, head_dim_v, q_stride, k_stride,
                 v_stride, out_stride, causal, scale, out_dtype, chunk_tiles);
  const int rc = tv::launch_flash_prefill(p, dtype, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
  if (rc == 1)
    return fail(TV_EUNSUPPORTED, "tv_flash_prefill: head_dim %d / %d not supported (max 256)", head_dim, head_dim_v);
  if (rc == 2)
    return fail(TV_EINVAL, "tv_flash_prefill: workspace of %zu bytes required (got %zu)",
                tv::prefill_workspace_bytes(p, dtype), workspace_bytes);
  return check_launch("tv_flash_prefill");
}

int tv_flash_prefill_varlen(void* out, const void* q, const void* k, const void* v, const int32_t* cu_seqlens_q,
                            const int32_t* cu_seqlens_k, const int32_t* seq_order, int num_seqs, int max_q_len,
                            int max_kv_len, int64_t total_q, int num_heads, int num_kv_heads, int head_dim,
                            int64_t q_stride, int64_t k_stride, int64_t v_stride, int64_t out_stride, int causal,
                            float scale, int dtype, int out_dtype, void* stream) {
  if (!out || !q || !k || !v || !cu_seqlens_q || !cu_seqlens_k)
    return fail(TV_EINVAL, "tv_flash_prefill_varlen: null pointer argument");
  if (!valid_dtype(dtype) || !(out_dtype == dtype || out_dtype == TV_F32))
    return fail(TV_EINVAL, "tv_flash_prefill_varlen: bad dtype %d / out_dtype %d", dtype, out_dtype);
  if (num_seqs <= 0 || num_seqs > 65535 || max_q_len <= 0 || max_kv_len <= 0 || total_q < max_q_len)
    return fail(TV_EINVAL, "tv_flash_prefill_varlen: bad sizes (num_seqs=%d, max_q_len=%d, max_kv_len=%d)",
                num_seqs, max_q_len, max_kv_len);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || num_heads > 65535)
    return fail(TV_EINVAL, "tv_flash_prefill_varlen: bad head counts (%d, %d)", num_heads, num_kv_heads);
  if (q_stride < (int64_t)num_heads * head_dim || k_stride < (int64_t)num_kv_heads * head_dim ||
      v_stride < (int64_t)num_kv_heads * head_dim || out_stride < (int64_t)num_heads * head_dim)
    return fail(TV_EINVAL, "tv_flash_prefill_varlen: token stride smaller than a token row");
  if (max_q_len > 65535 * 64) return fail(TV_EINVAL, "tv_flash_prefill_varlen: grid too large");
  tv::PrefillParams p;
  prefill_params(p, out, q, k, v, max_q_len, max_kv_len, num_heads, num_kv_heads, head_dim, head_dim, q_stride,
                 k_stride, v_stride, out_stride, causal, scale, out_dtype, 0);
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.seq_order = seq_order;
  const int rc = tv::launch_flash_prefill_varlen(p, num_seqs, max_q_len, max_kv_len, total_q, dtype,
                                                 reinterpret_cast<hipStream_t>(stream));
  if (rc == 1)
    return fail(TV_EUNSUPPORTED,
                "tv_flash_prefill_varlen: fp16 / bf16, head_dim 64 or 128 and 16-byte aligned rows only "
                "(dtype %d, head_dim %d)", dtype, head_dim);
  return check_launch("tv_flash_prefill_varlen");
}

int tv_flash_prefill_paged(void* out, const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* block_table, int num_blocks, int block_size, int q_len, int start_pos,
                           int num_heads, int num_kv_heads, int head_dim, int64_t q_stride, int64_t out_stride,
                           int causal, float scale, int dtype, int out_dtype, void* stream) {
  if (!out || !q || !k_cache || !v_cache || !block_table)
    return fail(TV_EINVAL, "tv_flash_prefill_paged: null pointer argument");
  if (!valid_dtype(dtype) || !(out_dtype == dtype || out_dtype == TV_F32))
    return fail(TV_EINVAL, "tv_flash_prefill_paged: bad dtype %d / out_dtype %d", dtype, out_dtype);
  if (q_len <= 0 || start_pos < 0 || num_blocks <= 0 || block_size <= 0 || (long long)start_pos + q_len > (1LL << 30))
    return fail(TV_EINVAL, "tv_flash_prefill_paged: bad sizes (q_len=%d, start_pos=%d, num_blocks=%d, block_size=%d)",
                q_len, start_pos, num_blocks, block_size);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || num_heads > 65535)
    return fail(TV_EINVAL, "tv_flash_prefill_paged: bad head counts (%d, %d)", num_heads, num_kv_heads);
  if (q_stride < (int64_t)num_heads * head_dim || out_stride < (int64_t)num_heads * head_dim)
    return fail(TV_EINVAL, "tv_flash_prefill_paged: token stride smaller than a token row");
  if (!pow2(block_size)) return fail(TV_EUNSUPPORTED, "tv_flash_prefill_paged: block_size %d is not a power of two",
                                     block_size);
  if (q_len > 65535 * 64) return fail(TV_EINVAL, "tv_flash_prefill_paged: grid too large");
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  tv::PrefillParams p;
  prefill_params(p, out, q, k_cache, v_cache, q_len, start_pos + q_len, num_heads, num_kv_heads, head_dim, head_dim,
                 q_stride, row, row, out_stride, causal, scale, out_dtype, 0);
  p.kv_table = block_table;
  p.kv_bs_log2 = ilog2(block_size);
  p.kv_num_blocks = num_blocks;
  p.q_pos_offset = start_pos;
  const int rc = tv::launch_flash_prefill_paged(p, dtype, reinterpret_cast<hipStream_t>(stream));
  if (rc == 1)
    return fail(TV_EUNSUPPORTED,
                "tv_flash_prefill_paged: fp16 / bf16, head_dim 64 or 128, 16-byte aligned rows and at most 4096 "
                "blocks only (dtype %d, head_dim %d)", dtype, head_dim);
  return check_launch("tv_flash_prefill_paged");
}

static int kv_write_common(const char* name, void* k_cache, void* v_cache, const void* k, const void* v,
                           const int32_t* slots, int base_slot, int num_tokens, int num_kv_heads, int head_dim,
                           int block_size, int num_blocks, int64_t k_stride, int64_t v_stride, int dtype,
                           uint32_t* err_count, void* stream) {
  if (!k_cache || !v_cache || !k || !v) return fail(TV_EINVAL, "%s: null pointer argument", name);
  if (!valid_dtype(dtype)) return fail(TV_EINVAL, "%s: bad dtype %d", name, dtype);
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks <= 0)
    return fail(TV_EINVAL, "%s: bad shape", name);
  const long long row = (long long)num_kv_heads * head_dim;
  if (k_stride < row || v_stride < row) return fail(TV_EINVAL, "%s: token stride smaller than a row", name);
  if (num_tokens == 0) return ok();
  const int es = elem_size(dtype);
  const int w = vec_width({row * es, k_stride * es, v_stride * es}, {k_cache, v_cache, k, v});
  tv::KVWriteParams p{};
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.k = k;
  p.v = v;
  p.slots = slots;
  p.base_slot = base_slot;
  p.num_tokens = num_tokens;
  p.row_vecs = (int)(row * es / w);
  p.k_stride = k_stride * es / w;
  p.v_stride = v_stride * es / w;
  p.num_slots = (long long)num_blocks * block_size;
  p.err_count = err_count;
  tv::launch_kv_write(p, w, reinterpret_cast<hipStream_t>(stream));
  return check_launch(name);
}

int tv_reshape_and_cache(void* k_cache, void* v_cache, const void* k, const void* v, const int32_t* slot_mapping,
                         int num_tokens, int num_kv_heads, int head_dim, int block_size, int num_blocks,
                         int64_t k_stride, int64_t v_stride, int dtype, uint32_t* err_count, void* stream) {
  if (!slot_mapping && num_tokens > 0) return fail(TV_EINVAL, "tv_reshape_and_cache: null slot_mapping");
  return kv_write_common("tv_reshape_and_cache", k_cache, v_cache, k, v, slot_mapping, 0, num_tokens, num_kv_heads,
                         head_dim, block_size, num_blocks, k_stride, v_stride, dtype, err_count, stream);
}

int tv_write_kv(void* k_cache, void* v_cache, const void* k, const void* v, int block_id, int start_offset,
                int num_tokens, int num_kv_heads, int head_dim, int block_size, int num_blocks, int64_t k_stride,
                int64_t v_stride, int dtype, void* stream) {
  if (block_id < 0 || block_id >= num_blocks)
    return fail(TV_EINVAL, "tv_write_kv: block_id %d outside [0, %d)", block_id, num_blocks);
  if (start_offset < 0 || num_tokens < 0 || start_offset + num_tokens > block_size)
    return fail(TV_EINVAL, "tv_write_kv: rows [%d, %d) do not fit a block of %d", start_offset,
                start_offset + num_tokens, block_size);
  return kv_write_common("tv_write_kv", k_cache, v_cache, k, v, nullptr, block_id * block_size + start_offset,
                         num_tokens, num_kv_heads, head_dim, block_size, num_blocks, k_stride, v_stride, dtype,
                         nullptr, stream);
}

int tv_read_kv_blocks(void* k_out, void* v_out, const void* k_cache, const void* v_cache, const int32_t* block_ids,
                      int num_block_ids, int context_len, int num_kv_heads, int head_dim, int block_size,
                      int num_blocks, int dtype, void* stream) {
  if (!valid_dtype(dtype)) return fail(TV_EINVAL, "tv_read_kv_blocks: bad dtype %d", dtype);
  if (context_len < 0 || num_block_ids < 0 || (long long)context_len > (long long)num_block_ids * block_size)
    return fail(TV_EINVAL, "tv_read_kv_blocks: context_len %d exceeds %d blocks of %d", context_len, num_block_ids,
                block_size);
  if (context_len == 0) return ok();
  if (!k_out || !v_out || !k_cache || !v_cache || !block_ids)
    return fail(TV_EINVAL, "tv_read_kv_blocks: null pointer argument");
  const int es = elem_size(dtype);
  const long long row = (long long)num_kv_heads * head_dim * es;
  const int w = vec_width({row}, {k_out, v_out, k_cache, v_cache});
  tv::KVGatherParams p{};
  p.k_out = k_out;
  p.v_out = v_out;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.block_ids = block_ids;
  p.context_len = context_len;
  p.block_size = block_size;
  p.row_vecs = (int)(row / w);
  p.num_blocks = num_blocks;
  tv::launch_kv_gather(p, w, reinterpret_cast<hipStream_t>(stream));
  return check_launch("tv_read_kv_blocks");
}

}  // extern "C"
