// Streaming-read ceiling: every 16-byte vector of a buffer read once, nothing
// written but one word per work-group when a never-taken test passes (so the
// loads stay live).  The measurement the HBM-bound kernels are compared with:
// how fast this part delivers a plain sequential read with ordinary or
// non-temporal 16-byte loads at a chosen number of loads in flight per lane.
#include "tv_common.h"
#include "tv_error.h"

#include "tv_attn.h"
#include "tv_bench.h"

namespace tv {

// Interleaved (CONTIG false): thread t of work-group g reads vectors
// g*256 + t + i*stride (stride = all lanes of the grid).  Contiguous (CONTIG
// true): work-group g reads its own range [g*per, (g+1)*per) of the buffer,
// 256*U consecutive vectors per iteration.  Either way U loads per lane are
// issued before the first is consumed.
template <int U, bool NT, bool CONTIG>
__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4* __restrict__ src, long long n, uint32_t* sink) {
  long long i, end, stride;
  if constexpr (CONTIG) {
    const long long per = (n + gridDim.x - 1) / gridDim.x;
    i = min((long long)blockIdx.x * per, n) + threadIdx.x;
    end = min((long long)(blockIdx.x + 1) * per, n);
    stride = 256;
  } else {
    i = (long long)blockIdx.x * 256 + threadIdx.x;
    end = n;
    stride = (long long)gridDim.x * 256;
  }
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (U - 1) * stride < end; i += U * stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(src + i + u * stride) : src[i + u * stride];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  for (; i < end; i += stride) acc ^= src[i];
  const uint32_t r = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (r == 0x9e3779b9u) sink[blockIdx.x] = r;
}

}  // namespace tv

extern "C" int tv_stream_read(const void* src, int64_t bytes, int nontemporal, int loads_in_flight,
                              int work_groups, int contiguous, uint32_t* sink, void* stream) {
  using namespace tv;
  if (!src || !sink || bytes <= 0 || bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(src) & 15) != 0)
    return fail(TV_EINVAL, "tv_stream_read: need a 16-byte aligned buffer of a multiple of 16 bytes");
  if (work_groups <= 0) return fail(TV_EINVAL, "tv_stream_read: work_groups must be positive");
  const auto* s = reinterpret_cast<const u32x4*>(src);
  const long long n = bytes / 16;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(work_groups), block(256);
#define TV_SR_CASE(U, NT, C)                                                                   \
  case (U) * 4 + (NT) * 2 + (C):                                                               \
    hipLaunchKernelGGL((stream_read_kernel<U, NT, C>), grid, block, 0, st, s, n, sink); break;
  switch (loads_in_flight * 4 + (nontemporal ? 2 : 0) + (contiguous ? 1 : 0)) {
    TV_SR_CASE(4, false, false)
    TV_SR_CASE(4, false, true)
    TV_SR_CASE(4, true, false)
    TV_SR_CASE(4, true, true)
    TV_SR_CASE(8, false, false)
    TV_SR_CASE(8, false, true)
    TV_SR_CASE(8, true, false)
    TV_SR_CASE(8, true, true)
    default: return fail(TV_EINVAL, "tv_stream_read: loads_in_flight must be 4 or 8");
  }
#undef TV_SR_CASE
  return check_launch("tv_stream_read");
}
