// KV-cache movement kernels for the paged layout [num_blocks, block_size, Hkv, D].
//
// kv_write_kernel: token t's K and V rows (Hkv*D contiguous elements) are copied
// to flat cache slot s_t = slot_mapping[t] (or base_slot + t when no mapping is
// given), i.e. block s_t / block_size, row s_t % block_size
// (tinyvllm/core/kv_cache.py:34-38, driven per chunk by llama.py:199-209 and per
// token by llama.py:381-386).  Negative slots are padding and are skipped; slots
// past the cache are skipped and counted in *err_count when it is non-null.
//
// kv_gather_kernel: read_kv_blocks (kv_cache.py:40-55): output row t is cache
// block ids[t / block_size], row t % block_size, for t < context_len.
#include "tv_common.h"
#include "tv_params.h"

namespace tv {

template <typename V>
__global__ void __launch_bounds__(256) kv_write_kernel(const KVWriteParams p) {
  const long long total = (long long)p.num_tokens * p.row_vecs;
  V* kc = reinterpret_cast<V*>(p.k_cache);
  V* vc = reinterpret_cast<V*>(p.v_cache);
  const V* k = reinterpret_cast<const V*>(p.k);
  const V* v = reinterpret_cast<const V*>(p.v);
  for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int t = (int)(idx / p.row_vecs);
    const int e = (int)(idx - (long long)t * p.row_vecs);
    const long long slot = p.slots ? (long long)p.slots[t] : (long long)p.base_slot + t;
    if (slot < 0) continue;
    if (slot >= p.num_slots) {
      if (e == 0 && p.err_count) atomicAdd(p.err_count, 1u);
      continue;
    }
    const long long dst = slot * p.row_vecs + e;
    kc[dst] = k[(long long)t * p.k_stride + e];
    vc[dst] = v[(long long)t * p.v_stride + e];
  }
}

template <typename V>
__global__ void __launch_bounds__(256) kv_gather_kernel(const KVGatherParams p) {
  const long long total = (long long)p.context_len * p.row_vecs;
  for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int t = (int)(idx / p.row_vecs);
    const int e = (int)(idx - (long long)t * p.row_vecs);
    const int blk = p.block_ids[t / p.block_size];
    V kv, vv;
    if ((unsigned)blk < (unsigned)p.num_blocks) {
      const long long src = ((long long)blk * p.block_size + t % p.block_size) * p.row_vecs + e;
      kv = reinterpret_cast<const V*>(p.k_cache)[src];
      vv = reinterpret_cast<const V*>(p.v_cache)[src];
    } else {
      kv = V{};
      vv = V{};
    }
    reinterpret_cast<V*>(p.k_out)[idx] = kv;
    reinterpret_cast<V*>(p.v_out)[idx] = vv;
  }
}

static int grid_for(long long total) {
  long long g = (total + 255) / 256;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

// vec_bytes in {16, 8, 4, 2}; row_vecs and strides are already in vector units.
void launch_kv_write(const KVWriteParams& p, int vec_bytes, hipStream_t stream) {
  const int grid = grid_for((long long)p.num_tokens * p.row_vecs);
  switch (vec_bytes) {
    case 16: hipLaunchKernelGGL(kv_write_kernel<u32x4>, dim3(grid), dim3(256), 0, stream, p); break;
    case 8: hipLaunchKernelGGL(kv_write_kernel<u32x2>, dim3(grid), dim3(256), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(kv_write_kernel<uint32_t>, dim3(grid), dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL(kv_write_kernel<uint16_t>, dim3(grid), dim3(256), 0, stream, p); break;
  }
}

void launch_kv_gather(const KVGatherParams& p, int vec_bytes, hipStream_t stream) {
  const int grid = grid_for((long long)p.context_len * p.row_vecs);
  switch (vec_bytes) {
    case 16: hipLaunchKernelGGL(kv_gather_kernel<u32x4>, dim3(grid), dim3(256), 0, stream, p); break;
    case 8: hipLaunchKernelGGL(kv_gather_kernel<u32x2>, dim3(grid), dim3(256), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(kv_gather_kernel<uint32_t>, dim3(grid), dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL(kv_gather_kernel<uint16_t>, dim3(grid), dim3(256), 0, stream, p); break;
  }
}

}  // namespace tv
