// Split-context (flash-decoding) merge: combines the per-partition partials
// written by paged_decode_kernel into the final output.
//
// Partition p of (sequence b, query head h) holds M_p (running max, log2
// units), L_p = sum 2^(s - M_p) and O_p = (sum 2^(s - M_p) v) / L_p.  The merged
// output is sum_p w_p O_p / sum_p w_p with w_p = L_p 2^(M_p - max_p M_p), which
// equals the single-pass softmax exactly in real arithmetic.
#include "paged_decode.cuh"

namespace tv {

__global__ void __launch_bounds__(64) paged_decode_reduce_kernel(const DecodeParams p, int head_dim) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  float bias;
  const int len = decode_len(p, b, bias);
  const int nparts = (len + p.partition_size - 1) / p.partition_size;
  if (nparts <= 1) return;

  const size_t base = ((size_t)b * p.num_heads + h) * p.max_parts;
  const float* ml = p.part_ml + base * 2;
  const float* po = p.part_o + base * head_dim;
  const int lane = threadIdx.x;
  // global maximum over the partitions (lane i reads partitions i, i+64, ...)
  float M = kNegInf;
  bool nan_seen = false;
  for (int i = lane; i < nparts; i += 64) {
    const float mi = ml[2 * i];
    nan_seen |= (mi != mi);
    M = fmaxf(M, mi);
  }
  M = group_max<64>(M);
  nan_seen = __builtin_amdgcn_ballot_w64(nan_seen) != 0;
  const float Mu = M == kNegInf ? 0.0f : M;
  // per-partition weights w_i = L_i * 2^(M_i - M) through LDS, in chunks of 256
  __shared__ float sw[256];
  float num[4] = {0.f, 0.f, 0.f, 0.f};
  float den = 0.0f;
  for (int c0 = 0; c0 < nparts; c0 += 256) {
    const int cn = min(256, nparts - c0);
    __syncthreads();
    for (int i = lane; i < cn; i += 64) {
      const float w = ml[2 * (c0 + i) + 1] * fast_exp2(ml[2 * (c0 + i)] - Mu);
      sw[i] = w;
      den += w;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int d = lane + 64 * t;
      if (d < head_dim) {
        float a = num[t];
#pragma unroll 4
        for (int i = 0; i < cn; ++i) a = fmaf(sw[i], po[(size_t)(c0 + i) * head_dim + d], a);
        num[t] = a;
      }
    }
  }
  den = group_sum<64>(den);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int d = lane + 64 * t;
    if (d < head_dim)
      store_as(p.out, ((size_t)b * p.num_heads + h) * head_dim + d, nan_seen ? __builtin_nanf("") : num[t] / den,
               p.out_dtype);
  }
}

// Longest-first schedule of an unsplit decode launch: order[rank] = b, where
// rank counts the sequences that attend to more positions than b (ties by
// index).  Work-groups are dispatched in grid order, so the longest sequences
// start first and the last ones to start are short: the launch does not end
// on a few long sequences streaming while most CUs idle.  Any permutation is
// correct; this one only shortens the tail.  grid ceil(B / 256), 256 threads.
__global__ void __launch_bounds__(256) decode_order_kernel(const int* context_lens, int num_seqs, int width,
                                                           int* order) {
  __shared__ int sl[256];
  const int b = blockIdx.x * 256 + threadIdx.x;
  auto eff = [&](int ctx) { return ctx <= 0 ? width : (ctx < width ? ctx : width); };
  const int mine = b < num_seqs ? eff(context_lens[b]) : 0;
  int rank = 0;
  for (int base = 0; base < num_seqs; base += 256) {
    __syncthreads();
    if (base + (int)threadIdx.x < num_seqs) sl[threadIdx.x] = eff(context_lens[base + threadIdx.x]);
    __syncthreads();
    const int n = min(256, num_seqs - base);
    for (int j = 0; j < n; ++j) {
      const int lj = sl[j];
      rank += (lj > mine) || (lj == mine && base + j < b);
    }
  }
  if (b < num_seqs) order[rank] = b;
}

}  // namespace tv
