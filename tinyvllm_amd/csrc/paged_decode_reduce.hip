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
  float M = kNegInf;
  bool nan_seen = false;
  for (int i = 0; i < nparts; ++i) {
    const float mi = ml[2 * i];
    nan_seen |= (mi != mi);
    M = fmaxf(M, mi);
  }
  const float Mu = M == kNegInf ? 0.0f : M;
  for (int d = threadIdx.x; d < head_dim; d += 64) {
    float num = 0.0f, den = 0.0f;
    for (int i = 0; i < nparts; ++i) {
      const float w = ml[2 * i + 1] * fast_exp2(ml[2 * i] - Mu);
      num = fmaf(w, p.part_o[(base + i) * head_dim + d], num);
      den += w;
    }
    const float val = nan_seen ? __builtin_nanf("") : num / den;
    store_as(p.out, ((size_t)b * p.num_heads + h) * head_dim + d, val, p.out_dtype);
  }
}

}  // namespace tv
