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

// Schedule of an unsplit launch for paged_decode_scheduled_kernel: sched[0] =
// KV heads per row, sched[1 + rank] = b.  Sequences are ranked by 16 length classes (attended
// length * 16 / (width + 1)), longest class first, batch order inside a class
// -- one ballot per class and wave instead of a full sort.  Work-groups are
// dispatched in grid order, so the longest sequences start first and the last
// ones to start are short: the launch does not end on a few long sequences
// streaming while most CUs idle.  Any permutation is correct; this one only
// shortens the tail.
// sched[0] = KV heads per row: 2 when pairing is allowed (pair_ok, decided on
// the host from the item count) and the lengths are spread (longest >=
// kDecodePairSpread * shortest), else 1.  Pairs read each cache row's two
// heads together, but halve the number of items and double their length;
// that pays when the longest-first order can fill the end of the launch with
// short sequences, and loses when lengths are alike (on MI355X, 256
// Llama-3-8B-head sequences: 384 vs 401 us for U[512, 4096] lengths, 442 vs
// 418 us for equal lengths).  One
// work-group of 1024 threads, num_seqs <= 1024.
__global__ void __launch_bounds__(1024) decode_order_kernel(const int* context_lens, int num_seqs, int width,
                                                            int pair_ok, int* sched) {
  constexpr int NC = 16;
  __shared__ int cnt[16][NC];   // [wave][class] members
  __shared__ int wmin[16], wmax[16];
  const int b = threadIdx.x;
  const int wave = b >> 6, lane = b & 63;
  int cls = -1;
  int len = 0;
  if (b < num_seqs) {
    const int ctx = context_lens[b];
    len = ctx <= 0 ? width : (ctx < width ? ctx : width);
    cls = (int)((long long)len * NC / ((long long)width + 1));
  }
  int before = 0;   // members of my class in my wave below my lane
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const unsigned long long m = __builtin_amdgcn_ballot_w64(cls == k);
    if (lane == 0) cnt[wave][k] = __builtin_popcountll(m);
    if (cls == k) before = __builtin_popcountll(m & ((1ull << lane) - 1));
  }
  int lo = b < num_seqs ? len : 0x7FFFFFFF, hi = b < num_seqs ? len : 0;
#pragma unroll
  for (int msk = 1; msk < 64; msk <<= 1) {
    const int src = (lane ^ msk) << 2;
    lo = min(lo, __builtin_amdgcn_ds_bpermute(src, lo));
    hi = max(hi, __builtin_amdgcn_ds_bpermute(src, hi));
  }
  if (lane == 0) {
    wmin[wave] = lo;
    wmax[wave] = hi;
  }
  __syncthreads();
  if (b == 0) {
    int mn = 0x7FFFFFFF, mx = 0;
    for (int w = 0; w < 16; ++w) {
      mn = min(mn, wmin[w]);
      mx = max(mx, wmax[w]);
    }
    sched[0] = pair_ok && (long long)mx >= (long long)kDecodePairSpread * mn ? 2 : 1;
  }
  if (b >= num_seqs) return;
  int rank = before;
  for (int w = 0; w < 16; ++w) {
#pragma unroll
    for (int k = 0; k < NC; ++k) rank += (k > cls || (k == cls && w < wave)) ? cnt[w][k] : 0;
  }
  sched[1 + rank] = b;
}

}  // namespace tv
