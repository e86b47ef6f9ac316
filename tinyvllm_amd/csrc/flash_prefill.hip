// Causal / full attention over one prompt ("flash prefill") for gfx950.
//
// Semantics follow tinyvllm/model/llama.py:58-94: q [Lq, Hq, D], k [Lk, Hkv, D],
// v [Lk, Hkv, Dv]; scores (q.k)*scale; with `causal`, key j is excluded for query
// i when j > i (top-left aligned, llama.py:86-90); query head h reads KV head
// h / (Hq/Hkv).  Every query row keeps key 0, so the reference's -1e9 additive
// mask and the exclusion used here give the same softmax.
//
// Two kernels:
//  * prefill_mfma_kernel<T, D>: fp16/bf16, D in {64, 128}, Dv == D.  A work-group
//    of 4 waves owns 64 query rows of one head; each wave owns 16 rows.  Key
//    tiles of 64 rows are staged in LDS (K row-major, V transposed).  Scores are
//    computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_{f16,bf16}; the
//    accumulator layout of S^T (lane = query column, 4 consecutive keys per
//    16-key block) is exactly the B-operand layout needed for O^T = V^T P^T once
//    the two operands agree on the order of the reduction index, so P never
//    leaves registers.
//  * prefill_generic_kernel<T>: any D, Dv <= 256, any element type (fp32 path and
//    odd head sizes).  One wave per (query row, head); 64 keys per step.
#include "tv_common.h"
#include "tv_params.h"

namespace tv {

// ---------------------------------------------------------------------------
// MFMA kernel
// ---------------------------------------------------------------------------

template <typename T> __device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma16x16x32<_Float16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma16x16x32<__bf16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<_Float16>(float a, float b) {
  return (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}
template <> __device__ __forceinline__ uint32_t pack2<__bf16>(float a, float b) {
  return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}

__device__ __forceinline__ int prefill_head(int x, int num_heads, int remap) {
  // Work-groups are dealt to the 8 XCDs round-robin by linear id; with the head
  // on grid.x, id % 8 == x % 8.  Mapping x -> (x % 8) * (Hq / 8) + x / 8 puts
  // Hq/8 consecutive heads (one GQA group or a part of one) on the same XCD so
  // their shared K/V tiles hit that XCD's L2.
  if (!remap) return x;
  const int per = num_heads >> 3;
  return (x & 7) * per + (x >> 3);
}

template <typename T, int D>
__global__ void __launch_bounds__(256) prefill_mfma_kernel(const PrefillParams p) {
  constexpr int BM = 64;          // query rows per work-group
  constexpr int BN = 64;          // keys per tile
  constexpr int KP = D + 8;       // LDS pitch of the K tile (elements)
  constexpr int VP = BN + 8;      // LDS pitch of the V^T tile (elements)
  constexpr int DB = D / 16;      // 16-row blocks of O^T
  constexpr int KS = D / 32;      // MFMA steps over the head dim
  __shared__ __attribute__((aligned(16))) uint16_t sk[BN * KP];
  __shared__ __attribute__((aligned(16))) uint16_t sv[D * VP];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;        // 0..3
  const int col = lane & 15;

  const int h = prefill_head(blockIdx.x, p.num_heads, p.xcd_remap);
  const int nqt = (p.q_len + BM - 1) / BM;
  const int qt = nqt - 1 - (int)blockIdx.y;   // longest causal rows first
  const int kvh = h / (p.num_heads / p.num_kv_heads);
  const int qi = qt * BM + wave * 16 + col;

  const T* qg = reinterpret_cast<const T*>(p.q);
  const T* kg = reinterpret_cast<const T*>(p.k);
  const T* vg = reinterpret_cast<const T*>(p.v);

  u32x4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (qi < p.q_len)
      qf[ks] = *reinterpret_cast<const u32x4*>(qg + (size_t)qi * p.q_stride + (size_t)h * D + ks * 32 + g * 8);
    else
      qf[ks] = u32x4{0, 0, 0, 0};
  }

  f32x4 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf;
  float lsum = 0.0f;
  const float c = p.scale * kLog2e;

  const int kend = p.causal ? min(p.kv_len, qt * BM + BM) : p.kv_len;
  const int nkt = (kend + BN - 1) / BN;

  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * BN;
    __syncthreads();
    // K tile -> LDS, row-major [key][d]
    for (int idx = tid; idx < BN * (D / 8); idx += 256) {
      const int key = idx / (D / 8);
      const int ch = idx - key * (D / 8);
      const int kidx = k0 + key;
      u32x4 val = u32x4{0, 0, 0, 0};
      if (kidx < p.kv_len)
        val = *reinterpret_cast<const u32x4*>(kg + (size_t)kidx * p.k_stride + (size_t)kvh * D + ch * 8);
      *reinterpret_cast<u32x4*>(&sk[key * KP + ch * 8]) = val;
    }
    // V tile -> LDS, transposed [d][key]
    for (int idx = tid; idx < BN * (D / 8); idx += 256) {
      const int key = idx % BN;
      const int ch = idx / BN;
      const int kidx = k0 + key;
      u32x4 val = u32x4{0, 0, 0, 0};
      if (kidx < p.kv_len)
        val = *reinterpret_cast<const u32x4*>(vg + (size_t)kidx * p.v_stride + (size_t)kvh * D + ch * 8);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        sv[(ch * 8 + 2 * w) * VP + key] = (uint16_t)(val[w] & 0xffffu);
        sv[(ch * 8 + 2 * w + 1) * VP + key] = (uint16_t)(val[w] >> 16);
      }
    }
    __syncthreads();

    // S^T = K Q^T for four 16-key blocks: st[kb][i] = S[q = qi][key = k0 + kb*16 + 4g + i]
    f32x4 st[BN / 16];
#pragma unroll
    for (int kb = 0; kb < BN / 16; ++kb) {
      st[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&sk[(kb * 16 + col) * KP + ks * 32 + g * 8]);
        st[kb] = mfma16x16x32<T>(a, qf[ks], st[kb]);
      }
    }

    // scale, mask, online softmax for this lane's query column
    float mt = kNegInf;
#pragma unroll
    for (int kb = 0; kb < BN / 16; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kidx = k0 + kb * 16 + 4 * g + i;
        const bool ok = kidx < p.kv_len && (!p.causal || kidx <= qi);
        const float x = ok ? st[kb][i] * c : kNegInf;
        st[kb][i] = x;
        mt = fmaxf(mt, x);
      }
    }
    mt = fmaxf(mt, shfl_xor(mt, 16));
    mt = fmaxf(mt, shfl_xor(mt, 32));
    const float mn = fmaxf(m, mt);
    const float mu = mn == kNegInf ? 0.0f : mn;
    const float alpha = fast_exp2(m - mu);
    m = mn;
    float ls = 0.0f;
#pragma unroll
    for (int kb = 0; kb < BN / 16; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = fast_exp2(st[kb][i] - mu);
        st[kb][i] = e;
        ls += e;
      }
    lsum = lsum * alpha + ls;
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] *= alpha;

    // P^T fragments: reduction index kk = 8g + j maps to key 4g+j (j<4) of block
    // 2*ks2 and key 4g+j-4 (j>=4) of block 2*ks2+1.
    u32x4 pf[BN / 32];
#pragma unroll
    for (int ks2 = 0; ks2 < BN / 32; ++ks2) {
      pf[ks2][0] = pack2<T>(st[2 * ks2][0], st[2 * ks2][1]);
      pf[ks2][1] = pack2<T>(st[2 * ks2][2], st[2 * ks2][3]);
      pf[ks2][2] = pack2<T>(st[2 * ks2 + 1][0], st[2 * ks2 + 1][1]);
      pf[ks2][3] = pack2<T>(st[2 * ks2 + 1][2], st[2 * ks2 + 1][3]);
    }
    // O^T += V^T P^T: oacc[db][i] = O[q = qi][d = db*16 + 4g + i]
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int ks2 = 0; ks2 < BN / 32; ++ks2) {
        const uint16_t* row = &sv[(db * 16 + col) * VP + ks2 * 32 + 4 * g];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(row);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(row + 16);
        const u32x4 a = u32x4{lo[0], lo[1], hi[0], hi[1]};
        oacc[db] = mfma16x16x32<T>(a, pf[ks2], oacc[db]);
      }
    }
  }

  lsum += shfl_xor(lsum, 16);
  lsum += shfl_xor(lsum, 32);
  if (qi < p.q_len) {
    const float inv = 1.0f / lsum;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store_as(p.out, (size_t)qi * p.out_stride + (size_t)h * D + db * 16 + 4 * g + i, oacc[db][i] * inv,
                 p.out_dtype);
  }
}

// ---------------------------------------------------------------------------
// Generic kernel (any element type, D and Dv up to 256)
// ---------------------------------------------------------------------------

template <typename T>
__global__ void __launch_bounds__(64) prefill_generic_kernel(const PrefillParams p) {
  __shared__ float sq[256];
  __shared__ float sp[64];
  const int lane = threadIdx.x;
  const int qi = blockIdx.x;
  const int h = blockIdx.y;
  const int kvh = h / (p.num_heads / p.num_kv_heads);
  const int D = p.head_dim;
  const int Dv = p.head_dim_v;
  const T* qg = reinterpret_cast<const T*>(p.q) + (size_t)qi * p.q_stride + (size_t)h * D;
  const T* kg = reinterpret_cast<const T*>(p.k);
  const T* vg = reinterpret_cast<const T*>(p.v);
  for (int d = lane; d < D; d += 64) sq[d] = to_float<T>(qg[d]);
  __syncthreads();

  const float c = p.scale * kLog2e;
  const int kend = p.causal ? min(p.kv_len, qi + 1) : p.kv_len;
  float m = kNegInf, l = 0.0f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < kend; k0 += 64) {
    const int kidx = k0 + lane;
    float x = kNegInf;
    if (kidx < kend) {
      const T* kr = kg + (size_t)kidx * p.k_stride + (size_t)kvh * D;
      float dot = 0.0f;
      for (int d = 0; d < D; ++d) dot = fmaf(sq[d], to_float<T>(kr[d]), dot);
      x = dot * c;
    }
    const float mt = group_max<64>(x);
    const float mn = fmaxf(m, mt);
    const float mu = mn == kNegInf ? 0.0f : mn;
    const float alpha = fast_exp2(m - mu);
    m = mn;
    const float e = fast_exp2(x - mu);
    l = l * alpha + group_sum<64>(e);
    __syncthreads();
    sp[lane] = e;
    __syncthreads();
    const int n = min(64, kend - k0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int d = lane + 64 * t;
      if (d < Dv) {
        float a = acc[t] * alpha;
        for (int j = 0; j < n; ++j)
          a = fmaf(sp[j], to_float<T>(vg[(size_t)(k0 + j) * p.v_stride + (size_t)kvh * Dv + d]), a);
        acc[t] = a;
      }
    }
  }
  const float inv = 1.0f / l;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int d = lane + 64 * t;
    if (d < Dv) store_as(p.out, (size_t)qi * p.out_stride + (size_t)h * Dv + d, acc[t] * inv, p.out_dtype);
  }
}

// ---------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------

// Returns 0 on launch, 1 if the shape has no kernel.
int launch_flash_prefill(const PrefillParams& p, int dtype, bool allow_mfma, hipStream_t stream) {
  // 16-byte fragment loads: token strides and base addresses must be 16 B aligned.
  const bool aligned = p.q_stride % 8 == 0 && p.k_stride % 8 == 0 && p.v_stride % 8 == 0 &&
                       ((uintptr_t)p.q % 16) == 0 && ((uintptr_t)p.k % 16) == 0 && ((uintptr_t)p.v % 16) == 0;
  const bool mfma_ok = allow_mfma && (dtype == kF16 || dtype == kBF16) && p.head_dim == p.head_dim_v &&
                       (p.head_dim == 64 || p.head_dim == 128) && aligned;
  if (mfma_ok) {
    PrefillParams pp = p;
    pp.xcd_remap = (p.num_heads % 8 == 0) ? 1 : 0;
    const dim3 grid(p.num_heads, (p.q_len + 63) / 64);
    if (dtype == kF16) {
      if (p.head_dim == 64) hipLaunchKernelGGL((prefill_mfma_kernel<_Float16, 64>), grid, dim3(256), 0, stream, pp);
      else hipLaunchKernelGGL((prefill_mfma_kernel<_Float16, 128>), grid, dim3(256), 0, stream, pp);
    } else {
      if (p.head_dim == 64) hipLaunchKernelGGL((prefill_mfma_kernel<__bf16, 64>), grid, dim3(256), 0, stream, pp);
      else hipLaunchKernelGGL((prefill_mfma_kernel<__bf16, 128>), grid, dim3(256), 0, stream, pp);
    }
    return 0;
  }
  if (p.head_dim > 256 || p.head_dim_v > 256) return 1;
  const dim3 grid(p.q_len, p.num_heads);
  if (dtype == kF32) hipLaunchKernelGGL((prefill_generic_kernel<float>), grid, dim3(64), 0, stream, p);
  else if (dtype == kF16) hipLaunchKernelGGL((prefill_generic_kernel<_Float16>), grid, dim3(64), 0, stream, p);
  else hipLaunchKernelGGL((prefill_generic_kernel<__bf16>), grid, dim3(64), 0, stream, p);
  return 0;
}

}  // namespace tv
