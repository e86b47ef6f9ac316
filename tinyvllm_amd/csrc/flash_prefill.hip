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

#include <algorithm>

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
  return __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});
}
template <> __device__ __forceinline__ uint32_t pack2<__bf16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2{(__bf16)a, (__bf16)b});
}

// max over the four lanes l, l^16, l^32, l^48 (one query column of the S^T
// accumulator) with gfx950 row / half-wave swaps (VALU, no LDS round trip).
__device__ __forceinline__ float max_over_g(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x), false, false);
  x = fmaxf(u32_as_f32(a[0]), u32_as_f32(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x), false, false);
  return fmaxf(u32_as_f32(b[0]), u32_as_f32(b[1]));
}
__device__ __forceinline__ float sum_over_g(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x), false, false);
  x = u32_as_f32(a[0]) + u32_as_f32(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x), false, false);
  return u32_as_f32(b[0]) + u32_as_f32(b[1]);
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

constexpr int kPrefillBM = 64;   // query rows per work unit (16 per wave)
constexpr int kPrefillBN = 64;   // keys per tile

// Key tiles query tile qt needs (causal rows stop at the diagonal).
__device__ __forceinline__ int prefill_key_tiles(const PrefillParams& p, int qt) {
  const int kend = p.causal ? min(p.kv_len, (qt + 1) * kPrefillBM) : p.kv_len;
  return (kend + kPrefillBN - 1) / kPrefillBN;
}

// Map grid.y (longest work first) to (query tile, chunk of key tiles).
__device__ __forceinline__ void prefill_unit(const PrefillParams& p, int u, int& qt, int& chunk, int& nchunks) {
  const int nqt = (p.q_len + kPrefillBM - 1) / kPrefillBM;
  for (qt = nqt - 1; qt > 0; --qt) {
    const int ch = (prefill_key_tiles(p, qt) + p.chunk_tiles - 1) / p.chunk_tiles;
    if (u < ch) break;
    u -= ch;
  }
  nchunks = (prefill_key_tiles(p, qt) + p.chunk_tiles - 1) / p.chunk_tiles;
  chunk = u;
}

template <typename T, int D>
__global__ void __launch_bounds__(256) prefill_mfma_kernel(const PrefillParams p) {
  constexpr int BM = kPrefillBM;
  constexpr int BN = kPrefillBN;
  constexpr int KP = D + 8;       // LDS pitch of the K tile (elements)
  constexpr int VP = BN + 8;      // LDS pitch of the V^T tile (elements)
  constexpr int DB = D / 16;      // 16-row blocks of O^T
  constexpr int KS = D / 32;      // MFMA steps over the head dim
  constexpr int VPT = BN * (D / 8) / 256;   // 16-byte vectors of K (and of V) per thread per tile
  __shared__ __attribute__((aligned(16))) uint16_t sk[BN * KP];
  __shared__ __attribute__((aligned(16))) uint16_t sv[D * VP];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;        // 0..3
  const int col = lane & 15;

  const int h = prefill_head(blockIdx.x, p.num_heads, p.xcd_remap);
  int qt, chunk, nchunks;
  prefill_unit(p, blockIdx.y, qt, chunk, nchunks);
  const int kvh = h / (p.num_heads / p.num_kv_heads);
  const int qi = qt * BM + wave * 16 + col;
  const int nkt = prefill_key_tiles(p, qt);
  const int kt0 = chunk * p.chunk_tiles;
  const int kt1 = min(kt0 + p.chunk_tiles, nkt);

  const T* qg = reinterpret_cast<const T*>(p.q);
  const T* kg = reinterpret_cast<const T*>(p.k) + (size_t)kvh * D;
  const T* vg = reinterpret_cast<const T*>(p.v) + (size_t)kvh * D;

  u32x4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (qi < p.q_len)
      qf[ks] = *reinterpret_cast<const u32x4*>(qg + (size_t)qi * p.q_stride + (size_t)h * D + ks * 32 + g * 8);
    else
      qf[ks] = u32x4{0, 0, 0, 0};
  }

  // next tile's K and V, fetched into registers while the current tile computes
  u32x4 kpre[VPT], vpre[VPT];
  auto gload = [&](int kt) {
    const int k0 = kt * BN;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int idx = tid + i * 256;
      const int kk = idx / (D / 8);                  // K: consecutive lanes walk a row
      const int kc = idx - kk * (D / 8);
      kpre[i] = k0 + kk < p.kv_len
                    ? *reinterpret_cast<const u32x4*>(kg + (size_t)(k0 + kk) * p.k_stride + kc * 8)
                    : u32x4{0, 0, 0, 0};
      const int vk = idx % BN;                       // V: consecutive lanes walk keys
      const int vc = idx / BN;
      vpre[i] = k0 + vk < p.kv_len
                    ? *reinterpret_cast<const u32x4*>(vg + (size_t)(k0 + vk) * p.v_stride + vc * 8)
                    : u32x4{0, 0, 0, 0};
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int idx = tid + i * 256;
      const int kk = idx / (D / 8);
      const int kc = idx - kk * (D / 8);
      *reinterpret_cast<u32x4*>(&sk[kk * KP + kc * 8]) = kpre[i];
      const int vk = idx % BN;
      const int vc = idx / BN;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        sv[(vc * 8 + 2 * w) * VP + vk] = (uint16_t)(vpre[i][w] & 0xffffu);
        sv[(vc * 8 + 2 * w + 1) * VP + vk] = (uint16_t)(vpre[i][w] >> 16);
      }
    }
  };

  f32x4 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf;
  float lsum = 0.0f;
  const float c = p.scale * kLog2e;

  if (kt0 < kt1) gload(kt0);
  for (int kt = kt0; kt < kt1; ++kt) {
    const int k0 = kt * BN;
    __syncthreads();
    lstore();
    __syncthreads();
    if (kt + 1 < kt1) gload(kt + 1);

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

    // scale (log2 domain) and mask; tiles fully below the diagonal need no mask
    const bool full = k0 + BN <= p.kv_len && (!p.causal || k0 + BN - 1 <= qt * BM);
    float mt = kNegInf;
#pragma unroll
    for (int kb = 0; kb < BN / 16; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = st[kb][i] * c;
        if (!full) {
          const int kidx = k0 + kb * 16 + 4 * g + i;
          const bool ok = kidx < p.kv_len && (!p.causal || kidx <= qi);
          x = ok ? x : kNegInf;
        }
        st[kb][i] = x;
        mt = fmaxf(mt, x);
      }
    }
    mt = max_over_g(mt);
    // raise the running max only when it grows by more than the slack (rare
    // after the first tile); weights stay <= 2^8
    if (__builtin_amdgcn_ballot_w64(mt > m + 8.0f) != 0) {
      __asm__ volatile("" ::: "memory");
      const float mn = mt > m + 8.0f ? fmaxf(m, mt) : m;
      const float alpha = mn == kNegInf ? 1.0f : fast_exp2(m - mn);
      m = mn;
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
    }
    const float mu = m == kNegInf ? 0.0f : m;
#pragma unroll
    for (int kb = 0; kb < BN / 16; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = fast_exp2(st[kb][i] - mu);
        st[kb][i] = e;
        lsum += e;
      }

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

  lsum = sum_over_g(lsum);
  if (qi >= p.q_len) return;
  if (nchunks == 1) {
    const float inv = 1.0f / lsum;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store_as(p.out, (size_t)qi * p.out_stride + (size_t)h * D + db * 16 + 4 * g + i, oacc[db][i] * inv,
                 p.out_dtype);
    return;
  }
  // partial of this key chunk: normalised O plus (max, sum) per query row
  const int nqt = (p.q_len + BM - 1) / BM;
  const size_t unit = ((size_t)h * nqt + qt) * p.max_chunks + chunk;
  const int row = qi - qt * BM;
  float* po = p.part_o + (unit * BM + row) * D;
  const float inv = 1.0f / lsum;
#pragma unroll
  for (int db = 0; db < DB; ++db)
    *reinterpret_cast<f32x4*>(po + db * 16 + 4 * g) = oacc[db] * inv;
  if (g == 0) {
    p.part_ml[(unit * BM + row) * 2] = m;
    p.part_ml[(unit * BM + row) * 2 + 1] = lsum;
  }
}

// Merge the key-chunk partials of query tiles that were split.  grid (Hq, nqt).
template <int D>
__global__ void __launch_bounds__(256) prefill_merge_kernel(const PrefillParams p) {
  constexpr int BM = kPrefillBM;
  const int h = blockIdx.x;
  const int qt = blockIdx.y;
  const int nchunks = (prefill_key_tiles(p, qt) + p.chunk_tiles - 1) / p.chunk_tiles;
  if (nchunks <= 1) return;
  const int nqt = (p.q_len + BM - 1) / BM;
  const size_t unit0 = ((size_t)h * nqt + qt) * p.max_chunks;
  for (int idx = threadIdx.x; idx < BM * D; idx += 256) {
    const int row = idx / D;
    const int d = idx - row * D;
    const int qi = qt * BM + row;
    if (qi >= p.q_len) break;
    float M = kNegInf;
    for (int ch = 0; ch < nchunks; ++ch) M = fmaxf(M, p.part_ml[((unit0 + ch) * BM + row) * 2]);
    const float Mu = M == kNegInf ? 0.0f : M;
    float num = 0.0f, den = 0.0f;
    for (int ch = 0; ch < nchunks; ++ch) {
      const size_t r = (unit0 + ch) * BM + row;
      const float w = p.part_ml[r * 2 + 1] * fast_exp2(p.part_ml[r * 2] - Mu);
      num = fmaf(w, p.part_o[r * D + d], num);
      den += w;
    }
    store_as(p.out, (size_t)qi * p.out_stride + (size_t)h * D + d, num / den, p.out_dtype);
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

// Work units per head and the largest number of key chunks of one query tile
// (host-side mirror of prefill_key_tiles / prefill_unit).
void prefill_units(const PrefillParams& p, int& units, int& max_chunks) {
  const int nqt = (p.q_len + kPrefillBM - 1) / kPrefillBM;
  units = 0;
  max_chunks = 1;
  for (int qt = 0; qt < nqt; ++qt) {
    const int kend = p.causal ? std::min(p.kv_len, (qt + 1) * kPrefillBM) : p.kv_len;
    const int nkt = (kend + kPrefillBN - 1) / kPrefillBN;
    const int ch = (nkt + p.chunk_tiles - 1) / p.chunk_tiles;
    units += ch;
    max_chunks = std::max(max_chunks, ch);
  }
}

bool prefill_uses_mfma(const PrefillParams& p, int dtype) {
  // 16-byte fragment loads: token strides and base addresses must be 16 B aligned.
  const bool aligned = p.q_stride % 8 == 0 && p.k_stride % 8 == 0 && p.v_stride % 8 == 0 &&
                       ((uintptr_t)p.q % 16) == 0 && ((uintptr_t)p.k % 16) == 0 && ((uintptr_t)p.v % 16) == 0;
  return (dtype == kF16 || dtype == kBF16) && p.head_dim == p.head_dim_v &&
         (p.head_dim == 64 || p.head_dim == 128) && aligned;
}

size_t prefill_workspace_bytes(const PrefillParams& p, int dtype) {
  if (!prefill_uses_mfma(p, dtype)) return 0;
  int units, max_chunks;
  prefill_units(p, units, max_chunks);
  if (max_chunks <= 1) return 0;
  const size_t nqt = (p.q_len + kPrefillBM - 1) / kPrefillBM;
  return (size_t)p.num_heads * nqt * max_chunks * kPrefillBM * (p.head_dim + 2) * sizeof(float);
}

// Returns 0 on launch, 1 if the shape has no kernel, 2 if the workspace is missing.
int launch_flash_prefill(const PrefillParams& p_in, int dtype, void* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  if (prefill_uses_mfma(p_in, dtype)) {
    PrefillParams pp = p_in;
    pp.xcd_remap = (pp.num_heads % 8 == 0) ? 1 : 0;
    int units, max_chunks;
    prefill_units(pp, units, max_chunks);
    pp.max_chunks = max_chunks;
    if (max_chunks > 1) {
      const size_t need = prefill_workspace_bytes(pp, dtype);
      if (!workspace || workspace_bytes < need) return 2;
      const size_t nqt = (pp.q_len + kPrefillBM - 1) / kPrefillBM;
      pp.part_o = reinterpret_cast<float*>(workspace);
      pp.part_ml = pp.part_o + (size_t)pp.num_heads * nqt * max_chunks * kPrefillBM * pp.head_dim;
    }
    const dim3 grid(pp.num_heads, units);
    const bool d64 = pp.head_dim == 64;
    if (dtype == kF16) {
      if (d64) hipLaunchKernelGGL((prefill_mfma_kernel<_Float16, 64>), grid, dim3(256), 0, stream, pp);
      else hipLaunchKernelGGL((prefill_mfma_kernel<_Float16, 128>), grid, dim3(256), 0, stream, pp);
    } else {
      if (d64) hipLaunchKernelGGL((prefill_mfma_kernel<__bf16, 64>), grid, dim3(256), 0, stream, pp);
      else hipLaunchKernelGGL((prefill_mfma_kernel<__bf16, 128>), grid, dim3(256), 0, stream, pp);
    }
    if (max_chunks > 1) {
      const dim3 mgrid(pp.num_heads, (pp.q_len + kPrefillBM - 1) / kPrefillBM);
      if (d64) hipLaunchKernelGGL((prefill_merge_kernel<64>), mgrid, dim3(256), 0, stream, pp);
      else hipLaunchKernelGGL((prefill_merge_kernel<128>), mgrid, dim3(256), 0, stream, pp);
    }
    return 0;
  }
  if (p_in.head_dim > 256 || p_in.head_dim_v > 256) return 1;
  const dim3 grid(p_in.q_len, p_in.num_heads);
  if (dtype == kF32) hipLaunchKernelGGL((prefill_generic_kernel<float>), grid, dim3(64), 0, stream, p_in);
  else if (dtype == kF16) hipLaunchKernelGGL((prefill_generic_kernel<_Float16>), grid, dim3(64), 0, stream, p_in);
  else hipLaunchKernelGGL((prefill_generic_kernel<__bf16>), grid, dim3(64), 0, stream, p_in);
  return 0;
}

}  // namespace tv
