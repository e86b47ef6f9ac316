// Paged-decode attention for gfx950: one query token per sequence against a
// block-paged K/V cache [num_blocks, block_size, Hkv, D].
//
// Work decomposition
//   grid.x = context partition, grid.y = (KV head, query-head chunk), grid.z = sequence.
//   A work-group of NW waves handles one KV head for GT query heads of its GQA
//   group, so every K/V row fetched from HBM is used by GT query heads.
//   Waves take interleaved tiles of TT tokens inside the partition.
//
// Lane layout inside a wave
//   A cache row (one token, one KV head) is D*sizeof(T) bytes.  LPR lanes cover
//   one row with 16-byte loads (VPL vectors each), so one load instruction
//   fetches RPI = 64/LPR rows; each lane holds NR rows of the tile.  The q.k
//   partial sums are combined across the LPR lanes of a row with DPP; lanes of
//   one row form a "group" that runs its own online softmax (running max m,
//   running sum l, unnormalised accumulator acc) in the log2 domain.
//   Groups and waves are merged once at the end (shuffles, then LDS).
//
// Semantics follow tinyvllm/model/llama.py:97-144: scores are (q.k)*scale,
// positions >= context_len are excluded (the reference adds -1e9, which
// underflows to an exact zero weight), query head h reads KV head h / (Hq/Hkv).
// A context length <= 0 reproduces the reference's all-masked case: every
// gathered position is used with score (q.k)*scale - 1e9 rounded in fp32.
// A block id outside [0, num_blocks) is never dereferenced; the affected
// (sequence, head) outputs are NaN.
#pragma once

#include "tv_common.h"

namespace tv {

struct DecodeParams {
  void* out;                 // [B, Hq, D] in out_dtype
  float* part_o;             // [B, Hq, max_parts, D] normalised partition outputs
  float* part_ml;            // [B, Hq, max_parts, 2] (max in log2 units, sum)
  const void* q;             // [B, Hq, D]
  const void* k_cache;       // [NB, bs, Hkv, D]
  const void* v_cache;       // [NB, bs, Hkv, D]
  const int* block_tables;   // [B, bt_stride]
  const int* context_lens;   // [B]
  int num_heads;
  int num_kv_heads;
  int head_chunks;           // (Hq/Hkv) / GT
  int block_size;
  int bs_log2;               // log2(block_size) or -1
  int num_blocks;
  int bt_stride;
  int max_blocks;            // table columns used (<= bt_stride)
  float scale;
  int partition_size;        // tokens per work-group
  int max_parts;             // ceil(max_blocks*block_size / partition_size)
  int out_dtype;
};

__device__ __forceinline__ int decode_len(const DecodeParams& p, int b, float& bias) {
  const int width = p.max_blocks * p.block_size;
  const int ctx = p.context_lens[b];
  bias = ctx <= 0 ? -1e9f : 0.0f;
  return ctx <= 0 ? width : (ctx < width ? ctx : width);
}

template <typename T, int D, int GT, int NW>
__global__ void __launch_bounds__(64 * NW) paged_decode_kernel(const DecodeParams p) {
  constexpr int ROW_BYTES = D * (int)sizeof(T);
  constexpr int LPR = ROW_BYTES / 16 < 16 ? ROW_BYTES / 16 : 16;
  constexpr int VPL = ROW_BYTES / (16 * LPR);
  constexpr int RPI = 64 / LPR;
  constexpr int NR = RPI >= 16 ? 1 : 16 / RPI;
  constexpr int TT = RPI * NR;
  constexpr int EPV = 16 / (int)sizeof(T);
  constexpr int EPL = VPL * EPV;
  static_assert(LPR >= 1 && VPL >= 1 && LPR * VPL * 16 == ROW_BYTES, "unsupported row size");

  __shared__ float sh_acc[NW][GT][D];
  __shared__ float sh_m[NW][GT];
  __shared__ float sh_l[NW][GT];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane / LPR;
  const int c = lane % LPR;
  const int part = blockIdx.x;
  const int b = blockIdx.z;
  const int kh = blockIdx.y / p.head_chunks;
  const int group = p.num_heads / p.num_kv_heads;
  const int h0 = kh * group + (blockIdx.y % p.head_chunks) * GT;

  float bias;
  const int len = decode_len(p, b, bias);
  const int nparts = (len + p.partition_size - 1) / p.partition_size;
  if (part >= nparts) return;
  const int start = part * p.partition_size;
  const int end = min(start + p.partition_size, len);

  const T* qp = reinterpret_cast<const T*>(p.q) + ((size_t)b * p.num_heads + h0) * D;
  const T* kc = reinterpret_cast<const T*>(p.k_cache);
  const T* vc = reinterpret_cast<const T*>(p.v_cache);
  const int* bt = p.block_tables + (size_t)b * p.bt_stride;

  u32x4 qv[GT][VPL];
#pragma unroll
  for (int g = 0; g < GT; ++g)
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      qv[g][v] = *reinterpret_cast<const u32x4*>(qp + g * D + (v * LPR + c) * EPV);

  float m[GT], l[GT], acc[GT][EPL];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    m[g] = kNegInf;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.0f;
  }
  bool bad = false;
  const float scale = p.scale;

  for (int t0 = start + wave * TT; t0 < end; t0 += NW * TT) {
    u32x4 kr[NR][VPL], vr[NR][VPL];
    bool valid[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const int pos = t0 + j * RPI + r;
      valid[j] = pos < end;
      size_t base = 0;
      if (valid[j]) {
        const int bi = p.bs_log2 >= 0 ? (pos >> p.bs_log2) : pos / p.block_size;
        const int off = pos - bi * p.block_size;
        const int blk = bt[bi];
        if ((unsigned)blk >= (unsigned)p.num_blocks) {
          bad = true;
          valid[j] = false;
        } else {
          base = (((size_t)blk * p.block_size + off) * p.num_kv_heads + kh) * D;
        }
      }
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        if (valid[j]) {
          kr[j][v] = *reinterpret_cast<const u32x4*>(kc + base + (v * LPR + c) * EPV);
          vr[j][v] = *reinterpret_cast<const u32x4*>(vc + base + (v * LPR + c) * EPV);
        } else {
          kr[j][v] = u32x4{0, 0, 0, 0};
          vr[j][v] = u32x4{0, 0, 0, 0};
        }
      }
    }

    // scores (log2 domain) for NR rows x GT heads
    float s[NR][GT];
#pragma unroll
    for (int j = 0; j < NR; ++j) {
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        float d = 0.0f;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            if constexpr (sizeof(T) == 4) {
              d = fmaf(u32_as_f32(qv[g][v][w]), u32_as_f32(kr[j][v][w]), d);
            } else {
              d = dot2<T>(qv[g][v][w], kr[j][v][w], d);
            }
          }
        }
        d = group_sum<LPR>(d);
        s[j][g] = valid[j] ? fmaf(d, scale, bias) * kLog2e : kNegInf;
      }
    }

    // online softmax update per head
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      float mt = s[0][g];
#pragma unroll
      for (int j = 1; j < NR; ++j) mt = fmaxf(mt, s[j][g]);
      const float mn = fmaxf(m[g], mt);
      const float mu = mn == kNegInf ? 0.0f : mn;
      const float alpha = fast_exp2(m[g] - mu);
      m[g] = mn;
      float ls = l[g] * alpha;
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        s[j][g] = fast_exp2(s[j][g] - mu);
        ls += s[j][g];
      }
      l[g] = ls;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
    }

    // acc += p * v
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      float vf[EPL];
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          if constexpr (sizeof(T) == 4) {
            vf[v * EPV + w] = u32_as_f32(vr[j][v][w]);
          } else {
            unpack2<T>(vr[j][v][w], vf[v * EPV + 2 * w], vf[v * EPV + 2 * w + 1]);
          }
        }
      }
#pragma unroll
      for (int g = 0; g < GT; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(s[j][g], vf[e], acc[g][e]);
    }
  }

  // merge the RPI row groups of this wave (lanes with equal c)
#pragma unroll
  for (int msk = LPR; msk < 64; msk <<= 1) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      const float mo = shfl_xor(m[g], msk);
      const float lo = shfl_xor(l[g], msk);
      const float mn = fmaxf(m[g], mo);
      const float mu = mn == kNegInf ? 0.0f : mn;
      const float fa = fast_exp2(m[g] - mu);
      const float fb = fast_exp2(mo - mu);
      l[g] = l[g] * fa + lo * fb;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float ao = shfl_xor(acc[g][e], msk);
        acc[g][e] = acc[g][e] * fa + ao * fb;
      }
      m[g] = mn;
    }
  }

  if (lane < LPR) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
#pragma unroll
      for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int e = 0; e < EPV; ++e) sh_acc[wave][g][(v * LPR + c) * EPV + e] = acc[g][v * EPV + e];
      if (c == 0) {
        sh_m[wave][g] = m[g];
        sh_l[wave][g] = l[g];
      }
    }
  }
  const bool any_bad = __syncthreads_or(bad ? 1 : 0) != 0;

  const int hq = p.num_heads;
  for (int idx = tid; idx < GT * D; idx += 64 * NW) {
    const int g = idx / D;
    const int d = idx - g * D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sh_m[w][g]);
    const float Mu = M == kNegInf ? 0.0f : M;
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = fast_exp2(sh_m[w][g] - Mu);
      L += sh_l[w][g] * f;
      O += sh_acc[w][g][d] * f;
    }
    const int h = h0 + g;
    if (nparts == 1) {
      const float val = any_bad ? __builtin_nanf("") : O / L;
      store_as(p.out, ((size_t)b * hq + h) * D + d, val, p.out_dtype);
    } else {
      const size_t slot = ((size_t)b * hq + h) * p.max_parts + part;
      p.part_o[slot * D + d] = O / L;
      if (d == 0) {
        p.part_ml[slot * 2] = any_bad ? __builtin_nanf("") : M;
        p.part_ml[slot * 2 + 1] = L;
      }
    }
  }
}

// Merge the partition partials of each (sequence, query head).  Launched with
// grid (Hq, B) and 64 threads; sequences that fit one partition were written by
// the main kernel and are skipped here.
__global__ void __launch_bounds__(64) paged_decode_reduce_kernel(const DecodeParams p, int head_dim);

}  // namespace tv
