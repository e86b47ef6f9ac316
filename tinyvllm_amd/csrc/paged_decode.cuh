// Paged-decode attention for gfx950: one query token per sequence against a
// block-paged K/V cache [num_blocks, block_size, Hkv, D].
//
// Work decomposition
//   A work-group of NW waves attends one sequence for one KV head -- or two
//   adjacent KV heads (hpw = 2) -- each for GT query heads of its GQA group, so
//   every K/V row fetched from HBM is used by GT query heads.  Wave w serves
//   head w % hpw; the NW / hpw waves of a head take interleaved tiles of TT
//   tokens, and with two heads the waves read the same tokens together (2 D
//   contiguous elements of each cache row [token, Hkv, D]).
//   paged_decode_kernel: grid (context partition, KV head x query-head chunk,
//   sequence), one KV head per work-group; partitions of a split context
//   leave partials for paged_decode_reduce_kernel.
//   paged_decode_scheduled_kernel: 1-D grid over (sequence, row) items in the
//   longest-first order of decode_order_kernel, which also picks hpw.

// Lane layout inside a wave
//   A cache row (one token, one KV head) is D*sizeof(T) bytes.  LPR lanes cover
//   one row with 16-byte loads (VPL vectors each), so one load instruction
//   fetches RPI = 64/LPR rows; each lane holds NR rows of the tile.  The q.k
//   partial sums are combined across the LPR lanes of a row with DPP; lanes of
//   one row form a "group" that runs its own online softmax (running max m,
//   running sum l, unnormalised accumulator acc) in the log2 domain.
//   Groups and waves are merged once at the end (DPP / swizzle, then LDS).
//   Split-context partials (m, l, o) go to the caller's workspace and a second
//   kernel merges them (flash-decoding).
//   When a cache block holds whole tiles (block_size % 16 == 0) each tile needs
//   a single wave-uniform block-table lookup, and its rows are read through a
//   buffer resource whose range ends at the tile's last attended row.
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

// Shape constants, measured on MI355X: at most 64 fp32 accumulators per lane
// (sets the lanes per cache row), 16-token tiles, and the VGPR budget sized for
// one work-group per CU.
constexpr int kDecodeAccMax = 64;
constexpr int kDecodeMinBlocks = 1;

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
  const int* sched;          // scheduled launch: [0] KV heads per row, [1..B] longest-first order
  int num_seqs;
};

__device__ __forceinline__ int decode_len(const DecodeParams& p, int b, float& bias) {
  const int width = p.max_blocks * p.block_size;
  const int ctx = p.context_lens[b];
  bias = ctx <= 0 ? -1e9f : 0.0f;
  return ctx <= 0 ? width : (ctx < width ? ctx : width);
}

// Compile-time lane layout of the decode kernel for element type T, head_dim D
// and GT query heads per work-group.
//   LPR  lanes per cache row; chosen so each lane keeps at most 64 fp32
//        accumulators (GT * D / LPR <= 64), capped at 16 (one DPP row) and at
//        one 16-byte vector per lane.
//   VPL  16-byte vectors per lane per row (lane c holds vectors c, c+LPR, ...,
//        so every load instruction covers LPR*16 contiguous bytes of a row).
//   RPI  rows fetched by one load instruction; NR rows per lane per tile;
//        TT = RPI*NR tokens per wave-tile (16 unless a row needs < 4 lanes).
template <typename T, int D, int GT>
struct DecodeShape {
  static constexpr int ROW_BYTES = D * (int)sizeof(T);
  static constexpr int MAXL = ROW_BYTES / 16 < 16 ? ROW_BYTES / 16 : 16;
  static constexpr int WANT = D * GT / kDecodeAccMax < 1 ? 1 : D * GT / kDecodeAccMax;
  static constexpr int LPR = WANT < MAXL ? WANT : MAXL;
  static constexpr int VPL = ROW_BYTES / (16 * LPR);
  static constexpr int RPI = 64 / LPR;
  static constexpr int NR = RPI >= 16 ? 1 : 16 / RPI;
  static constexpr int TT = RPI * NR;
  static constexpr int EPV = 16 / (int)sizeof(T);
  static constexpr int EPL = VPL * EPV;
  static_assert(LPR >= 1 && VPL >= 1 && LPR * VPL * 16 == ROW_BYTES, "unsupported row size");
};

// 16-byte cache-row load; K/V rows are read exactly once per launch, so they
// bypass cache retention (non-temporal).
__device__ __forceinline__ u32x4 load_row16(const void* ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ptr));
}

__device__ __forceinline__ u32x4 buffer_load_nt16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2));
}

// Whether every TT-token tile of a launch lies in one cache block (one
// wave-uniform table lookup per tile, buffer loads from the tile's first row).
template <typename T, int D, int GT>
inline bool decode_uniform_tiles(int block_size, int partition_size, int num_kv_heads) {
  constexpr int TT = DecodeShape<T, D, GT>::TT;
  const bool pow2 = block_size > 0 && (block_size & (block_size - 1)) == 0;
  return pow2 && block_size % TT == 0 && partition_size % TT == 0 &&
         (long long)TT * num_kv_heads * D * (long long)sizeof(T) < (1LL << 31);
}

// VGPRs per lane of two tiles in flight (K and V rows), the accumulators and
// the query vectors of the decode kernel's shape: the part of its register
// budget that grows when a second tile is requested ahead.
template <typename T, int D, int GT>
constexpr int kDecodePipeRegs = 2 * (2 * DecodeShape<T, D, GT>::NR * DecodeShape<T, D, GT>::VPL * 4) +
                                GT * DecodeShape<T, D, GT>::EPL + GT * DecodeShape<T, D, GT>::VPL * 4;

// Running maxima are only raised when a tile's maximum exceeds them by more
// than this many log2 units, so most tiles skip the rescale of l and acc; the
// unnormalised weights stay <= 2^kRescaleSlack, far from fp32 overflow.
constexpr float kRescaleSlack = 8.0f;

template <int CTRL, int N> __device__ __forceinline__ void dpp_add_arr(float (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp<CTRL>(x[i]);
}

// All-reduce sum over aligned groups of G lanes (G <= 16) for N independent
// values; the steps are interleaved across the values so no DPP hazard stalls.
template <int G, int N> __device__ __forceinline__ void group_sum_arr(float (&x)[N]) {
  if constexpr (G >= 2) dpp_add_arr<kDppXor1>(x);
  if constexpr (G >= 4) dpp_add_arr<kDppXor2>(x);
  if constexpr (G >= 8) dpp_add_arr<kDppHalfMirror>(x);
  if constexpr (G >= 16) dpp_add_arr<kDppMirror>(x);
}

// Sum over the lanes of each 16-lane row that share lane % G (G <= 16 a power
// of two), using row rotations; every lane receives its class total.
template <int G> __device__ __forceinline__ float row_class_sum(float x) {
  if constexpr (G <= 1) x += dpp<0x121>(x);   // row_ror:1
  if constexpr (G <= 2) x += dpp<0x122>(x);   // row_ror:2
  if constexpr (G <= 4) x += dpp<0x124>(x);   // row_ror:4
  if constexpr (G <= 8) x += dpp<0x128>(x);   // row_ror:8
  return x;
}

// Maximum over the lanes of each 16-lane row that share lane % G, as above.
template <int G> __device__ __forceinline__ float row_class_max(float x) {
  if constexpr (G <= 1) x = fmaxf(x, dpp<0x121>(x));
  if constexpr (G <= 2) x = fmaxf(x, dpp<0x122>(x));
  if constexpr (G <= 4) x = fmaxf(x, dpp<0x124>(x));
  if constexpr (G <= 8) x = fmaxf(x, dpp<0x128>(x));
  return x;
}

__device__ __forceinline__ float swizzle_xor16(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401F));
}

// Shared memory of one decode work-group: per wave and 32-lane half the
// unnormalised accumulators and sums of its GT query heads, per wave the maxima.
template <int D, int GT, int NW>
struct DecodeSmem {
  float acc[NW][2][GT][D];
  float l[NW][2][GT];
  float m[NW][GT];
};

// Where one pass over a token range leaves its result: the final output
// out[b, h, :], or a partial -- output normalised by its own sum, running
// maximum (log2 units) and sum -- at slot slot0 + (h - first query head of the
// work-group) * slot_step of part_o [*, D] / part_ml [*, 2].
struct DecodeDest {
  bool final_out;
  size_t slot0;
  int slot_step;
};

// First query head served by work-group row ky with hpw KV heads per work-group.
template <int GT>
__device__ __forceinline__ int decode_first_head(const DecodeParams& p, int ky, int hpw) {
  const int group = p.num_heads / p.num_kv_heads;
  return (ky / p.head_chunks) * hpw * group + (ky % p.head_chunks) * GT;
}

// Attention of work-group row ky's query heads over tokens [start, end) of
// sequence b (start < end), with hpw (1, or HPW when HPW > 1) KV heads per
// work-group.  Wave w serves KV head (ky / head_chunks) * hpw + w % hpw with
// the GT query heads (ky % head_chunks) * GT .. of its GQA group;
// bias is the reference's additive mask term (-1e9 when context_len <= 0).
// Ends with the merged result written to dst.  Uses sm from its merge step on:
// a caller that runs several ranges in one work-group separates them with a
// barrier.
template <typename T, int D, int GT, int NW, int HPW, bool UB>
__device__ __forceinline__ void decode_range(const DecodeParams& p, DecodeSmem<D, GT, NW>& sm, int b, int ky,
                                             int hpw_in, int start, int end, float bias,
                                             const DecodeDest& dst) {
  using S = DecodeShape<T, D, GT>;
  constexpr int LPR = S::LPR, VPL = S::VPL, RPI = S::RPI, NR = S::NR, TT = S::TT;
  constexpr int EPV = S::EPV, EPL = S::EPL;
  static_assert(HPW == 1 || HPW == 2, "one or two KV heads per work-group");
  const int hpw = HPW == 1 ? 1 : hpw_in;
  const int wph = NW / hpw;       // waves per KV head

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane / LPR;
  const int c = lane % LPR;
  const int hw = wave & (hpw - 1);   // head of this work-group served by the wave
  const int wi = wave / hpw;         // the wave's index among that head's waves
  const int kh = (ky / p.head_chunks) * hpw + hw;
  const int group = p.num_heads / p.num_kv_heads;
  const int hfirst = decode_first_head<GT>(p, ky, hpw);
  const int h0 = hfirst + hw * group;   // first query head of this wave

  const T* qp = reinterpret_cast<const T*>(p.q) + ((size_t)b * p.num_heads + h0) * D;
  const T* kc = reinterpret_cast<const T*>(p.k_cache) + (size_t)kh * D;
  const T* vc = reinterpret_cast<const T*>(p.v_cache) + (size_t)kh * D;
  const int* bt = p.block_tables + (size_t)b * p.bt_stride;
  const size_t row_stride = (size_t)p.num_kv_heads * D;          // elements between cache rows
  const int lane_off = (int)((r * row_stride + c * EPV) * sizeof(T));   // bytes from a tile's first row

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
  const float sc = p.scale * kLog2e;
  const float bi2 = bias * kLog2e;

  // Uniform tiles (UB): the K/V rows of the tile starting at token t0, which
  // lies in cache block blk (rows past `end` or in an invalid block are zero
  // and marked invalid; with live false the tile has no rows and consumes as
  // nothing).
  auto fetch_block = [&](int t0, int blk, u32x4 (&kr)[NR][VPL], u32x4 (&vr)[NR][VPL], bool (&valid)[NR],
                         bool live) {
    const bool blk_ok = (unsigned)blk < (unsigned)p.num_blocks;
    bad |= live && !blk_ok;
    const int rows = blk_ok && live ? min(TT, end - t0) : 0;
    const size_t row0 = (size_t)(blk_ok ? blk : 0) * p.block_size + (t0 & (p.block_size - 1));
    const unsigned long long nrec = (unsigned long long)rows * row_stride * sizeof(T);
    const auto kres = make_rsrc(kc + row0 * row_stride, nrec);
    const auto vres = make_rsrc(vc + row0 * row_stride, nrec);
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      valid[j] = j * RPI + r < rows;
      const int off = lane_off + j * RPI * (int)(row_stride * sizeof(T));
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        kr[j][v] = buffer_load_nt16(kres, off + v * LPR * 16, 0);
        vr[j][v] = buffer_load_nt16(vres, off + v * LPR * 16, 0);
      }
    }
  };
  auto fetch = [&](int t0, u32x4 (&kr)[NR][VPL], u32x4 (&vr)[NR][VPL], bool (&valid)[NR]) {
    if constexpr (UB) {
      // The whole tile lies in one cache block: one wave-uniform table lookup,
      // then buffer loads from the tile's first row.  The buffer's range ends
      // at the last attended row of the tile (nothing when the block id is
      // invalid), so rows past it read as zero without per-row branches, and
      // the lane offsets are the same for every tile.
      fetch_block(t0, bt[t0 >> p.bs_log2], kr, vr, valid, true);
    } else {
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
            base = ((size_t)blk * p.block_size + off) * row_stride;
          }
        }
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          if (valid[j]) {
            kr[j][v] = load_row16(kc + base + (v * LPR + c) * EPV);
            vr[j][v] = load_row16(vc + base + (v * LPR + c) * EPV);
          } else {
            kr[j][v] = u32x4{0, 0, 0, 0};
            vr[j][v] = u32x4{0, 0, 0, 0};
          }
        }
      }
    }

  };

  // Scores, online-softmax update and P.V accumulation for one fetched tile.
  auto consume = [&](u32x4 (&kr)[NR][VPL], u32x4 (&vr)[NR][VPL], bool (&valid)[NR]) {
    // partial q.k over this lane's slice, then all-reduce over the LPR lanes of the row
    float s[NR * GT];
#pragma unroll
    for (int j = 0; j < NR; ++j) {
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        float d = 0.0f;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          const u32x4 qg = qv[g][v];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            if constexpr (sizeof(T) == 4) {
              d = fmaf(u32_as_f32(qg[w]), u32_as_f32(kr[j][v][w]), d);
            } else {
              d = dot2<T>(qg[w], kr[j][v][w], d);
            }
          }
        }
        s[j * GT + g] = d;
      }
    }
    group_sum_arr<LPR>(s);
#pragma unroll
    for (int j = 0; j < NR; ++j)
#pragma unroll
      for (int g = 0; g < GT; ++g)
        s[j * GT + g] = valid[j] ? fmaf(s[j * GT + g], sc, bi2) : kNegInf;

    // raise the running maxima only when a tile exceeds them by the slack
    float mt[GT];
    bool raise = false;
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      mt[g] = s[g];
#pragma unroll
      for (int j = 1; j < NR; ++j) mt[g] = fmaxf(mt[g], s[j * GT + g]);
      raise |= mt[g] > m[g] + kRescaleSlack;
    }
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {
      // opaque to the optimiser: keeps this rarely taken block a real branch
      // instead of an if-converted multiply of every accumulator per tile
      __asm__ volatile("" ::: "memory");
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        const float mn = mt[g] > m[g] + kRescaleSlack ? fmaxf(m[g], mt[g]) : m[g];
        const float alpha = mn == kNegInf ? 1.0f : fast_exp2(m[g] - mn);
        m[g] = mn;
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
      }
    }
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      const float mu = m[g] == kNegInf ? 0.0f : m[g];
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const float pj = fast_exp2(s[j * GT + g] - mu);
        s[j * GT + g] = pj;
        l[g] += pj;
      }
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
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(s[j * GT + g], vf[e], acc[g][e]);
    }
  };

  // 8-wave work-groups (small launches, where dependent round trips set the
  // time) whose waves have at most two tiles: both tiles' block ids are
  // requested together and both tiles' rows before either is consumed (one
  // round trip for the table and one for the rows instead of two each; the
  // second tile of a one-tile wave is a dead re-read of the first).  Only
  // shapes whose two tiles in flight fit beside the accumulators (no spills
  // at 256 VGPRs, checked in the compiled code).
  const int first = start + wi * TT, stride = wph * TT;
  bool done = false;
  if constexpr (NW >= 8 && UB && kDecodePipeRegs<T, D, GT> <= 192) {
    const int n = first < end ? (end - first + stride - 1) / stride : 0;
    if (n == 1 || n == 2) {
      const int t1 = first + (n - 1) * stride;
      const int blk0 = bt[first >> p.bs_log2];
      const int blk1 = bt[t1 >> p.bs_log2];
      u32x4 kr0[NR][VPL], vr0[NR][VPL], kr1[NR][VPL], vr1[NR][VPL];
      bool valid0[NR], valid1[NR];
      fetch_block(first, blk0, kr0, vr0, valid0, true);
      fetch_block(t1, blk1, kr1, vr1, valid1, n == 2);
      consume(kr0, vr0, valid0);
      consume(kr1, vr1, valid1);
      done = true;
    }
  }
  if (!done) {
    for (int t0 = first; t0 < end; t0 += stride) {
      u32x4 kr[NR][VPL], vr[NR][VPL];
      bool valid[NR];
      fetch(t0, kr, vr, valid);
      consume(kr, vr, valid);
    }
  }

  // ---- merge row groups and waves ------------------------------------------
  // 1) common maximum per head across the wave; rescale each group onto it
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    // over the row groups of a 16-lane row (DPP), then across rows and halves
    // (permlane swaps), on the VALU: 7.46 -> 7.14 us at TinyLlama fp32 B4
    // against three dependent ds_bpermute per head.  (The sums below stay on
    // ds_swizzle: on the VALU too they measured 7.63 us, the VALU being the
    // busy unit of that launch.)
    float mw = m[g];
    if constexpr (LPR < 16) mw = row_class_max<LPR>(mw);
    mw = max_over_g(mw);
    const float f = mw == kNegInf ? 0.0f : fast_exp2(m[g] - mw);
    l[g] *= f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] *= f;
    m[g] = mw;
  }
  // 2) sum the groups of each 16-lane row (lanes with equal c), then the two
  //    rows of each 32-lane half
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    if constexpr (LPR < 16) l[g] = row_class_sum<LPR>(l[g]);
    l[g] += swizzle_xor16(l[g]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      if constexpr (LPR < 16) acc[g][e] = row_class_sum<LPR>(acc[g][e]);
      acc[g][e] += swizzle_xor16(acc[g][e]);
    }
  }
  // 3) lanes 0..LPR-1 and 32..32+LPR-1 publish their half's partial sums
  const int half = lane >> 5;
  if ((lane & 31) < LPR) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
#pragma unroll
      for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int e = 0; e < EPV; ++e) sm.acc[wave][half][g][(v * LPR + c) * EPV + e] = acc[g][v * EPV + e];
      if (c == 0) {
        sm.l[wave][half][g] = l[g];
        if (half == 0) sm.m[wave][g] = m[g];
      }
    }
  }
  const bool any_bad = __syncthreads_or(bad ? 1 : 0) != 0;

  const int hq = p.num_heads;
  for (int idx = tid; idx < hpw * GT * D; idx += 64 * NW) {
    const int oh = idx / (GT * D);      // head of the work-group; its waves are oh, oh + hpw, ...
    const int g = (idx / D) % GT;
    const int d = idx % D;
    float M = kNegInf;
#pragma unroll
    for (int k = 0; k < NW; ++k)
      if (k < wph) M = fmaxf(M, sm.m[oh + k * hpw][g]);
    const float Mu = M == kNegInf ? 0.0f : M;
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      if (k >= wph) break;
      const int w = oh + k * hpw;
      const float f = fast_exp2(sm.m[w][g] - Mu);
      L += (sm.l[w][0][g] + sm.l[w][1][g]) * f;
      O += (sm.acc[w][0][g][d] + sm.acc[w][1][g][d]) * f;
    }
    const int h = hfirst + oh * group + g;
    if (dst.final_out) {
      const float val = any_bad ? __builtin_nanf("") : O / L;
      store_as(p.out, ((size_t)b * hq + h) * D + d, val, p.out_dtype);
    } else {
      const size_t slot = dst.slot0 + (size_t)(h - hfirst) * dst.slot_step;
      p.part_o[slot * D + d] = O / L;
      if (d == 0) {
        p.part_ml[slot * 2] = any_bad ? __builtin_nanf("") : M;
        p.part_ml[slot * 2 + 1] = L;
      }
    }
  }
}


// One work-group per (partition, KV head x query-head chunk, sequence).
template <typename T, int D, int GT, int NW, bool UB>
__global__ void __launch_bounds__(64 * NW, kDecodeMinBlocks) paged_decode_kernel(const DecodeParams p) {
  __shared__ DecodeSmem<D, GT, NW> sm;
  const int part = blockIdx.x;
  const int b = blockIdx.z;
  float bias;
  const int len = decode_len(p, b, bias);
  const int nparts = (len + p.partition_size - 1) / p.partition_size;
  if (part >= nparts) return;
  const int start = part * p.partition_size;
  const int end = min(start + p.partition_size, len);
  const int ky = blockIdx.y;
  const DecodeDest dst{nparts == 1, ((size_t)b * p.num_heads + decode_first_head<GT>(p, ky, 1)) * p.max_parts + part,
                       p.max_parts};
  decode_range<T, D, GT, NW, 1, UB>(p, sm, b, ky, 1, start, end, bias, dst);
}

// Scheduled launch of whole sequences: work-group i of a 1-D grid takes item i
// -- (sequence, row) with the sequences in the longest-first order of
// decode_order_kernel and hpw KV heads per row.  Work-groups are dispatched in
// index order (dealt round-robin to the XCDs), so the items start longest
// first.  The grid has one work-group per item at hpw = 1; with head pairs the
// upper half, dispatched last, has no item and exits.
template <typename T, int D, int GT, int NW, int HPW, bool UB>
__global__ void __launch_bounds__(64 * NW, kDecodeMinBlocks) paged_decode_scheduled_kernel(const DecodeParams p) {
  __shared__ DecodeSmem<D, GT, NW> sm;
  const int hpw = HPW > 1 ? p.sched[0] : 1;
  const int rows = p.num_kv_heads / hpw * p.head_chunks;
  const int item = blockIdx.x;
  if (item >= p.num_seqs * rows) return;
  const int b = p.sched[1 + item / rows];
  float bias;
  const int len = decode_len(p, b, bias);
  const DecodeDest dst{true, 0, 0};
  decode_range<T, D, GT, NW, HPW, UB>(p, sm, b, item % rows, hpw, 0, len, bias, dst);
}

// Merge the partition partials of each (sequence, query head).  Launched with
// grid (Hq, B) and 64 threads; sequences that fit one partition were written by
// the main kernel and are skipped here.
__global__ void __launch_bounds__(64) paged_decode_reduce_kernel(const DecodeParams p, int head_dim);

// KV heads are paired in the scheduled launch when the longest context is at
// least this many times the shortest (decode_order_kernel).
constexpr int kDecodePairSpread = 3;
__global__ void __launch_bounds__(1024) decode_order_kernel(const int* context_lens, int num_seqs, int width,
                                                            int pair_ok, int* sched);


}  // namespace tv
