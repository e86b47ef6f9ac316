// Attention of the batched decode step (gfx950), fused with the end of the
// q|k|v projection.  One work-group per (sequence, KV head):
//  1. sums the split-K partials of the fused projection for the G = Hq/Hkv
//     query heads of the group and for k, v, and rotates q and k
//     (apply_rope, llama.py:34-55);
//  2. writes k, v into the cache slot of the position -- before attention, or
//     after it in the reference's order (llama.py:378-386);
//  3. attends over the cached context on MFMA: S^T = K Q^T with the group's
//     query heads as the 16 columns (heads >= G are zero), an online softmax
//     over 32-token tiles, O^T += V^T P^T with P kept in registers as the B
//     operand and V^T staged per wave in LDS;
//  4. merges the waves' (max, sum, O) in LDS and stores the G output rows.
// With 8 query heads per KV head at head_dim 64, scores and P.V cost 4
// multiply-adds per cached byte: more than the VALU delivers at HBM speed on
// MI355X (a wave64 fp32 FMA occupies a SIMD for 4 cycles), so this kernel
// runs them on the matrix cores and stays bound by the K/V stream.  Semantics
// are those of paged_decode_attention (llama.py:97-144): softmax over the first
// context_len cached positions (all table positions when context_len <= 0),
// scale 1/sqrt(D), query head h on KV head h / G.
#include "tv_common.h"
#include "tv_dense.h"

namespace tv {

// 16 bytes of a cached K / V row: ordinary or non-temporal load.  V rows are
// read whole (8 lanes per 128-byte row) and stream non-temporally; a K load
// instruction reads half of each 128-byte row (the MFMA operand layout), and
// non-temporal K loads made the TinyLlama decode step 4% slower (V alone: 0.2%
// faster).
template <int NT, typename E> __device__ __forceinline__ u32x4 ld_tile(const E* p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else return *reinterpret_cast<const u32x4*>(p);
}

// A zero the compiler cannot prove uniform: a load indexed by it stays a
// vector load, waited for by vmcnt in order with the other vector loads.
__device__ __forceinline__ int lane_zero() {
  int z;
  __asm__ volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

template <typename T, int D, int NW, int PF>
__global__ void __launch_bounds__(64 * NW) step_attn_kernel(const StepAttnParams p) {
  constexpr int KS = D / 32;        // MFMA k steps over the head dim
  constexpr int DB = D / 16;        // 16-dim blocks of O^T
  constexpr int VP = D + 16;        // V tile row pitch (2 D + 32 bytes): conflict-free transposing reads
  constexpr int CPR = D / 8;        // 16-byte chunks per row
  constexpr int VU = 32 * CPR / 64; // V (token, chunk) units per lane per tile
  constexpr int SVT = NW * 32 * VP; // V tiles of all waves (elements)
  constexpr int SO = NW * 16 * D * 2;   // merge buffer [NW][16][D] floats, in elements
  constexpr int UNION = SVT > SO ? SVT : SO;
  __shared__ __attribute__((aligned(16))) uint16_t smem[16 * D + UNION];
  __shared__ __attribute__((aligned(16))) uint32_t snew[D];   // k (D/2 words) then v of the new token
  __shared__ float sm[NW][16];
  __shared__ float sl[NW][16];
  uint16_t* sq = smem;                       // [16 heads][D] query rows, heads >= G zero
  uint16_t* svt = smem + 16 * D;      // [NW][32 tokens][VP] row-major V tiles

  const int kvh = blockIdx.x;
  const int b = blockIdx.y;
  const int G = p.Hq / p.Hkv;
  const int N = (p.Hq + 2 * p.Hkv) * D;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int col = lane & 15;
  const int bs = p.block_size;
  const int width = p.max_blocks * bs;
  const int ctx = p.context_lens[b];
  const int len = ctx <= 0 ? width : min(ctx, width);
  const int* bt = p.block_tables + (size_t)b * p.bt_stride;
  const int pos = p.positions[b];
  const size_t rs = (size_t)p.Hkv * D;   // elements between cache rows
  T* kcache = reinterpret_cast<T*>(p.k_cache) + (size_t)kvh * D;
  T* vcache = reinterpret_cast<T*>(p.v_cache) + (size_t)kvh * D;
  const int ntiles = (len + 31) >> 5;
  const int nt = ntiles > wave ? (ntiles - wave + NW - 1) / NW : 0;   // this wave's tiles: wave + NW j

  // Block ids of this wave's tiles j0 .. j0+31, one per lane: lane 2 i + h holds
  // the block of half h (16 tokens) of tile j0 + i.  One vector load instead of
  // a dependent table lookup per tile.
  auto load_blocks = [&](int j0) {
    const int tok = (wave + NW * (j0 + (lane >> 1))) * 32 + 16 * (lane & 1);
    return bt[min(tok / bs, p.max_blocks - 1)];
  };
  int blkv = load_blocks(0);

  struct Tile {
    u32x4 k[2][KS];
    u32x4 v[VU];
    int t0;
    bool ok0, ok1;
  };
  // Tile j of this wave: tokens t0 .. t0+31, two 16-token halves each inside
  // one cache block (block_size is a multiple of 16).
  // (j - j0 < 32: the block ids of tiles j0 .. j0+31 are in blkv)
  auto load = [&](int j, int j0, Tile& r) {
    const int t0 = (wave + NW * j) * 32;
    r.t0 = t0;
    int b0 = __builtin_amdgcn_readlane(blkv, 2 * (j - j0));
    int b1 = __builtin_amdgcn_readlane(blkv, 2 * (j - j0) + 1);
    r.ok0 = (unsigned)b0 < (unsigned)p.num_blocks;
    r.ok1 = (unsigned)b1 < (unsigned)p.num_blocks;
    b0 = r.ok0 ? b0 : 0;
    b1 = r.ok1 ? b1 : 0;
    const size_t base0 = ((size_t)b0 * bs + t0 % bs) * rs;
    const size_t base1 = ((size_t)b1 * bs + (t0 + 16) % bs) * rs;
    // K rows: lane (token col of the half, 8-dim group g)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      r.k[0][ks] = ld_tile<0>(kcache + base0 + col * rs + 32 * ks + 8 * g);
      r.k[1][ks] = ld_tile<0>(kcache + base1 + col * rs + 32 * ks + 8 * g);
    }
    // V rows: unit (token, 16-byte chunk), staged row-major in LDS
#pragma unroll
    for (int i = 0; i < VU; ++i) {
      const int unit = lane + 64 * i;
      const int tok = unit / CPR;
      const int ch = unit % CPR;
      r.v[i] = ld_tile<1>(vcache + (tok < 16 ? base0 : base1) + (size_t)(tok & 15) * rs + 8 * ch);
    }
  };

  // ---- q, k, v of the new token: loads ------------------------------------
  // Thread tid's first item of the group's q | k | v columns (G*D/2 q pairs,
  // D/2 k pairs, D/2 v pairs): all its split partials and its RoPE pair are
  // requested here, after the block ids and before the tile loads, so the
  // tile loads wait only for the block ids and the sums below only for these
  // loads -- one round trip instead of one per split.  Loads are unconditional
  // (clamped item and split indexes); the extras are dropped.
  constexpr int SB = 8;                    // split partials requested at once
  const int nq = G * (D / 2);
  const int nitems = nq + D;
  const int pr = min(max(pos, 0), p.rope_len - 1);
  const float* part = p.part + (size_t)b * N;
  const size_t sstride = (size_t)p.B * N;
  auto item_col = [&](int it, int& d2) {   // output column of item it, and its rotation pair index
    if (it < nq) {
      d2 = it % (D / 2);
      return (kvh * G + it / (D / 2)) * D + 2 * d2;
    }
    if (it < nq + D / 2) {
      d2 = it - nq;
      return p.Hq * D + kvh * D + 2 * d2;
    }
    d2 = it - nq - D / 2;
    return (p.Hq + p.Hkv) * D + kvh * D + 2 * d2;
  };
  auto load_parts = [&](int n, int s0, float2 (&pv)[SB]) {
#pragma unroll
    for (int s = 0; s < SB; ++s)
      pv[s] = *reinterpret_cast<const float2*>(part + (size_t)min(s0 + s, p.splits - 1) * sstride + n);
  };
  int d2_0;
  const int n0 = item_col(min(tid, nitems - 1), d2_0);
  float2 pv0[SB];
  load_parts(n0, 0, pv0);
  const float2 cs0 = *reinterpret_cast<const float2*>(p.rope + ((size_t)pr * (D / 2) + d2_0) * 2);
  // The block of the step's token, for its cache slot: a vector load issued
  // before the tile loads and waited for only where k / v are stored.  (A
  // scalar load after the tile loads returned ~4 us after the position,
  // behind the tile stream, by per-work-group clock stamps of a timing copy;
  // the launch itself is ~0.1 us shorter this way, TinyLlama step at B64.)
  const int slot_blk = bt[(pos >= 0 ? min(pos / bs, p.bt_stride - 1) : 0) + lane_zero()];
  __builtin_amdgcn_sched_barrier(0);   // issued here, ahead of the tile loads

  // The first tiles' K / V loads depend only on the block table: issue them
  // before the prologue's arithmetic so their latency overlaps it (tile 0 of
  // the wave is a valid address even when the wave has no tile; it is not used).
  Tile t[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) load(min(i, max(nt, 1) - 1), 0, t[i]);

  // ---- q, k, v of the new token: sums, RoPE, stores --------------------------
  const long long slot = pos >= 0 && pos / bs < p.bt_stride && slot_blk >= 0 && slot_blk < p.num_blocks
                            ? (long long)slot_blk * bs + pos % bs : -1;
  {
    auto finish_item = [&](int it, int d2, float v0, float v1, float2 cs) {
      if (it < nq + D / 2) {
        const float a = v0 * cs.x - v1 * cs.y;
        const float c2 = v0 * cs.y + v1 * cs.x;
        v0 = a;
        v1 = c2;
      }
      const uint32_t w = pack2<T>(v0, v1);
      if (it < nq) {
        *reinterpret_cast<uint32_t*>(&sq[(it / (D / 2)) * D + 2 * d2]) = w;
      } else {
        snew[it - nq] = w;
        // written now for later steps; this step's attention takes them from snew
        if (p.write_before && slot >= 0)
          *reinterpret_cast<uint32_t*>((it < nq + D / 2 ? kcache : vcache) + (size_t)slot * rs + 2 * d2) = w;
      }
    };
    // splits summed in order 0, 1, 2, ... whichever batch they arrive in
    auto sum_item = [&](int n, const float2 (&first)[SB], float& v0, float& v1) {
      v0 = 0.0f;
      v1 = 0.0f;
#pragma unroll
      for (int s = 0; s < SB; ++s)
        if (s < p.splits) {
          v0 += first[s].x;
          v1 += first[s].y;
        }
      for (int s0 = SB; s0 < p.splits; s0 += SB) {
        float2 pv[SB];
        load_parts(n, s0, pv);
#pragma unroll
        for (int s = 0; s < SB; ++s)
          if (s0 + s < p.splits) {
            v0 += pv[s].x;
            v1 += pv[s].y;
          }
      }
    };
    if (tid < nitems) {
      float v0, v1;
      sum_item(n0, pv0, v0, v1);
      finish_item(tid, d2_0, v0, v1, cs0);
    }
    // items beyond the first of a thread (head_dim 128, or large groups)
    for (int it = tid + 64 * NW; it < nitems; it += 64 * NW) {
      int d2;
      const int n = item_col(it, d2);
      float2 pv[SB];
      load_parts(n, 0, pv);
      const float2 cs = *reinterpret_cast<const float2*>(p.rope + ((size_t)pr * (D / 2) + d2) * 2);
      float v0, v1;
      sum_item(n, pv, v0, v1);
      finish_item(it, d2, v0, v1, cs);
    }
    for (int it = tid; it < (16 - G) * (D / 2); it += 64 * NW)
      *reinterpret_cast<uint32_t*>(&sq[G * D + 2 * it]) = 0u;
  }
  lds_barrier();   // q rows and the new k/v in LDS

  // ---- attention over [0, len) ----------------------------------------------
  u32x4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(&sq[col * D + 32 * ks + 8 * g]);
  const float c = p.scale * kLog2e;
  float m = kNegInf;
  float lsum = 0.0f;
  f32x4 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint16_t* vt = svt + wave * (32 * VP);

  auto consume = [&](Tile& r) {
    if (p.write_before && r.t0 <= pos && pos < r.t0 + 32) {
      // the new token's row, from LDS (its cache store need not be visible yet)
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
        if (r.t0 + 16 * tb + col == pos) {
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) r.k[tb][ks] = *reinterpret_cast<const u32x4*>(&snew[16 * ks + 4 * g]);
        }
#pragma unroll
      for (int i = 0; i < VU; ++i) {
        const int unit = lane + 64 * i;
        if (r.t0 + unit / CPR == pos) r.v[i] = *reinterpret_cast<const u32x4*>(&snew[D / 2 + 4 * (unit % CPR)]);
      }
    }
    // S^T: st[tb][i] = q_head(col) . k(token t0 + 16 tb + 4 g + i)
    f32x4 st[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      st[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) st[tb] = mfma16x16x32<T>(r.k[tb][ks], qf[ks], st[tb]);
    }
    const bool partial = r.t0 + 32 > len || !r.ok0 || !r.ok1;
    if (partial) {
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool ok = r.t0 + 16 * tb + 4 * g + i < len && (tb ? r.ok1 : r.ok0);
          st[tb][i] = ok ? st[tb][i] : kNegInf;
        }
    }
    float mt = fmaxf(fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3])),
                     fmaxf(fmaxf(st[1][0], st[1][1]), fmaxf(st[1][2], st[1][3])));
    mt = max_over_g(mt);
    // the running max is only raised when it grows by more than 8 log2 units
    const float mtc = mt * c;
    float mc = m == kNegInf ? kNegInf : m * c;
    if (__builtin_amdgcn_ballot_w64(mtc > mc + 8.0f) != 0) {
      __asm__ volatile("" ::: "memory");
      const float mn = mtc > mc + 8.0f ? fmaxf(m, mt) : m;
      const float alpha = mn == kNegInf ? 1.0f : fast_exp2((m - mn) * c);
      m = mn;
      mc = m == kNegInf ? kNegInf : m * c;
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
    }
    if (mc == kNegInf) mc = 0.0f;
    float e[2][4];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        e[tb][i] = fast_exp2(fmaf(st[tb][i], c, -mc));
        lsum += e[tb][i];
      }
    // reduction index kk = 8 g + j: token 4 g + j of the first half for j < 4,
    // token 16 + 4 g + j - 4 for j >= 4, on both MFMA operands
    const u32x4 pf = u32x4{pack2<T>(e[0][0], e[0][1]), pack2<T>(e[0][2], e[0][3]), pack2<T>(e[1][0], e[1][1]),
                           pack2<T>(e[1][2], e[1][3])};
    // V tile rows in LDS (rows of masked tokens zeroed), read back as the V^T
    // operand by transposing reads: rows 4 g + (col >> 2) (+16), columns
    // db * 16 + 4 (col & 3) give lane (g, col) V[token(8 g + j)][db * 16 + col]
#pragma unroll
    for (int i = 0; i < VU; ++i) {
      const int unit = lane + 64 * i;
      const int tok = unit / CPR;
      u32x4 v = r.v[i];
      if (partial && (!(tok < 16 ? r.ok0 : r.ok1) || r.t0 + tok >= len)) v = u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(&vt[tok * VP + 8 * (unit % CPR)]) = v;
    }
    // O^T += V^T P^T
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const uint16_t* a = &vt[(4 * g + (col >> 2)) * VP + db * 16 + 4 * (col & 3)];
      const u32x2 lo = lds_read_tr16(a);
      const u32x2 hi = lds_read_tr16(a + 16 * VP);
      o[db] = mfma16x16x32<T>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pf, o[db]);
    }
  };

  // Chunks of 32 tiles (one block id per lane and half); within a chunk PF
  // tiles are in flight and the loads are unconditional (the chunk's last tile
  // is re-read) so the compiler waits for exactly the tile it consumes.
  for (int j0 = 0; j0 < nt; j0 += 32) {
    const int je = min(nt, j0 + 32);
    if (j0 > 0) {
      blkv = load_blocks(j0);
#pragma unroll
      for (int i = 0; i < PF; ++i) load(min(j0 + i, je - 1), j0, t[i]);
    }
    int j = j0;
    for (; j + PF - 1 < je; j += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        consume(t[i]);
        load(min(j + PF + i, je - 1), j0, t[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < PF - 1; ++i)
      if (j + i < je) consume(t[i]);
  }

  // ---- merge the waves ----------------------------------------------------------
  lsum = sum_over_g(lsum);
  lds_barrier();   // every wave is done with its V^T tile: the buffer becomes [NW][16][D] floats
  float* so = reinterpret_cast<float*>(svt);
  if (g == 0) {
    sm[wave][col] = m;
    sl[wave][col] = lsum;
  }
#pragma unroll
  for (int db = 0; db < DB; ++db)
    *reinterpret_cast<f32x4*>(&so[(wave * 16 + col) * D + db * 16 + 4 * g]) = o[db];
  lds_barrier();
  T* out = reinterpret_cast<T*>(p.out) + ((size_t)b * p.Hq + (size_t)kvh * G) * D;
  for (int it = tid; it < G * D; it += 64 * NW) {
    const int h = it / D;
    const int d = it - h * D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm[w][h]);
    float L = 0.0f, acc = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = sm[w][h] == kNegInf ? 0.0f : fast_exp2((sm[w][h] - M) * c);
      L += sl[w][h] * f;
      acc += so[(w * 16 + h) * D + d] * f;
    }
    out[it] = from_float<T>(L > 0.0f ? acc / L : 0.0f);
  }
  if (!p.write_before && slot >= 0 && tid < D) {
    // the reference's order: the step's k/v reach the cache after attention
    T* dst = (tid < D / 2 ? kcache : vcache) + (size_t)slot * rs + 2 * (tid % (D / 2));
    *reinterpret_cast<uint32_t*>(dst) = snew[tid];
  }
}

bool step_attn_supported(int head_dim, int group, int block_size) {
  return (head_dim == 64 || head_dim == 128) && group >= 1 && group <= 16 && block_size % 16 == 0;
}

constexpr int kStepAttnWaves64 = 6;      // waves per work-group at head_dim 64
constexpr int kStepAttnInFlight64 = 2;   // tiles in flight per wave at head_dim 64

// head_dim 64: 6 waves and two tiles in flight per wave (TinyLlama step, batch
// 64 x 4 KV heads, one work-group per CU: 1480 us/step against 1482 with one
// tile in flight, 1487 with 8 waves and one tile, 1496 with 8 waves and two,
// 1543 with 12, 1548 with 16); head_dim 128: 4 waves, whose larger tiles need
// more than the 256 registers two waves per SIMD allow.
void launch_step_attn(const StepAttnParams& p, int head_dim, int dtype, hipStream_t s) {
  constexpr int W64 = kStepAttnWaves64, PF64 = kStepAttnInFlight64;
  const dim3 grid(p.Hkv, p.B);
  if (dtype == kF16) {
    if (head_dim == 64) hipLaunchKernelGGL((step_attn_kernel<_Float16, 64, W64, PF64>), grid, dim3(64 * W64), 0, s, p);
    else hipLaunchKernelGGL((step_attn_kernel<_Float16, 128, 4, 2>), grid, dim3(256), 0, s, p);
  } else {
    if (head_dim == 64) hipLaunchKernelGGL((step_attn_kernel<__bf16, 64, W64, PF64>), grid, dim3(64 * W64), 0, s, p);
    else hipLaunchKernelGGL((step_attn_kernel<__bf16, 128, 4, 2>), grid, dim3(256), 0, s, p);
  }
}

}  // namespace tv
