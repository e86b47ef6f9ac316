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
#ifndef TV_PREFILL_BN
#define TV_PREFILL_BN 64
#endif
constexpr int kPrefillBN = TV_PREFILL_BN;   // keys per tile (64 or 128)
#ifndef TV_PREFILL_KSPLIT
#define TV_PREFILL_KSPLIT 2   // groups of 4 waves splitting a row block's key tiles (head_dim 64)
#endif

// Key tiles query tile qt needs (causal rows stop at the diagonal).
__device__ __forceinline__ int prefill_key_tiles(const PrefillParams& p, int qt) {
  const int kend = p.causal ? min(p.kv_len, (qt + 1) * kPrefillBM) : p.kv_len;
  return (kend + kPrefillBN - 1) / kPrefillBN;
}

// Map grid.y to (query tile, chunk of key tiles).  Without chunk splitting
// the order is zig-zag: the longer half of the causal query tiles longest
// first, then the shorter half shortest first, so the two work-groups that
// become resident on one CU (linear ids i and i + grid/2) carry about the
// same total number of key tiles.  With splitting: longest first.
__device__ __forceinline__ void prefill_unit(const PrefillParams& p, int u, int& qt, int& chunk, int& nchunks) {
  const int nqt = (p.q_len + kPrefillBM - 1) / kPrefillBM;
  if (p.max_chunks == 1) {
    const int half = (nqt + 1) / 2;
    qt = u < half ? nqt - 1 - u : u - half;
    chunk = 0;
    nchunks = 1;
    return;
  }
  for (qt = nqt - 1; qt > 0; --qt) {
    const int ch = (prefill_key_tiles(p, qt) + p.chunk_tiles - 1) / p.chunk_tiles;
    if (u < ch) break;
    u -= ch;
  }
  nchunks = (prefill_key_tiles(p, qt) + p.chunk_tiles - 1) / p.chunk_tiles;
  chunk = u;
}

// Store 4 consecutive output elements (a row slice of one query) as out_dtype.
template <typename T>
__device__ __forceinline__ void store4(void* base, size_t idx, f32x4 v, int out_dtype) {
  if (out_dtype == kF32) {
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(base) + idx) = v;
  } else {
    const u32x2 w = u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(base) + idx) = w;
  }
}

// KSPLIT groups of 4 waves share the 64 query rows of a work-group; group s
// takes key tiles kt0 + s, kt0 + s + KSPLIT, ... in its own LDS buffers and the
// groups merge their (max, row sum, O) through LDS at the end.  Every group
// runs the same number of steps (idle groups load and skip a clamped tile) so
// all waves meet at every barrier.
template <typename T, int D, int KSPLIT>
__global__ void __launch_bounds__(256 * KSPLIT) prefill_mfma_kernel(const PrefillParams p) {
  constexpr int BM = kPrefillBM;
  constexpr int BN = kPrefillBN;
  constexpr int KP = D + 8;       // LDS pitch of the K tile (elements)
  constexpr int VP = BN + 4;      // LDS pitch of the V^T tile: 8-byte reads of 16 rows hit distinct banks
  constexpr int DB = D / 16;      // 16-row blocks of O^T; block DB holds the row sums
  constexpr int KS = D / 32;      // MFMA steps over the head dim
  constexpr int VPT = BN * (D / 8) / 256;          // 16-byte K vectors per thread per tile
  constexpr int VPT2 = (BN / 2) * (D / 8) / 256;   // V key pairs per thread per tile
  constexpr int SK = BN * KP;                // K tile (elements)
  constexpr int SV = (D + 16) * VP;          // V^T tile plus 16 rows of ones
  // V^T tile plus 16 rows of ones: the MFMA against them yields the softmax
  // row sums of the (rounded) P that the numerator uses, for free.
  // tile buffers of all groups; reused afterwards for the group merge
  constexpr int TILE_ELEMS = KSPLIT * (SK + SV);
  constexpr int MERGE_ELEMS = KSPLIT > 1 ? KSPLIT * (BM * (D + 16) + BM) * 2 : 0;
  __shared__ __attribute__((aligned(16))) uint16_t smem[TILE_ELEMS > MERGE_ELEMS ? TILE_ELEMS : MERGE_ELEMS];

  const int grp = threadIdx.x >> 8;          // key-split group
  const int tid = threadIdx.x & 255;         // thread within the group
  const int wave = tid >> 6;
  uint16_t* sk = smem + grp * (SK + SV);
  uint16_t* sv = sk + SK;
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
  for (int ks = 0; ks < KS; ++ks)
    qf[ks] = qi < p.q_len
                 ? *reinterpret_cast<const u32x4*>(qg + (size_t)qi * p.q_stride + (size_t)h * D + ks * 32 + g * 8)
                 : u32x4{0, 0, 0, 0};

  {  // ones rows of the extended V^T (never overwritten by tile stores)
    const uint16_t one = __builtin_bit_cast(uint16_t, from_float<T>(1.0f));
    for (int idx = tid; idx < 16 * VP; idx += 256) sv[D * VP + idx] = one;
  }

  // Per-thread element offsets inside a tile (the tile base is wave-uniform).
  // K: thread -> (key, 8-dim chunk), consecutive lanes along a row.
  // V: thread -> (key pair, 8-dim chunk); pairs are interleaved into 32-bit
  //    words with v_perm so V^T is written with ds_write_b32.
  int k_row[VPT], k_col[VPT], v_row[VPT2], v_col[VPT2];
  size_t k_off[VPT], v_off[VPT2];   // element offsets from the tile's first row (full tiles)
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = tid + i * 256;
    k_row[i] = idx / (D / 8);
    k_col[i] = idx - k_row[i] * (D / 8);
    k_off[i] = (size_t)k_row[i] * p.k_stride + k_col[i] * 8;
  }
#pragma unroll
  for (int i = 0; i < VPT2; ++i) {
    const int unit = tid + i * 256;
    v_row[i] = 2 * (unit % (BN / 2));
    v_col[i] = unit / (BN / 2);
    v_off[i] = (size_t)v_row[i] * p.v_stride + v_col[i] * 8;
  }

  struct TileRegs {
    u32x4 k[VPT];
    u32x4 v[VPT2][2];
    int k0;   // first key of the tile
  };
  // Every step issues the same loads (rows past kv_len re-read the last valid
  // row), so the compiler waits for exactly the tile it needs; the registers
  // are not touched until lstore.
  auto gload = [&](int kt, TileRegs& r) {
    const int k0 = kt * BN;
    r.k0 = k0;
    const T* kb = kg + (size_t)k0 * p.k_stride;
    const T* vb = vg + (size_t)k0 * p.v_stride;
    if (k0 + BN <= p.kv_len) {
#pragma unroll
      for (int i = 0; i < VPT; ++i) r.k[i] = *reinterpret_cast<const u32x4*>(kb + k_off[i]);
#pragma unroll
      for (int i = 0; i < VPT2; ++i) {
        r.v[i][0] = *reinterpret_cast<const u32x4*>(vb + v_off[i]);
        r.v[i][1] = *reinterpret_cast<const u32x4*>(vb + v_off[i] + p.v_stride);
      }
    } else {
      const int last = p.kv_len - 1 - k0;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        r.k[i] = *reinterpret_cast<const u32x4*>(kb + (size_t)min(k_row[i], last) * p.k_stride + k_col[i] * 8);
#pragma unroll
      for (int i = 0; i < VPT2; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          r.v[i][t] = *reinterpret_cast<const u32x4*>(vb + (size_t)min(v_row[i] + t, last) * p.v_stride +
                                                       v_col[i] * 8);
    }
  };
  auto lstore = [&](const TileRegs& r) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) *reinterpret_cast<u32x4*>(&sk[k_row[i] * KP + k_col[i] * 8]) = r.k[i];
    const bool partial = r.k0 + BN > p.kv_len;   // zero V rows past the sequence
#pragma unroll
    for (int i = 0; i < VPT2; ++i) {
      u32x4 v0 = r.v[i][0], v1 = r.v[i][1];
      if (partial) {
        if (r.k0 + v_row[i] >= p.kv_len) v0 = u32x4{0, 0, 0, 0};
        if (r.k0 + v_row[i] + 1 >= p.kv_len) v1 = u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint16_t* dst = &sv[(v_col[i] * 8 + 2 * w) * VP + v_row[i]];
        *reinterpret_cast<uint32_t*>(dst) = __builtin_amdgcn_perm(v1[w], v0[w], 0x05040100u);
        *reinterpret_cast<uint32_t*>(dst + VP) = __builtin_amdgcn_perm(v1[w], v0[w], 0x07060302u);
      }
    }
  };

  f32x4 oacc[DB + 1];
#pragma unroll
  for (int i = 0; i <= DB; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf;      // running max of the raw scores q.k of this query column
  const float c = p.scale * kLog2e;

  auto compute = [&](int kt) {
    const int k0 = kt * BN;
    // S^T = K Q^T: st[kb][i] = q.k for query qi and key k0 + kb*16 + 4g + i
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
    // mask only tiles that cross the diagonal or the end of the sequence
    if (!(k0 + BN <= p.kv_len && (!p.causal || k0 + BN - 1 <= qt * BM))) {
      const int lim = p.causal ? min(p.kv_len - 1, qi) : p.kv_len - 1;   // last visible key
#pragma unroll
      for (int kb = 0; kb < BN / 16; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[kb][i] = k0 + kb * 16 + 4 * g + i <= lim ? st[kb][i] : kNegInf;
    }
    float mt;
    {  // max of the 4*BN/16 raw scores with a v_max3 tree
      float r[BN / 16 * 4];
#pragma unroll
      for (int kb = 0; kb < BN / 16; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) r[kb * 4 + i] = st[kb][i];
      constexpr int N = BN / 16 * 4;
      float t[(N + 2) / 3];
#pragma unroll
      for (int a = 0; a < N / 3; ++a) t[a] = fmaxf(fmaxf(r[3 * a], r[3 * a + 1]), r[3 * a + 2]);
      int nt = N / 3;
      if constexpr (N % 3 == 1) t[nt++] = r[N - 1];
      if constexpr (N % 3 == 2) t[nt++] = fmaxf(r[N - 2], r[N - 1]);
      mt = t[0];
#pragma unroll
      for (int a = 1; a + 1 < (N + 2) / 3; a += 2) mt = fmaxf(fmaxf(mt, t[a]), t[a + 1]);
      if constexpr (((N + 2) / 3) % 2 == 0) mt = fmaxf(mt, t[(N + 2) / 3 - 1]);
    }
    mt = max_over_g(mt);
    // the running max is only raised when it grows by more than 8 log2 units
    // (rare after the first tile); unnormalised weights stay <= 2^8
    const float mtc = mt * c;
    float mc = m == kNegInf ? kNegInf : m * c;
    if (__builtin_amdgcn_ballot_w64(mtc > mc + 8.0f) != 0) {
      __asm__ volatile("" ::: "memory");
      const float mn = mtc > mc + 8.0f ? fmaxf(m, mt) : m;
      const float alpha = mn == kNegInf ? 1.0f : fast_exp2((m - mn) * c);
      m = mn;
      mc = m == kNegInf ? kNegInf : m * c;
#pragma unroll
      for (int db = 0; db <= DB; ++db) oacc[db] *= alpha;
    }
    if (mc == kNegInf) mc = 0.0f;
    u32x4 pf[BN / 32];
#pragma unroll
    for (int kb = 0; kb < BN / 16; ++kb) {
      const float e0 = fast_exp2(fmaf(st[kb][0], c, -mc));
      const float e1 = fast_exp2(fmaf(st[kb][1], c, -mc));
      const float e2 = fast_exp2(fmaf(st[kb][2], c, -mc));
      const float e3 = fast_exp2(fmaf(st[kb][3], c, -mc));
      // reduction index kk = 8g + j maps to key 4g+j (j<4) of block 2*ks2 and
      // key 4g+j-4 (j>=4) of block 2*ks2+1 on both MFMA operands
      pf[kb >> 1][(kb & 1) * 2] = pack2<T>(e0, e1);
      pf[kb >> 1][(kb & 1) * 2 + 1] = pack2<T>(e2, e3);
    }
    // O^T += V^T P^T (block DB: the ones rows -> row sums)
#pragma unroll
    for (int db = 0; db <= DB; ++db) {
#pragma unroll
      for (int ks2 = 0; ks2 < BN / 32; ++ks2) {
        const uint16_t* row = &sv[(db * 16 + col) * VP + ks2 * 32 + 4 * g];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(row);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(row + 16);
        oacc[db] = mfma16x16x32<T>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pf[ks2], oacc[db]);
      }
    }
  };
  // group tile sequence: kt0 + grp + KSPLIT * j, j < nsteps (same count for all groups)
  const int nsteps = (kt1 - kt0 + KSPLIT - 1) / KSPLIT;
  auto tile_of = [&](int j) { return min(kt0 + grp + KSPLIT * j, kt1 - 1); };
  auto step = [&](int j, TileRegs& r) {
    lds_barrier();
    lstore(r);
    lds_barrier();
    gload(tile_of(j + 2), r);          // two steps ahead (clamped: re-reads are unused)
    if (kt0 + grp + KSPLIT * j < kt1) compute(kt0 + grp + KSPLIT * j);
  };

  TileRegs ra, rb;
  gload(tile_of(0), ra);
  gload(tile_of(1), rb);
  // both steps of the loop body are unconditional so the number of loads in
  // flight is the same on every path (the final odd step is peeled)
  int j = 0;
  for (; j + 1 < nsteps; j += 2) {
    step(j, ra);
    step(j + 1, rb);
  }
  if (j < nsteps) step(j, ra);

  if constexpr (KSPLIT > 1) {
    // merge the groups: each publishes (scaled max, O unnormalised incl. row sums)
    lds_barrier();
    float* so = reinterpret_cast<float*>(smem);                  // [KSPLIT][64 rows][D + 16]
    float* sm = so + KSPLIT * BM * (D + 16);                     // [KSPLIT][64 rows]
    const int row = wave * 16 + col;
#pragma unroll
    for (int db = 0; db <= DB; ++db)
      *reinterpret_cast<f32x4*>(&so[(grp * BM + row) * (D + 16) + db * 16 + 4 * g]) = oacc[db];
    if (g == 0) sm[grp * BM + row] = m == kNegInf ? kNegInf : m * c;
    lds_barrier();
    if (grp != 0) return;
    float M = kNegInf;
#pragma unroll
    for (int s2 = 0; s2 < KSPLIT; ++s2) M = fmaxf(M, sm[s2 * BM + row]);
#pragma unroll
    for (int db = 0; db <= DB; ++db) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s2 = 0; s2 < KSPLIT; ++s2) {
      const float ms = sm[s2 * BM + row];
      const float f = ms == kNegInf ? 0.0f : fast_exp2(ms - M);
#pragma unroll
      for (int db = 0; db <= DB; ++db)
        oacc[db] += *reinterpret_cast<const f32x4*>(&so[(s2 * BM + row) * (D + 16) + db * 16 + 4 * g]) * f;
    }
    m = M == kNegInf ? kNegInf : M / c;
  }

  const float lsum = oacc[DB][0];
  if (qi >= p.q_len) return;
  const float inv = 1.0f / lsum;
  if (nchunks == 1) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
      store4<T>(p.out, (size_t)qi * p.out_stride + (size_t)h * D + db * 16 + 4 * g, oacc[db] * inv, p.out_dtype);
    return;
  }
  // partial of this key chunk: normalised O plus (max, sum) per query row
  const int nqt = (p.q_len + BM - 1) / BM;
  const size_t unit = ((size_t)h * nqt + qt) * p.max_chunks + chunk;
  const int row = qi - qt * BM;
  float* po = p.part_o + (unit * BM + row) * D;
#pragma unroll
  for (int db = 0; db < DB; ++db) *reinterpret_cast<f32x4*>(po + db * 16 + 4 * g) = oacc[db] * inv;
  if (g == 0) {
    p.part_ml[(unit * BM + row) * 2] = m == kNegInf ? kNegInf : m * c;
    p.part_ml[(unit * BM + row) * 2 + 1] = lsum;
  }
}

// ---------------------------------------------------------------------------
// MFMA kernel, head_dim 64: register-lean softmax, double-buffered tiles
// ---------------------------------------------------------------------------
//
// A work-group owns 64 query rows of one head.  KS groups of QW = 4 / RB waves
// split the row block's key tiles (group s takes tiles kt0 + s + KS j); every
// wave owns RB blocks of 16 query rows, so each K / V fragment read from LDS
// feeds RB matrix products.  Per 64-key tile a wave computes S^T = K Q^T with
// Q pre-scaled by scale * log2(e) and the accumulator initialised to -m (the
// running reference maximum of the query), so the scores come out of the
// matrix cores already in the log2 domain relative to m and go straight into
// v_exp_f32.  m is raised only when a tile exceeds it by more than 8, which
// after the first tile is rare.  V is staged row-major in LDS and read as
// the V^T operand with ds_read_b64_tr_b16; the softmax row sums come from one
// extra MFMA of P against a register of ones.  Tiles are double-buffered in LDS
// and loaded two steps ahead through buffer loads whose range ends at the last
// key row (rows past kv_len read as zero), one barrier per step.

template <typename T> __device__ __forceinline__ u32x4 scale8(u32x4 w, float c) {
  u32x4 r;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float a, b;
    unpack2<T>(w[k], a, b);
    r[k] = pack2<T>(a * c, b * c);
  }
  return r;
}

template <typename T> constexpr uint32_t kOnes2 = 0;
template <> constexpr uint32_t kOnes2<_Float16> = 0x3C003C00u;
template <> constexpr uint32_t kOnes2<__bf16> = 0x3F803F80u;

// maximum of the 4 KB values of one S^T tile (v_max3 tree)
template <int KB> __device__ __forceinline__ float max_tile(const f32x4 (&st)[KB]) {
  float t[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) t[kb] = fmaxf(fmaxf(st[kb][0], st[kb][1]), fmaxf(st[kb][2], st[kb][3]));
#pragma unroll
  for (int w = 1; w < KB; w *= 2)
#pragma unroll
    for (int kb = 0; kb + w < KB; kb += 2 * w) t[kb] = fmaxf(t[kb], t[kb + w]);
  return t[0];
}

#ifndef TV_PREFILL_RB
#define TV_PREFILL_RB 2       // 16-row query blocks per wave (head_dim 64)
#endif
#ifndef TV_PREFILL_KS
#define TV_PREFILL_KS 2       // key-tile groups per work-group (head_dim 64)
#endif
#ifndef TV_PREFILL_FA_BN
#define TV_PREFILL_FA_BN 64
#endif
#ifndef TV_PREFILL_WAVES_PER_EU
#define TV_PREFILL_WAVES_PER_EU 2
#endif

template <typename T, int D, int RB, int KS, int BN>
__global__ void __launch_bounds__(256 / RB * KS) __attribute__((amdgpu_waves_per_eu(TV_PREFILL_WAVES_PER_EU)))
prefill_fa_kernel(const PrefillParams p) {
  constexpr int QW = 4 / RB;              // waves of a group along the 64 query rows
  constexpr int GT = 64 * QW;             // threads of a group
  constexpr int BM = kPrefillBM;
  constexpr int KB = BN / 16;             // 16-key blocks of a tile
  // Row pitches of 2 D + 32 bytes (an odd multiple of 32 modulo 256): measured
  // conflict-free for the 16-byte fragment reads of K and the transposing
  // 8-byte reads of V (a pitch of 2 D + 16 bytes costs the K reads ~20%).
  constexpr int KP = D + 16;
  constexpr int VP = D + 16;
  constexpr int SKT = BN * KP;
  constexpr int BUF = SKT + BN * VP;      // one K + V tile buffer (elements)
  constexpr int KSD = D / 32;             // MFMA steps over the head dim
  constexpr int DB = D / 16;              // 16-dim blocks of O^T
  constexpr int CPR = D / 8;              // 16-byte vectors per row
  constexpr int NV = BN * CPR / GT;       // vectors per thread per tile, each of K and V
  constexpr int MP = D + 4;               // merge row pitch (floats): the 16 rows of a store hit distinct banks
  constexpr int MERGE = KS > 1 ? KS * BM * (MP + 2) * 2 : 0;   // merge area (uint16 units)
  constexpr int SMEM = KS * 2 * BUF > MERGE ? KS * 2 * BUF : MERGE;
  static_assert(BN % 32 == 0 && NV * GT == BN * CPR, "tile shape");
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];

  const int grp = __builtin_amdgcn_readfirstlane(threadIdx.x / GT);
  const int tid = threadIdx.x - grp * GT;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int col = lane & 15;
  uint16_t* const tiles = smem + grp * 2 * BUF;

  const int h = prefill_head(blockIdx.x, p.num_heads, p.xcd_remap);
  int qt, chunk, nchunks;
  prefill_unit(p, blockIdx.y, qt, chunk, nchunks);
  const int kvh = h / (p.num_heads / p.num_kv_heads);
  // keys [kbeg, kend) of this unit (64-key units of the chunking), in BN-key tiles
  const int nkt = prefill_key_tiles(p, qt);
  const int kt0 = chunk * p.chunk_tiles;
  const int kt1 = min(kt0 + p.chunk_tiles, nkt);
  const int kbeg = kt0 * kPrefillBN;
  const int klim = min(kt1 * kPrefillBN, p.kv_len);                 // end before the causal limit
  const int kend = p.causal ? min(klim, (qt + 1) * BM) : klim;
  const int ntiles = (kend - kbeg + BN - 1) / BN;
  const float c = p.scale * kLog2e;
  const int row0 = qt * BM + wave * RB * 16;   // first query row of this wave

  int qi[RB];
  u32x4 qf[RB][KSD];
  {
    const T* qg = reinterpret_cast<const T*>(p.q) + (size_t)h * D;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      qi[r] = row0 + r * 16 + col;
#pragma unroll
      for (int ks = 0; ks < KSD; ++ks)
        qf[r][ks] = qi[r] < p.q_len
                        ? scale8<T>(*reinterpret_cast<const u32x4*>(qg + (size_t)qi[r] * p.q_stride + ks * 32 + g * 8), c)
                        : u32x4{0, 0, 0, 0};
    }
  }

  // global -> LDS staging: thread vector i = (row, 16-byte column chunk)
  const T* kbase = reinterpret_cast<const T*>(p.k) + (size_t)kvh * D;
  const T* vbase = reinterpret_cast<const T*>(p.v) + (size_t)kvh * D;
  int koff[NV], voff[NV], kdst[NV], vdst[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = tid + i * GT;
    const int row = v / CPR, ch = v - (v / CPR) * CPR;
    koff[i] = (int)(row * p.k_stride + ch * 8) * (int)sizeof(T);
    voff[i] = (int)(row * p.v_stride + ch * 8) * (int)sizeof(T);
    kdst[i] = row * KP + ch * 8;
    vdst[i] = SKT + row * VP + ch * 8;
  }
  struct Stage {
    u32x4 k[NV], v[NV];
  };
  auto tile_of = [&](int j) { return min(grp + KS * j, ntiles - 1); };
  // per-tile buffer resources: base at the tile's first row, range ending at
  // the last key row, so rows past kv_len read as zero (byte quantities in
  // scalar registers, one multiply per tile)
  const char* kfirst = reinterpret_cast<const char*>(kbase + (size_t)kbeg * p.k_stride);
  const char* vfirst = reinterpret_cast<const char*>(vbase + (size_t)kbeg * p.v_stride);
  const unsigned long long kstep = (unsigned long long)BN * p.k_stride * sizeof(T);
  const unsigned long long vstep = (unsigned long long)BN * p.v_stride * sizeof(T);
  const unsigned long long kbytes = ((unsigned long long)(p.kv_len - 1 - kbeg) * p.k_stride + D) * sizeof(T);
  const unsigned long long vbytes = ((unsigned long long)(p.kv_len - 1 - kbeg) * p.v_stride + D) * sizeof(T);
  auto gload = [&](int j, Stage& s) {
    const unsigned t = (unsigned)tile_of(j);
    const unsigned long long ko = t * kstep, vo = t * vstep;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kfirst + ko, kbytes - ko);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vfirst + vo, vbytes - vo);
#pragma unroll
    for (int i = 0; i < NV; ++i) s.k[i] = buffer_load16(rk, koff[i], 0);
#pragma unroll
    for (int i = 0; i < NV; ++i) s.v[i] = buffer_load16(rv, voff[i], 0);
  };
  auto lstore = [&](const Stage& s, int b) {
    uint16_t* t = tiles + b * BUF;
#pragma unroll
    for (int i = 0; i < NV; ++i) *reinterpret_cast<u32x4*>(t + kdst[i]) = s.k[i];
#pragma unroll
    for (int i = 0; i < NV; ++i) *reinterpret_cast<u32x4*>(t + vdst[i]) = s.v[i];
  };

  f32x4 oacc[RB][DB + 1];
  f32x4 negm[RB];       // -m in every element: the S^T accumulator's initial value
  float mref[RB];       // running reference maximum (log2 units) of this lane's query
  float thr[RB];        // rescale threshold: -FLT_MAX until the first visible key
#pragma unroll
  for (int r = 0; r < RB; ++r) {
#pragma unroll
    for (int db = 0; db <= DB; ++db) oacc[r][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    negm[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    mref[r] = 0.0f;
    thr[r] = -__FLT_MAX__;
  }
  const u32x4 ones = u32x4{kOnes2<T>, kOnes2<T>, kOnes2<T>, kOnes2<T>};

  auto compute = [&](int b, int t) {
    const uint16_t* sk = tiles + b * BUF;
    const uint16_t* sv = sk + SKT;
    const int k0 = kbeg + t * BN;
    u32x4 kf[KB][KSD];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int ks = 0; ks < KSD; ++ks)
        kf[kb][ks] = *reinterpret_cast<const u32x4*>(sk + (kb * 16 + col) * KP + ks * 32 + g * 8);
    f32x4 st[RB][KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        st[r][kb] = mfma16x16x32<T>(kf[kb][0], qf[r][0], negm[r]);
#pragma unroll
        for (int ks = 1; ks < KSD; ++ks) st[r][kb] = mfma16x16x32<T>(kf[kb][ks], qf[r][ks], st[r][kb]);
      }
    // V^T fragments: rows (keys) ks2*32 + 4g + (col >> 2) (+16), columns db*16 + 4 (col & 3)
    u32x4 vf[DB][BN / 32];
#pragma unroll
    for (int ks2 = 0; ks2 < BN / 32; ++ks2)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint16_t* a = sv + (ks2 * 32 + 4 * g + (col >> 2)) * VP + db * 16 + 4 * (col & 3);
        const u32x2 lo = lds_read_tr16(a);
        const u32x2 hi = lds_read_tr16(a + 16 * VP);
        vf[db][ks2] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
    if (!(k0 + BN <= klim && (!p.causal || k0 + BN - 1 <= row0))) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int lim = p.causal ? min(klim - 1, qi[r]) : klim - 1;   // last visible key
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            st[r][kb][i] = k0 + kb * 16 + 4 * g + i <= lim ? st[r][kb][i] : kNegInf;
      }
    }
    float mt[RB];
    bool need_any = false;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      mt[r] = max_over_g(max_tile<KB>(st[r]));
      need_any = need_any || mt[r] > thr[r];
    }
    if (__builtin_amdgcn_ballot_w64(need_any) != 0) {
      __asm__ volatile("" ::: "memory");
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const bool need = mt[r] > thr[r];
        const float delta = need ? mt[r] : 0.0f;
        const float alpha = need && thr[r] > 0.0f ? fast_exp2(-delta) : 1.0f;
#pragma unroll
        for (int db = 0; db <= DB; ++db) oacc[r][db] *= alpha;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) st[r][kb] -= delta;
        mref[r] += delta;
        negm[r] = f32x4{-mref[r], -mref[r], -mref[r], -mref[r]};
        thr[r] = need ? 8.0f : thr[r];
      }
    }
    u32x4 pf[RB][BN / 32];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        // reduction index 8g + j: key 4g + j of block 2 ks2 (j < 4), 4g + j - 4 of block 2 ks2 + 1
        pf[r][kb >> 1][(kb & 1) * 2] = pack2<T>(fast_exp2(st[r][kb][0]), fast_exp2(st[r][kb][1]));
        pf[r][kb >> 1][(kb & 1) * 2 + 1] = pack2<T>(fast_exp2(st[r][kb][2]), fast_exp2(st[r][kb][3]));
      }
#pragma unroll
    for (int ks2 = 0; ks2 < BN / 32; ++ks2)
#pragma unroll
      for (int r = 0; r < RB; ++r) {
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[r][db] = mfma16x16x32<T>(vf[db][ks2], pf[r][ks2], oacc[r][db]);
        oacc[r][DB] = mfma16x16x32<T>(ones, pf[r][ks2], oacc[r][DB]);
      }
  };

  // group tile sequence grp + KS j; steps padded to even so the loop body
  // (two steps, one per LDS buffer) has no exit and the same loads on every path
  const int nsteps = (ntiles + KS - 1) / KS;
  const int nsteps2 = (nsteps + 1) & ~1;
  Stage sa, sb;
  gload(0, sa);
  gload(1, sb);
  lstore(sa, 0);
  gload(2, sa);
  lds_barrier();
  for (int j = 0; j < nsteps2; j += 2) {
    if (grp + KS * j < ntiles) compute(0, grp + KS * j);
    lstore(sb, 1);
    gload(j + 3, sb);
    lds_barrier();
    if (grp + KS * (j + 1) < ntiles) compute(1, grp + KS * (j + 1));
    lstore(sa, 0);
    gload(j + 4, sa);
    lds_barrier();
  }

  float mfin[RB], lfin[RB];
  if constexpr (KS > 1) {
    float* so = reinterpret_cast<float*>(smem);   // [KS][64 rows][MP]
    float* ssum = so + KS * BM * MP;              // [KS][64 rows]
    float* smax = ssum + KS * BM;                 // [KS][64 rows]
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int row = (wave * RB + r) * 16 + col;
#pragma unroll
      for (int db = 0; db < DB; ++db) *reinterpret_cast<f32x4*>(&so[(grp * BM + row) * MP + db * 16 + 4 * g]) = oacc[r][db];
      if (g == 0) {
        ssum[grp * BM + row] = oacc[r][DB][0];
        smax[grp * BM + row] = thr[r] > 0.0f ? mref[r] : kNegInf;
      }
    }
    lds_barrier();
    if (grp != 0) return;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int row = (wave * RB + r) * 16 + col;
      float M = kNegInf;
#pragma unroll
      for (int s = 0; s < KS; ++s) M = fmaxf(M, smax[s * BM + row]);
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[r][db] = f32x4{0.f, 0.f, 0.f, 0.f};
      float L = 0.0f;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const float ms = smax[s * BM + row];
        const float f = ms == kNegInf ? 0.0f : fast_exp2(ms - M);
        L = fmaf(ssum[s * BM + row], f, L);
#pragma unroll
        for (int db = 0; db < DB; ++db)
          oacc[r][db] += *reinterpret_cast<const f32x4*>(&so[(s * BM + row) * MP + db * 16 + 4 * g]) * f;
      }
      mfin[r] = M;
      lfin[r] = L;
    }
  } else {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      mfin[r] = thr[r] > 0.0f ? mref[r] : kNegInf;
      lfin[r] = oacc[r][DB][0];
    }
  }

  const int nqt = (p.q_len + BM - 1) / BM;
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    if (qi[r] >= p.q_len) continue;
    const float inv = 1.0f / lfin[r];
    if (nchunks == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
        store4<T>(p.out, (size_t)qi[r] * p.out_stride + (size_t)h * D + db * 16 + 4 * g, oacc[r][db] * inv,
                  p.out_dtype);
    } else {
      const size_t unit = ((size_t)h * nqt + qt) * p.max_chunks + chunk;
      const int row = qi[r] - qt * BM;
      float* po = p.part_o + (unit * BM + row) * D;
#pragma unroll
      for (int db = 0; db < DB; ++db) *reinterpret_cast<f32x4*>(po + db * 16 + 4 * g) = oacc[r][db] * inv;
      if (g == 0) {
        p.part_ml[(unit * BM + row) * 2] = mfin[r];
        p.part_ml[(unit * BM + row) * 2 + 1] = lfin[r];
      }
    }
  }
}

// Merge the key-chunk partials of query tiles that were split.  grid (Hq, nqt),
// 256 threads: thread (row, quarter) merges 16 output dims of one query row.
// Chunks are read four at a time with every load of a batch issued together
// (indexes past the last chunk re-read it and are dropped), so a merge of up to
// four chunks is one round trip.
template <int D>
__global__ void __launch_bounds__(256) prefill_merge_kernel(const PrefillParams p) {
  constexpr int BM = kPrefillBM;
  constexpr int DQ = D / 4;        // dims per thread
  constexpr int NV = DQ / 4;       // float4 per thread
  const int h = blockIdx.x;
  const int qt = blockIdx.y;
  const int nchunks = (prefill_key_tiles(p, qt) + p.chunk_tiles - 1) / p.chunk_tiles;
  if (nchunks <= 1) return;
  const int nqt = (p.q_len + BM - 1) / BM;
  const size_t unit0 = ((size_t)h * nqt + qt) * p.max_chunks;
  const int row = threadIdx.x >> 2;
  const int d0 = (threadIdx.x & 3) * DQ;
  const int qi = qt * BM + row;
  if (qi >= p.q_len) return;
  float M = kNegInf;
  for (int c0 = 0; c0 < nchunks; c0 += 4) {
    float mv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) mv[u] = p.part_ml[((unit0 + min(c0 + u, nchunks - 1)) * BM + row) * 2];
#pragma unroll
    for (int u = 0; u < 4; ++u) M = fmaxf(M, mv[u]);
  }
  const float Mu = M == kNegInf ? 0.0f : M;
  f32x4 num[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) num[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float den = 0.0f;
  for (int c0 = 0; c0 < nchunks; c0 += 4) {
    float2 ml[4];
    f32x4 o[4][NV];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const size_t r = (unit0 + min(c0 + u, nchunks - 1)) * BM + row;
      ml[u] = *reinterpret_cast<const float2*>(p.part_ml + r * 2);
#pragma unroll
      for (int i = 0; i < NV; ++i) o[u][i] = *reinterpret_cast<const f32x4*>(p.part_o + r * D + d0 + 4 * i);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (c0 + u >= nchunks) break;
      const float w = ml[u].y * fast_exp2(ml[u].x - Mu);
      den += w;
#pragma unroll
      for (int i = 0; i < NV; ++i) num[i] += o[u][i] * w;
    }
  }
  const float inv = 1.0f / den;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (p.out_dtype == kBF16)
      store4<__bf16>(p.out, (size_t)qi * p.out_stride + (size_t)h * D + d0 + 4 * i, num[i] * inv, p.out_dtype);
    else   // f16 or f32 (store4 writes f32 for kF32 whatever T is)
      store4<_Float16>(p.out, (size_t)qi * p.out_stride + (size_t)h * D + d0 + 4 * i, num[i] * inv, p.out_dtype);
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
  // 32-bit buffer offsets inside one 64-row key tile
  const bool small_stride = p.k_stride < (1ll << 24) && p.v_stride < (1ll << 24);
  return (dtype == kF16 || dtype == kBF16) && p.head_dim == p.head_dim_v &&
         (p.head_dim == 64 || p.head_dim == 128) && aligned && small_stride;
}

size_t prefill_workspace_bytes(const PrefillParams& p, int dtype) {
  if (!prefill_uses_mfma(p, dtype)) return 0;
  int units, max_chunks;
  prefill_units(p, units, max_chunks);
  if (max_chunks <= 1) return 0;
  const size_t nqt = (p.q_len + kPrefillBM - 1) / kPrefillBM;
  return (size_t)p.num_heads * nqt * max_chunks * kPrefillBM * (p.head_dim + 2) * sizeof(float);
}

// Key tiles of the last query tile (the longest causal row), host side.
int prefill_key_tiles_host(const PrefillParams& p, int qt) {
  const int kend = p.causal ? std::min(p.kv_len, (qt + 1) * kPrefillBM) : p.kv_len;
  return (kend + kPrefillBN - 1) / kPrefillBN;
}

// head_dim 64 kernel shapes (16-row waves): 0 = 2 key groups of 64-key tiles
// (512 threads); 1 = 1 key group (256 threads); 2 = 2 key groups of 32-key
// tiles (512 threads).
template <typename T> void launch_fa(int cfg, dim3 grid, const PrefillParams& pp, hipStream_t stream) {
#ifdef TV_PREFILL_FIXED
  (void)cfg;
  hipLaunchKernelGGL((prefill_fa_kernel<T, 64, TV_PREFILL_RB, TV_PREFILL_KS, TV_PREFILL_FA_BN>), grid,
                     dim3(256 / TV_PREFILL_RB * TV_PREFILL_KS), 0, stream, pp);
#else
  if (cfg == 0) hipLaunchKernelGGL((prefill_fa_kernel<T, 64, 1, 2, 64>), grid, dim3(512), 0, stream, pp);
  else if (cfg == 2) hipLaunchKernelGGL((prefill_fa_kernel<T, 64, 1, 2, 32>), grid, dim3(512), 0, stream, pp);
  else hipLaunchKernelGGL((prefill_fa_kernel<T, 64, 1, 1, 64>), grid, dim3(256), 0, stream, pp);
#endif
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
    const bool d64 = pp.head_dim == 64;
    const dim3 grid(pp.num_heads, units);
#ifdef TV_PREFILL_V1
    constexpr int KSP = TV_PREFILL_KSPLIT;
    const dim3 block(256 * KSP);
    if (dtype == kF16) {
      if (d64) hipLaunchKernelGGL((prefill_mfma_kernel<_Float16, 64, KSP>), grid, block, 0, stream, pp);
      else hipLaunchKernelGGL((prefill_mfma_kernel<_Float16, 128, 1>), grid, dim3(256), 0, stream, pp);
    } else {
      if (d64) hipLaunchKernelGGL((prefill_mfma_kernel<__bf16, 64, KSP>), grid, block, 0, stream, pp);
      else hipLaunchKernelGGL((prefill_mfma_kernel<__bf16, 128, 1>), grid, dim3(256), 0, stream, pp);
    }
#else
    if (d64) {
      // Rows of 8+ key tiles on a grid of fewer than 4 work-groups per CU:
      // two key groups of 4 waves halve the longest chain; between one and
      // four per CU also 32-key tiles (smaller registers: 4 waves per SIMD
      // instead of 2).  Otherwise 4 waves, no split and no merge.  (Measured
      // at Hq 32: L = 64 / 256 / 512 / 1024 / 2048 take 4.2 / 5.9 / 7.9 / 13.6 /
      // 35 us; 32-row waves and 4 key groups were slower at every length.)
      const long long wgs = (long long)grid.x * grid.y;
      const bool long_rows = prefill_key_tiles_host(pp, (pp.q_len + kPrefillBM - 1) / kPrefillBM - 1) >= 8;
      const int cfg = long_rows && wgs <= 256 ? 0 : (long_rows && wgs < 1024 ? 2 : 1);
      if (dtype == kF16) launch_fa<_Float16>(cfg, grid, pp, stream);
      else launch_fa<__bf16>(cfg, grid, pp, stream);
    } else if (dtype == kF16) {
      hipLaunchKernelGGL((prefill_mfma_kernel<_Float16, 128, 1>), grid, dim3(256), 0, stream, pp);
    } else {
      hipLaunchKernelGGL((prefill_mfma_kernel<__bf16, 128, 1>), grid, dim3(256), 0, stream, pp);
    }
#endif
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
