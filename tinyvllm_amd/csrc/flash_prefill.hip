// Causal / full attention over one prompt ("flash prefill") for gfx950.
//
// Semantics follow tinyvllm/model/llama.py:58-94: q [Lq, Hq, D], k [Lk, Hkv, D],
// v [Lk, Hkv, Dv]; scores (q.k)*scale; with `causal`, key j is excluded for query
// i when j > i (top-left aligned, llama.py:86-90); query head h reads KV head
// h / (Hq/Hkv).  Every query row keeps key 0, so the reference's -1e9 additive
// mask and the exclusion used here give the same softmax.
//
// Kernels:
//  * prefill_fa_kernel<T, D, RB, KS, BN>: fp16/bf16, D in {64, 128}, Dv == D.
//    A work-group owns 64 query rows of one head; KS groups of waves split the
//    row block's BN-key tiles.  Scores are computed transposed, S^T = K Q^T,
//    with v_mfma_f32_16x16x32_{f16,bf16}; the accumulator layout of S^T (lane =
//    query column, 4 consecutive keys per 16-key block) is exactly the
//    B-operand layout needed for O^T = V^T P^T once the two operands agree on
//    the order of the reduction index, so P never leaves registers.
//  * prefill_merge_kernel<D>: merges rows split into key chunks.
//  * prefill_generic_kernel<T>: any D, Dv <= 256, any element type (fp32 path and
//    odd head sizes).  One wave per (query row, head); 64 keys per step.
#include "tv_common.h"
#include "tv_paged_keys.h"
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
constexpr int kPrefillBN = 64;   // keys per unit of the chunking and of prefill_key_tiles

// Key tiles query tile qt needs (causal rows stop at the diagonal).
__device__ __forceinline__ int prefill_key_tiles(const PrefillParams& p, int qt) {
  const int kend = prefill_unit_key_end(p.causal != 0, p.kv_len, qt, kPrefillBM, p.q_pos_offset);
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

// Store 4 quiet NaNs as out_dtype, as bit patterns written by integer stores:
// the prefill kernels are compiled without NaN semantics, so a NaN produced by
// floating-point arithmetic there is undefined.
__device__ __forceinline__ void store4_nan(void* base, size_t idx, int out_dtype) {
  if (out_dtype == kF32) {
    *reinterpret_cast<u32x4*>(reinterpret_cast<uint32_t*>(base) + idx) =
        u32x4{0x7FC00000u, 0x7FC00000u, 0x7FC00000u, 0x7FC00000u};
  } else {
    const uint32_t w = out_dtype == kF16 ? 0x7E007E00u : 0x7FC07FC0u;
    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(base) + idx) = u32x2{w, w};
  }
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

// ---------------------------------------------------------------------------
// MFMA kernel: register-lean softmax, double-buffered tiles
// ---------------------------------------------------------------------------
//
// A work-group owns 64 query rows of one head.  KS groups of QW = 4 / RB waves
// split the row block's BN-key tiles (group s takes tiles s + KS j of its key
// range); every wave owns RB blocks of 16 query rows, so each K / V fragment
// read from LDS feeds RB matrix products.  Per tile a wave computes S^T = K Q^T
// and brings the scores into the log2 domain relative to m, the running
// reference maximum of the query (for fp16 inside the matrix cores, with Q
// pre-scaled and the accumulator initialised to -m; for bf16 with one fp32 fma
// per score, see kPreScaleQ), so they go straight into v_exp_f32.  m is
// raised only when a tile exceeds it by more than 8, which after the first
// tile is rare.  V is staged row-major in LDS and read as the V^T operand with
// ds_read_b64_tr_b16; the softmax row sums come from one extra MFMA of P
// against a register of ones.  (Row sums by v_dot2 on the VALU instead, as
// the 128-row kernel does, measured 2-8% slower here: TinyLlama heads L 512 /
// 1024 7.97 / 13.5 against 8.13 / 13.8 us, both in one launch 15.1 against
// 15.7, a 512-row chunk over 3584 cached tokens 30.7 against 31.4 -- the matrix
// pipe has room, the VALU path of a step does not.)  Tiles are double-buffered in LDS
// and loaded two steps ahead through buffer loads whose range ends at the last
// key row (rows past kv_len read as zero), one barrier per step.

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

constexpr int kPrefillWavesPerEu = 2;   // occupancy the VGPR budget of the 64-row kernel allows

template <typename T, int D, int RB, int KS, int BN, bool PAGED>
__global__ void __launch_bounds__(256 / RB * KS) __attribute__((amdgpu_waves_per_eu(kPrefillWavesPerEu)))
prefill_fa_kernel(const PrefillParams pa) {
  // Several prompts per launch: this work-group's prompt is seq_order[blockIdx.z];
  // its rows become the whole problem (pointers and lengths rebased).  Chunked
  // key splits are off then, so a query tile is one unit and units past the
  // prompt's tiles have nothing to do.
  PrefillParams p = pa;
  if (pa.cu_q) {
    const int z = pa.seq_order ? pa.seq_order[blockIdx.z] : (int)blockIdx.z;
    const int q0 = pa.cu_q[z], k0 = pa.cu_k[z];
    p.q_len = pa.cu_q[z + 1] - q0;
    p.kv_len = pa.cu_k[z + 1] - k0;
    if ((int)blockIdx.y * kPrefillBM >= p.q_len || p.kv_len <= 0) return;
    p.q = reinterpret_cast<const T*>(pa.q) + (size_t)q0 * pa.q_stride;
    p.k = reinterpret_cast<const T*>(pa.k) + (size_t)k0 * pa.k_stride;
    p.v = reinterpret_cast<const T*>(pa.v) + (size_t)k0 * pa.v_stride;
    p.out = reinterpret_cast<char*>(pa.out) + (size_t)q0 * pa.out_stride * (pa.out_dtype == kF32 ? 4 : 2);
  }
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
  const int qoff = p.q_pos_offset;
  const int kend = prefill_unit_key_end(p.causal != 0, klim, qt, BM, qoff);
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
      for (int ks = 0; ks < KSD; ++ks) {
        const u32x4 raw = qi[r] < p.q_len ? *reinterpret_cast<const u32x4*>(qg + (size_t)qi[r] * p.q_stride + ks * 32 + g * 8)
                                          : u32x4{0, 0, 0, 0};
        qf[r][ks] = kPreScaleQ<T> ? scale8<T>(raw, c) : raw;
      }
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
    if constexpr (PAGED) {
      koff[i] = row;            // row of the tile and element column: the cache row comes from the table
      voff[i] = ch * 8;
    } else {
      koff[i] = (int)(row * p.k_stride + ch * 8) * (int)sizeof(T);
      voff[i] = (int)(row * p.v_stride + ch * 8) * (int)sizeof(T);
    }
    kdst[i] = row * KP + ch * 8;
    vdst[i] = SKT + row * VP + ch * 8;
  }
  // paged prompt: the block ids of keys [kbeg, kend) in LDS
  __shared__ int stbl[PAGED ? kPagedTableMax : 1];
  const int lg = p.kv_bs_log2;
  const int blk0 = kbeg >> lg;
  __shared__ int sbad;
  bool bad = false;
  const int kstage = paged_stage_end(kbeg, kend);   // keys whose block ids are staged: [kbeg, kstage)
  if constexpr (PAGED) {
    const int nblk = paged_staged_blocks(kbeg, kstage, lg);
    if (threadIdx.x == 0) sbad = 0;
    lds_barrier();
    for (int i = threadIdx.x; i < nblk; i += blockDim.x) {
      const int b = p.kv_table[blk0 + i];
      const bool ok = (unsigned)b < (unsigned)p.kv_num_blocks;
      stbl[i] = ok ? b : 0;                   // an invalid id reads block 0 (in bounds) ...
      if (!ok) sbad = 1;
    }
    lds_barrier();
    bad = sbad != 0;                          // ... and the head's outputs become NaN
  }
  struct Stage {
    u32x4 k[NV], v[NV];
  };
  auto tile_of = [&](int j) { return prefill_group_tile(grp, KS, j, ntiles); };
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
    if constexpr (PAGED) {
      // keys at or past kend (masked for every row of the unit) re-read the
      // last staged key: the table is in LDS for keys [kbeg, kend) only
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int key = paged_load_key(kbeg, kstage, (int)t, BN, koff[i]);
        const long long row = ((long long)stbl[paged_stage_slot(key, kbeg, lg)] << lg) + (key & ((1 << lg) - 1));
        s.k[i] = *reinterpret_cast<const u32x4*>(kbase + row * p.k_stride + voff[i]);
        s.v[i] = *reinterpret_cast<const u32x4*>(vbase + row * p.v_stride + voff[i]);
      }
    } else {
      const unsigned long long ko = t * kstep, vo = t * vstep;
      const __amdgpu_buffer_rsrc_t rk = make_rsrc(kfirst + ko, kbytes - ko);
      const __amdgpu_buffer_rsrc_t rv = make_rsrc(vfirst + vo, vbytes - vo);
#pragma unroll
      for (int i = 0; i < NV; ++i) s.k[i] = buffer_load16(rk, koff[i], 0);
#pragma unroll
      for (int i = 0; i < NV; ++i) s.v[i] = buffer_load16(rv, voff[i], 0);
    }
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
  u32x4 ones = u32x4{kOnes2<T>, kOnes2<T>, kOnes2<T>, kOnes2<T>};

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
    if constexpr (!kPreScaleQ<T>) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[r][kb][i] = fmaf(st[r][kb][i], c, -mref[r]);
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
    if (!(k0 + BN <= klim && (!p.causal || k0 + BN - 1 <= row0 + qoff))) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        // last visible key, relative to this lane's first key k0 + 4 g: each
        // element is then one compare against a constant and one select
        const int rel = (p.causal ? min(klim - 1, qi[r] + qoff) : klim - 1) - (k0 + 4 * g);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            st[r][kb][i] = kb * 16 + i <= rel ? st[r][kb][i] : kNegInf;
      }
    }
    // Each lane tests its own keys against the threshold; a query's maximum
    // over the tile exceeds it exactly when one of its four lanes' does, so
    // the cross-lane maximum is only formed on the (rare) rescale path.
    float lm[RB];
    bool need_any = false;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      lm[r] = max_tile<KB>(st[r]);
      need_any = need_any || lm[r] > thr[r];
    }
    if (__builtin_amdgcn_ballot_w64(need_any) != 0) {
      __asm__ volatile("" ::: "memory");
      float mt[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) mt[r] = max_over_g(lm[r]);
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
        if constexpr (kPreScaleQ<T>) negm[r] = f32x4{-mref[r], -mref[r], -mref[r], -mref[r]};
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
    // opaque to the optimiser: keeps the ones vector in its registers across
    // steps instead of rebuilding it (three moves) after they are reused
    __asm__ volatile("" : "+v"(ones));
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
      for (int db = 0; db < DB; ++db) {
        const size_t idx = (size_t)qi[r] * p.out_stride + (size_t)h * D + db * 16 + 4 * g;
        if (bad) store4_nan(p.out, idx, p.out_dtype);    // a block id outside the cache
        else store4<T>(p.out, idx, oacc[r][db] * inv, p.out_dtype);
      }
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
    const int kend = prefill_unit_key_end(p.causal != 0, p.kv_len, qt, kPrefillBM, p.q_pos_offset);
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

// 128-row work-groups with LDS-DMA tiles (prefill_rows_kernel,
// flash_prefill_rows.hip) for long head_dim-128 prompts, where they measured
// faster (MI355X, Hq 32 / Hkv 8: L 2048 54-56 against 64-68 us, L 4096
// 174 against 207-210); below 2048 rows, or at head_dim 64, this file's 64-row
// kernel wins.
constexpr int kRowsMinLen = 2048;

bool use_rows_kernel(int head_dim, long long max_q_len) { return head_dim == 128 && max_q_len >= kRowsMinLen; }

size_t prefill_workspace_bytes(const PrefillParams& p, int dtype) {
  if (!prefill_uses_mfma(p, dtype)) return 0;
  int units, max_chunks;
  prefill_units(p, units, max_chunks);
  if (max_chunks <= 1) return use_rows_kernel(p.head_dim, p.q_len) ? prefill_rows_workspace_bytes(p, dtype) : 0;
  const size_t nqt = (p.q_len + kPrefillBM - 1) / kPrefillBM;
  return (size_t)p.num_heads * nqt * max_chunks * kPrefillBM * (p.head_dim + 2) * sizeof(float);
}

// Key tiles of the last query tile (the longest causal row), host side.
int prefill_key_tiles_host(const PrefillParams& p, int qt) {
  const int kend = prefill_unit_key_end(p.causal != 0, p.kv_len, qt, kPrefillBM, p.q_pos_offset);
  return (kend + kPrefillBN - 1) / kPrefillBN;
}

// Kernel shapes (16-row waves): 0 = 2 key groups (512 threads) of 64-key
// tiles at head_dim 64, 32-key tiles at 128; 1 = 1 key group (256 threads) of
// 64-key tiles at head_dim 64, 32-key at 128; 2 = 2 key groups of 32-key tiles.
template <typename T, int D, bool PAGED = false>
void launch_fa(int cfg, dim3 grid, const PrefillParams& pp, hipStream_t stream) {
  constexpr int BN = D == 64 ? 64 : 32;
  if constexpr (D == 64) {
    if (cfg == 3) {
      hipLaunchKernelGGL((prefill_fa_kernel<T, D, 1, 4, 32, PAGED>), grid, dim3(1024), 0, stream, pp);
      return;
    }
  }
  if (cfg == 0 || cfg == 3) hipLaunchKernelGGL((prefill_fa_kernel<T, D, 1, 2, BN, PAGED>), grid, dim3(512), 0, stream, pp);
  else if (cfg == 2) hipLaunchKernelGGL((prefill_fa_kernel<T, D, 1, 2, 32, PAGED>), grid, dim3(512), 0, stream, pp);
  else hipLaunchKernelGGL((prefill_fa_kernel<T, D, 1, 1, BN, PAGED>), grid, dim3(256), 0, stream, pp);
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
    if (max_chunks == 1 && use_rows_kernel(pp.head_dim, pp.q_len)) {
      // the key-half split needs the workspace; without one the prompt runs
      // unsplit (a workspace smaller than asked for is the caller's error)
      const size_t need = prefill_rows_workspace_bytes(pp, dtype);
      if (need && workspace && workspace_bytes < need) return 2;
      if (launch_prefill_rows(pp, dtype, 1, pp.q_len, need ? workspace : nullptr, stream)) return 0;
    }
    if (max_chunks > 1) {
      const size_t need = prefill_workspace_bytes(pp, dtype);
      if (!workspace || workspace_bytes < need) return 2;
      const size_t nqt = (pp.q_len + kPrefillBM - 1) / kPrefillBM;
      pp.part_o = reinterpret_cast<float*>(workspace);
      pp.part_ml = pp.part_o + (size_t)pp.num_heads * nqt * max_chunks * kPrefillBM * pp.head_dim;
    }
    const bool d64 = pp.head_dim == 64;
    const dim3 grid(pp.num_heads, units);
    // Rows of 8+ key tiles on a grid of fewer than 4 work-groups per CU: two
    // key groups of 4 waves halve the longest chain; between one and four per
    // CU (head_dim 64) also 32-key tiles (fewer registers: 4 waves per SIMD
    // instead of 2).  Otherwise 4 waves, no split and no merge.  (Measured at
    // Hq 32, head_dim 64: L = 64 / 256 / 512 / 1024 / 2048 take 4.2 / 5.9 /
    // 7.9 / 13.6 / 35 us; 32-row waves and 4 key groups were slower at every
    // length.  Head_dim 128, Hkv 8, 32-key tiles: L = 512 / 1024 / 2048 take
    // 11.9 / 24.6 / 62.9 us; two key groups at L = 1024 took 28.6.)
    const long long wgs = (long long)grid.x * grid.y;
    const bool long_rows = prefill_key_tiles_host(pp, (pp.q_len + kPrefillBM - 1) / kPrefillBM - 1) >= 8;
    const int cfg = long_rows && wgs <= 256 ? 0 : (d64 && long_rows && wgs < 1024 ? 2 : 1);
    if (dtype == kF16) {
      if (d64) launch_fa<_Float16, 64>(cfg, grid, pp, stream);
      else launch_fa<_Float16, 128>(cfg, grid, pp, stream);
    } else {
      if (d64) launch_fa<__bf16, 64>(cfg, grid, pp, stream);
      else launch_fa<__bf16, 128>(cfg, grid, pp, stream);
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

// One prompt whose keys and values are read through a block table
// (kv_table set) with query rows at positions q_pos_offset ..: the 64-row
// kernel with its loads going through the table.  Returns 1 when the shape has
// no such kernel (fp32, head_dim other than 64 / 128, a block size that is
// not a power of two, or more than kPagedTableMax blocks).
int launch_flash_prefill_paged(const PrefillParams& p_in, int dtype, hipStream_t stream) {
  PrefillParams pp = p_in;
  if (!prefill_uses_mfma(pp, dtype) || !pp.kv_table || pp.kv_bs_log2 < 0 || pp.kv_bs_log2 > 20) return 1;
  if (((long long)pp.kv_len + (1LL << pp.kv_bs_log2) - 1) >> pp.kv_bs_log2 > kPagedTableMax) return 1;
  pp.xcd_remap = (pp.num_heads % 8 == 0) ? 1 : 0;
  pp.chunk_tiles = 1 << 20;
  int units, max_chunks;
  prefill_units(pp, units, max_chunks);
  pp.max_chunks = 1;
  const bool d64 = pp.head_dim == 64;
  const dim3 grid(pp.num_heads, units);
  const long long wgs = (long long)grid.x * grid.y;
  const bool long_rows = prefill_key_tiles_host(pp, (pp.q_len + kPrefillBM - 1) / kPrefillBM - 1) >= 8;
  // At head_dim 64 a one-per-CU grid of long rows takes four key groups of
  // 32-key tiles here (a 512-row chunk over 3584 cached tokens, TinyLlama
  // heads: 34.7 against 36.6 us with two groups of 64-key tiles); prompts
  // without a prefix keep two groups, which were faster at L = 512.
  int cfg = long_rows && wgs <= 256 ? 0 : (d64 && long_rows && wgs < 1024 ? 2 : 1);
  if (cfg == 0 && d64) cfg = 3;
  if (dtype == kF16) {
    if (d64) launch_fa<_Float16, 64, true>(cfg, grid, pp, stream);
    else launch_fa<_Float16, 128, true>(cfg, grid, pp, stream);
  } else {
    if (d64) launch_fa<__bf16, 64, true>(cfg, grid, pp, stream);
    else launch_fa<__bf16, 128, true>(cfg, grid, pp, stream);
  }
  return 0;
}

// Several prompts in one launch (MFMA path only): grid (Hq, query tiles of the
// longest prompt, prompts); the kernel shape is chosen as for one prompt of the
// longest length with the live work-groups of all prompts.  Returns 1 if the
// shape has no MFMA kernel.
int launch_flash_prefill_varlen(const PrefillParams& p_in, int num_seqs, int max_q_len, int max_kv_len,
                                long long total_q, int dtype, hipStream_t stream) {
  PrefillParams pp = p_in;
  pp.q_len = max_q_len;
  pp.kv_len = max_kv_len;
  if (!prefill_uses_mfma(pp, dtype)) return 1;
  pp.xcd_remap = (pp.num_heads % 8 == 0) ? 1 : 0;
  pp.chunk_tiles = 1 << 20;
  pp.max_chunks = 1;
  pp.part_o = nullptr;
  pp.part_ml = nullptr;
  if (use_rows_kernel(pp.head_dim, max_q_len) &&
      launch_prefill_rows(pp, dtype, num_seqs, max_q_len, nullptr, stream))
    return 0;
  const int nqt = (max_q_len + kPrefillBM - 1) / kPrefillBM;
  const dim3 grid(pp.num_heads, nqt, num_seqs);
  const long long wgs = (long long)pp.num_heads * ((total_q + kPrefillBM - 1) / kPrefillBM + num_seqs);
  const bool d64 = pp.head_dim == 64;
  const bool long_rows = prefill_key_tiles_host(pp, nqt - 1) >= 8;
  // One prompt: the single-prompt choice.  Several: one key group of 4 waves
  // unless everything fits one work-group per CU -- the shorter prompts' work
  // groups fill the slots the long rows leave, so more resident work-groups
  // beat halving the longest chain (MI355X, fp16 D 64: L 512 + 1024 in 15.2
  // against 17.8 us with two key groups of 32-key tiles; 16 x 64 tokens 5.6
  // against 6.7; 1024 + 1024 + 512 + 256 22.7 against 26.9).
  const int cfg = long_rows && wgs <= 256 ? 0
                  : (num_seqs == 1 && d64 && long_rows && wgs < 1024 ? 2 : 1);
  if (dtype == kF16) {
    if (d64) launch_fa<_Float16, 64>(cfg, grid, pp, stream);
    else launch_fa<_Float16, 128>(cfg, grid, pp, stream);
  } else {
    if (d64) launch_fa<__bf16, 64>(cfg, grid, pp, stream);
    else launch_fa<__bf16, 128>(cfg, grid, pp, stream);
  }
  return 0;
}

}  // namespace tv
