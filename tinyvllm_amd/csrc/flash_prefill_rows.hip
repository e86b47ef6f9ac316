// Causal / full prefill attention for large grids: 128 query rows per
// work-group, 32 per wave, K/V tiles loaded straight into LDS.
//
// Same semantics as prefill_fa_kernel (flash_prefill.hip; reference
// tinyvllm/model/llama.py:58-94): scores (q.k)*scale, key j excluded for query
// i when j > i with `causal` (top-left aligned), query head h on KV head
// h / (Hq/Hkv), fp16 / bf16 inputs, fp32 accumulation.  Launched for head_dim
// 128 (the kernel body is written for any head_dim whose tile fills the DMA
// shape; at 64 the 64-row kernel was faster at every length measured).
//
// Why a second kernel.  In the 64-row kernel every wave owns 16 query rows, so
// each K / V byte read from LDS feeds 16 rows of MFMA work: at full matrix
// rate a CU would need ~256 B/clk of LDS reads, all the LDS has, and every
// tile also passes through VGPRs and ds_write_b128 on its way in.  Here:
//  * a wave owns 32 query rows (two 16-row blocks), so every K / V fragment
//    read from LDS feeds two MFMAs -- half the LDS read traffic per FLOP;
//  * the four waves of a work-group (128 rows) share each staged tile;
//  * tiles arrive by buffer_load_dwordx4 ... lds (each lane's 16 bytes land at
//    M0 + 16 * lane): no staging registers, no LDS write instructions;
//  * since such a load writes 1 KB contiguously, rows are not padded; instead
//    the 16-byte chunks of row r are XOR-permuted (chunk c at slot c ^ f(r)),
//    chosen so that both the 16-row K fragment reads (ds_read_b128) and the
//    transposing V reads (ds_read_b64_tr_b16) touch distinct banks;
//  * four tile buffers used as two pairs: a pair of tiles (64 keys) is
//    requested when the previous pair starts, and each pair is one step (one
//    barrier, one softmax over its 64 keys).
// The softmax is the 64-row kernel's: log2 domain, lazy rescale (threshold 8),
// P kept in registers as the B operand of O^T = V^T P^T.  Where the scale
// enters depends on the type (kPreScaleQ, tv_common.h): fp16 pre-scales Q by
// scale * log2(e) and starts the score accumulator at -m, so scores leave the
// matrix cores ready for exp2; bf16 keeps Q as given and applies
// s * scale * log2(e) - m in one fp32 fma after the product, the reference's
// order (llama.py:84).
// Row sums accumulate per lane as fp32 adds of the exponentials (before their
// rounding to T for the P V product) and are summed over the four lanes of a
// query at the end.  v_dot2 against ones on the packed P cannot issue beside
// the wave's in-flight MFMAs on gfx950; the adds can, and measured 2-3.5%
// faster at L 2048 / 8192 (1.5% slower at 4096).
//
// Measured on MI355X (Llama-3-8B heads, Hq 32 / Hkv 8, head_dim 128, fp16,
// causal): L 2048 54-56 us (51 us replayed in a graph) against 64-68 for the
// 64-row kernel, L 4096 174 against 207-210; at L <= 1024 and at head_dim 64
// the 64-row kernel is faster (L 512 / 1024 at head_dim 64: 7.6 / 13.0 us
// against 12.1 / 20.7), so the launcher uses this one only for long
// head_dim-128 prompts.  A tile step of the longest work-group takes ~2000
// cycles against 512 of MFMA work (clock stamps): the LDS-DMA issue, LDS read
// issue, score wait and softmax are serial within a wave, and with 2 waves per
// SIMD (236 VGPRs fp16, 230 bf16) little of it overlaps.  Splitting a work-group's key tiles
// over two 4-wave groups in ping-pong (one group's MFMA phase against the
// other's softmax phase, a barrier per phase) was correct but 2x slower: the
// softmax phase of one wave ran ~4x longer while the other issued MFMAs.
// Balancing the causal work by pairing query tiles i and nqt-1-i was correct
// but no faster at L 2048: split over the two 4-wave groups of one 8-wave
// work-group (both waves of a SIMD then pass the same barrier, in phase) or
// run back to back by one work-group (one work-group per CU leaves one wave
// per SIMD, ~1.1 us per tile step against ~1.5 us for two waves' steps
// together).  Nor did balancing inside each wave (16 rows of 64-row tile i and
// 16 of tile n - 1 - i, the first block skipped past its diagonal; every
// work-group the same causal work, 2 per CU): 59.3 / 211 us at L 2048 / 4096
// against 57.1 / 192.  The work-group holding the last rows still walks every
// key tile (64 at L 2048), and a one-block step beside another work-group
// costs about what a two-block step costs alone, so the longest chain of
// steps, not the total work, sets the time.  Two independent work-groups per
// CU, drifting out of phase, are what keeps the matrix pipes busiest here.
//
// Where the time goes (L 2048 / 4096 / 8192, same heads).  Copies of this
// kernel that skip work, timed: without the K and V fragment reads from LDS no
// faster (LDS bandwidth is not the limit); without the tile loads into LDS 15-20%
// faster (53 / 163 / 515 us against 62 / 202 / 645 us).  Requesting the tiles
// four ahead instead of three (five buffers, 2 x 80 KB per CU) changes nothing,
// and the tile descriptors advanced by 64-bit adds instead of recomputed with
// 64-bit multiplies gave ~3% (about 50 fewer scalar instructions per step).  L2
// serves the K / V re-reads (95.6% hit rate at L 8192; FETCH_SIZE about the
// unique input bytes).  A software-pipelined form -- the scores of tile j + 1
// formed while tile j's softmax runs, exponentials and V reads interleaved
// between the score and P V products with sched_group_barrier, O kept in one
// register set by sending every tile through one code path -- was correct and
// cut the waits for LDS data 3x, but the time moved to the barrier: 63 / 200 /
// 635 us against 60 / 198 / 630 us.
#include "tv_common.h"
#include "tv_params.h"
#include "tv_device_cache.h"
#include "tv_paged_keys.h"
#include "tv_tile_dma.h"

#include <type_traits>

namespace tv {

namespace {

constexpr int kRowsBM = 128;   // query rows per work-group
constexpr int kRowsBN = 32;    // keys per tile
constexpr int kRowsBuf = 4;    // tile buffers: two pairs

}  // namespace

// Query tile of unit u.  Grids whose work-groups are all resident at once:
// zig-zag, the longer half of the causal tiles longest first, then the shorter
// half shortest first (dispatched a slot per CU at a time, so a CU's two
// work-groups hold a long and a short tile).  Larger grids: longest first, so
// the last work-groups to start are the shortest (MI355X, Llama-3-8B heads,
// fp16: L 2048 54.6 us zig-zag against 58.1 longest first; L 4096 174 against
// 188-191 and L 8192 562 against 598 longest first against zig-zag; ascending
// and alternating orders were slower at every length).
__device__ __forceinline__ int rows_unit_tile(int u, int nqt, bool longest_first) {
  if (longest_first) return nqt - 1 - u;
  const int half = (nqt + 1) / 2;
  return u < half ? nqt - 1 - u : u - half;
}

// Split halves are stored as fp32 unless the input and the output are fp16.
template <typename T>
__host__ __device__ constexpr bool rows_split_f32(int out_dtype) {
  return out_dtype == kF32 || !std::is_same_v<T, _Float16>;
}

template <typename T, int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
prefill_rows_kernel(const PrefillParams pa) {
  PrefillParams p = pa;
  if (pa.cu_q) {
    const int z = pa.seq_order ? pa.seq_order[blockIdx.z] : (int)blockIdx.z;
    const int q0 = pa.cu_q[z], k0 = pa.cu_k[z];
    p.q_len = pa.cu_q[z + 1] - q0;
    p.kv_len = pa.cu_k[z + 1] - k0;
    if ((int)blockIdx.y * kRowsBM >= p.q_len || p.kv_len <= 0) return;
    p.q = reinterpret_cast<const T*>(pa.q) + (size_t)q0 * pa.q_stride;
    p.k = reinterpret_cast<const T*>(pa.k) + (size_t)k0 * pa.k_stride;
    p.v = reinterpret_cast<const T*>(pa.v) + (size_t)k0 * pa.v_stride;
    p.out = reinterpret_cast<char*>(pa.out) + (size_t)q0 * pa.out_stride * (pa.out_dtype == kF32 ? 4 : 2);
  }
  constexpr int BM = kRowsBM, BN = kRowsBN, NB = kRowsBuf;
  constexpr int RB = 2;                    // 16-row blocks per wave
  constexpr int KB = BN / 16;              // 16-key blocks per tile
  constexpr int KSD = D / 32;              // MFMA steps over the head dim
  constexpr int DB = D / 16;               // 16-dim blocks of O^T
  constexpr int ROWB = 2 * D;              // bytes per tile row
  constexpr int TILEB = BN * ROWB;         // bytes of the K (or V) tile
  constexpr int BUFB = 2 * TILEB;          // one K + V buffer
  constexpr int NI = TILEB / 1024 / 4;     // LDS-DMA instructions per wave per tile, each of K and V
  constexpr int RPI = 1024 / ROWB;         // tile rows per DMA instruction
  constexpr int SPR = ROWB / 16;           // 16-byte chunks per row
  static_assert(NI >= 1 && NI * 4 * 1024 == TILEB, "tile / DMA shape");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NB * BUFB];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int col = lane & 15;

  const int h = p.xcd_remap ? ((int)(blockIdx.x & 7) * (p.num_heads >> 3) + (int)(blockIdx.x >> 3)) : (int)blockIdx.x;
  const int nqt = (p.q_len + BM - 1) / BM;
  int qt, half = -1;       // half: -1 the tile's whole key range, 0 / 1 its first / second half
  if (p.rows_split < nqt) rows_split_unit(blockIdx.y, nqt, p.rows_split, qt, half);
  else qt = rows_unit_tile(blockIdx.y, nqt, p.longest_first != 0);
  const int kvh = h / (p.num_heads / p.num_kv_heads);
  const int klim = p.kv_len;
  int kbeg, kend;          // this unit's keys
  rows_unit_keys(qt, half, p.causal ? min(klim, (qt + 1) * BM) : klim, kbeg, kend);
  const int ntiles = (kend - kbeg + BN - 1) / BN;
  const float c = p.scale * kLog2e;
  const int row0 = qt * BM + wave * 32;    // first query row of this wave

  // ---- Q fragments (B operand of S^T = K Q^T) ----
  int qi[RB];
  u32x4 qf[RB][KSD];
  {
    const T* qg = reinterpret_cast<const T*>(p.q) + (size_t)h * D;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      qi[r] = row0 + r * 16 + col;
#pragma unroll
      for (int ks = 0; ks < KSD; ++ks) {
        const u32x4 raw = qi[r] < p.q_len
                              ? *reinterpret_cast<const u32x4*>(qg + (size_t)qi[r] * p.q_stride + ks * 32 + g * 8)
                              : u32x4{0, 0, 0, 0};
        qf[r][ks] = kPreScaleQ<T> ? scale8<T>(raw, c) : raw;
      }
    }
  }

  // ---- LDS-DMA addressing: wave w loads instructions w*NI .. w*NI+NI-1 of each tile ----
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  const char* kbase = reinterpret_cast<const char*>(reinterpret_cast<const T*>(p.k) + (size_t)kvh * D);
  const char* vbase = reinterpret_cast<const char*>(reinterpret_cast<const T*>(p.v) + (size_t)kvh * D);
  const unsigned long long kstr = (unsigned long long)p.k_stride * sizeof(T);
  const unsigned long long vstr = (unsigned long long)p.v_stride * sizeof(T);
  uint32_t kvoff[NI], vvoff[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = (wave * NI + i) * RPI + lane / SPR;
    const int slot = lane % SPR;
    const int chunk = slot ^ tile_chunk_perm<D>(row);
    kvoff[i] = (uint32_t)(row * kstr + chunk * 16);
    vvoff[i] = (uint32_t)(row * vstr + chunk * 16);
  }
  // Tile t (keys kbeg + 32 t ..) into buffer t % NB.  Its K / V buffer
  // descriptors: base at the tile's first key row, range ending at the last
  // key row.  Tiles are requested in order t = 0, 1, 2, ...; each request
  // advances the descriptors by one tile (64-bit adds, no per-request
  // multiplies on the scalar unit), and from t = ntiles on the last tile is
  // requested again.
  unsigned long long ka = reinterpret_cast<unsigned long long>(kbase) + (unsigned long long)kbeg * kstr;
  unsigned long long va = reinterpret_cast<unsigned long long>(vbase) + (unsigned long long)kbeg * vstr;
  unsigned long long kr = (unsigned long long)(klim - 1 - kbeg) * kstr + D * sizeof(T);
  unsigned long long vr = (unsigned long long)(klim - 1 - kbeg) * vstr + D * sizeof(T);
  const unsigned long long kstep = (unsigned long long)BN * kstr;
  const unsigned long long vstep = (unsigned long long)BN * vstr;
  auto issue = [&](int t) {
    if (t > 0 && t < ntiles) {
      ka += kstep;
      kr -= kstep;
      va += vstep;
      vr -= vstep;
    }
    const u32x4 rk = rsrc_words(reinterpret_cast<const void*>(ka), kr);
    const u32x4 rv = rsrc_words(reinterpret_cast<const void*>(va), vr);
    const uint32_t buf = lds0 + (uint32_t)((t % NB) * BUFB);
#pragma unroll
    for (int i = 0; i < NI; ++i) load_lds16(rk, sgpr(buf + (uint32_t)((wave * NI + i) * 1024)), kvoff[i]);
#pragma unroll
    for (int i = 0; i < NI; ++i) load_lds16(rv, sgpr(buf + (uint32_t)(TILEB + (wave * NI + i) * 1024)), vvoff[i]);
  };

  // The Q loads are the only global loads the compiler tracks; retire them
  // here so its own wait for them cannot land inside the tile loop (where it
  // would also drain the LDS-DMA loads in flight).
  wait_vmcnt<0>();
  // Rows past kv_len read as zero through the resource range; the buffers start
  // zeroed so nothing non-finite can reach a masked product.
  for (int i = threadIdx.x; i < NB * BUFB / 16; i += 256) reinterpret_cast<u32x4*>(smem)[i] = u32x4{0, 0, 0, 0};
  lds_barrier();
  issue(0);
  issue(1);

  // fragment read offsets inside a buffer (bytes).  chunk_perm(r + 16) ==
  // chunk_perm(r), so the second 16-key block and the upper 16 V rows are the
  // same offsets plus a constant.  K chunk 4 ks + g of row col sits at slot
  // ((ks ^ fk) << 2) | (g ^ (f & 3)) with f = chunk_perm(col), fk = f >> 2; V
  // chunk 2 db + b of row r at ((db ^ fv) << 1) | (b ^ (f_r & 1)), fv = f_r >> 1:
  // one base and one XOR key per operand instead of a register per offset.
  const int kperm = tile_chunk_perm<D>(col);
  const int kofs0 = col * ROWB + ((g ^ (kperm & 3)) << 4);
  const int kkey = kperm >> 2;
  auto koff = [&](int ks) { return kofs0 + ((ks ^ kkey) << 6); };
  const int vrow = 4 * g + (col >> 2);
  const int vperm = tile_chunk_perm<D>(vrow);
  const int vofs0 = TILEB + vrow * ROWB + ((((col & 3) >> 1) ^ (vperm & 1)) << 4) + 8 * (col & 1);
  const int vkey = vperm >> 1;
  auto voff = [&](int db) { return vofs0 + ((db ^ vkey) << 5); };

  f32x4 oacc[RB][DB];
  float lpart[RB];      // this lane's share of the row sum (keys 4g..4g+3 of every 16)
  float mref[RB], thr[RB];
  f32x4 negm[RB];       // -m in every element: the fp16 score accumulator's initial value
#pragma unroll
  for (int r = 0; r < RB; ++r) {
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[r][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    lpart[r] = 0.0f;
    mref[r] = 0.0f;
    thr[r] = -__FLT_MAX__;
    negm[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // scores of a tile starting at key k0 -> log2 domain relative to the running
  // maximum (fp16: already, from the pre-scaled Q and the -m accumulator; bf16:
  // one fma), masked, rescaled when a row's maximum moved by more than 8
  auto softmax = [&](auto& st, int k0) {
    constexpr int NKB = std::extent<std::remove_reference_t<decltype(st)>, 1>::value;   // 16-key blocks
    if constexpr (!kPreScaleQ<T>) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[r][kb][i] = fmaf(st[r][kb][i], c, -mref[r]);
    }
    if (!(k0 + 16 * NKB <= kend && (!p.causal || k0 + 16 * NKB - 1 <= row0))) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int rel = (p.causal ? min(kend - 1, qi[r]) : kend - 1) - (k0 + 4 * g);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[r][kb][i] = kb * 16 + i <= rel ? st[r][kb][i] : kNegInf;
      }
    }
    float lm[RB];
    bool need_any = false;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      // a chain of three-input maxima (v_max3_f32): the 4 NKB values (an even
      // count) as one pair, then two more per step
      float t0 = fmaxf(st[r][0][0], st[r][0][1]);
#pragma unroll
      for (int j = 2; j < 4 * NKB; j += 2) t0 = fmaxf(t0, fmaxf(st[r][j >> 2][j & 3], st[r][(j + 1) >> 2][(j + 1) & 3]));
      lm[r] = t0;
      need_any = need_any || lm[r] > thr[r];
    }
    if (__builtin_amdgcn_ballot_w64(need_any) != 0) {
      __asm__ volatile("" ::: "memory");
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const float mt = max_over_g(lm[r]);
        const bool need = mt > thr[r];
        const float delta = need ? mt : 0.0f;
        const float alpha = need && thr[r] > 0.0f ? fast_exp2(-delta) : 1.0f;
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[r][db] *= alpha;
        lpart[r] *= alpha;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) st[r][kb] -= delta;
        mref[r] += delta;
        thr[r] = need ? 8.0f : thr[r];
        if constexpr (kPreScaleQ<T>) negm[r] = f32x4{-mref[r], -mref[r], -mref[r], -mref[r]};
      }
    }
  };

  const bool idle = row0 >= p.q_len;       // rows past the prompt: nothing to compute
  // Tiles in pairs (2s, 2s + 1), buffers 0-1 and 2-3 in turn, one step and
  // one barrier per pair: the barrier makes every wave's loads of the pair
  // visible and frees the previous pair's buffers, the next pair is requested
  // into them, then the pair's 64 keys go through one softmax -- score
  // products of both tiles, one maximum / rescale decision, P V per 32-key
  // half.  A second tile past the last one holds a re-request of the last
  // tile; its keys are past kend and the mask removes them.  (One barrier per
  // tile with tiles three ahead: 58.9 / 192 / 613 us at L 2048 / 4096 / 8192,
  // Llama-3-8B heads; a barrier per pair with a softmax per tile: 56.7 / 192 /
  // 610; one softmax per pair: 56.1 / 191 / 600.)
  auto step = [&](auto bufc, int jj) {
    constexpr int B = decltype(bufc)::value;
    wait_vmcnt<0>();
    lds_barrier();
    issue(jj + 2);
    issue(jj + 3);
    const int k0 = kbeg + jj * BN;
    if (idle || (p.causal && k0 > row0 + 31)) return;
    f32x4 st[RB][2 * KB];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint8_t* sb = smem + (B + hf) * BUFB;
      u32x4 kf[KB][KSD];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int ks = 0; ks < KSD; ++ks) kf[kb][ks] = *reinterpret_cast<const u32x4*>(sb + koff(ks) + kb * 16 * ROWB);
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          f32x4 a = mfma16x16x32<T>(kf[kb][0], qf[r][0], kPreScaleQ<T> ? negm[r] : f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int ks = 1; ks < KSD; ++ks) a = mfma16x16x32<T>(kf[kb][ks], qf[r][ks], a);
          st[r][hf * KB + kb] = a;
        }
    }
    softmax(st, k0);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint8_t* sb = smem + (B + hf) * BUFB;
      u32x4 vf[DB];
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const u32x2 lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(sb + voff(db)));
        const u32x2 hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(sb + voff(db) + 16 * ROWB));
        vf[db] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        // reduction index 8g + j: key 4g + j of the half's first 16-key block
        // (j < 4), 4g + j - 4 of its second
        const f32x4 s0 = st[r][hf * KB], s1 = st[r][hf * KB + 1];
        float e[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          e[i] = fast_exp2(s0[i]);
          e[4 + i] = fast_exp2(s1[i]);
        }
        const u32x4 pf = u32x4{pack2<T>(e[0], e[1]), pack2<T>(e[2], e[3]), pack2<T>(e[4], e[5]), pack2<T>(e[6], e[7])};
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[r][db] = mfma16x16x32<T>(vf[db], pf, oacc[r][db]);
        lpart[r] += ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
      }
    }
  };
  for (int jj = 0; jj < ntiles; jj += NB) {    // unrolled over the buffers: LDS offsets are constants
    step(std::integral_constant<int, 0>{}, jj);
    if (jj + 2 < ntiles) step(std::integral_constant<int, 2>{}, jj + 2);
  }
  wait_vmcnt<0>();               // the clamped trailing loads land before the work-group ends

  // Normalised rows to out; a split tile's halves to split_o instead (rows of
  // a half contiguous, fp32 unless both input and output are fp16: one
  // rounding of a bf16 half plus the output's would double the output's
  // rounding error), with their (max, sum) -- the log2-domain reference
  // maximum and the row sum relative to it -- for the merge.
  const size_t sunit = half >= 0 ? (size_t)h * (nqt - p.rows_split) + (qt - p.rows_split) : 0;
  void* const obase = half >= 0 ? p.split_o : p.out;
  const bool f32rows = half >= 0 ? rows_split_f32<T>(p.out_dtype) : p.out_dtype == kF32;
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const float lsum = sum_over_g(lpart[r]);
    if (qi[r] >= p.q_len) continue;
    const float inv = 1.0f / lsum;
    const size_t hrow = (sunit * 2 + (half > 0)) * BM + (qi[r] - qt * BM);   // row of a half
    if (half >= 0 && g == 0) *reinterpret_cast<float2*>(p.split_ml + hrow * 2) = float2{mref[r], lsum};
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const size_t idx = (half >= 0 ? hrow * D : (size_t)qi[r] * p.out_stride + (size_t)h * D) + db * 16 + 4 * g;
      const f32x4 v = oacc[r][db] * inv;
      if (f32rows) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(obase) + idx) = v;
      } else {
        const u32x2 w = u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(obase) + idx) = w;
      }
    }
  }
}

// Combines the two key halves of each split query tile: rows (h, qt) of the
// halves a and b, normalised, with (max, sum) pairs (m_a, l_a), (m_b, l_b)
// in the log2 domain, become
//   (w_a O_a + w_b O_b) / (w_a + w_b),  w = l * 2^(m - max(m_a, m_b)),
// the softmax over the whole key range, written to out.  Grid (Hq,
// nqt - rows_split, kRowsMergeParts), 256 threads: work-group z merges rows
// z BM / kRowsMergeParts .. of the tile, a thread 8 elements of a row.  H: the
// halves' element type, E: the output's.
constexpr int kRowsMergeParts = 4;

template <typename H, typename E, int D>
__global__ void __launch_bounds__(256) prefill_rows_merge_kernel(const PrefillParams p) {
  constexpr int BM = kRowsBM;
  constexpr int PR = D / 8;                 // threads per row
  constexpr int RP = 256 / PR;              // rows per pass
  constexpr int RZ = BM / kRowsMergeParts;  // rows per work-group
  const int h = blockIdx.x, qt = p.rows_split + (int)blockIdx.y;
  const size_t sunit = (size_t)h * gridDim.y + blockIdx.y;
  const int piece = threadIdx.x % PR;
  // 8 elements of type X at x as floats
  auto load8 = [](const auto* x, float (&f)[8]) {
    using X = std::remove_cv_t<std::remove_pointer_t<decltype(x)>>;
    if constexpr (sizeof(X) == 4) {
      const f32x4 lo = *reinterpret_cast<const f32x4*>(x), hi = *reinterpret_cast<const f32x4*>(x + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[i] = lo[i];
        f[4 + i] = hi[i];
      }
    } else {
      const u32x4 w = *reinterpret_cast<const u32x4*>(x);
#pragma unroll
      for (int i = 0; i < 4; ++i) unpack2<X>(w[i], f[2 * i], f[2 * i + 1]);
    }
  };
  for (int row = (int)blockIdx.z * RZ + threadIdx.x / PR; row < ((int)blockIdx.z + 1) * RZ; row += RP) {
    const int qi = qt * BM + row;
    if (qi >= p.q_len) break;
    const size_t ra = (sunit * 2) * BM + row, rb = ra + BM;
    const float2 a = *reinterpret_cast<const float2*>(p.split_ml + ra * 2);
    const float2 b = *reinterpret_cast<const float2*>(p.split_ml + rb * 2);
    const float m = fmaxf(a.x, b.x);
    const float wa = a.y * fast_exp2(a.x - m), wb = b.y * fast_exp2(b.x - m);
    const float inv = 1.0f / (wa + wb);
    const float ca = wa * inv, cb = wb * inv;
    const H* const hs = reinterpret_cast<const H*>(p.split_o);
    float fa[8], fb[8];
    load8(hs + ra * D + piece * 8, fa);
    load8(hs + rb * D + piece * 8, fb);
    E* const op = reinterpret_cast<E*>(p.out) + (size_t)qi * p.out_stride + (size_t)h * D + piece * 8;
    if constexpr (sizeof(E) == 4) {
      *reinterpret_cast<f32x4*>(op) = f32x4{fa[0] * ca + fb[0] * cb, fa[1] * ca + fb[1] * cb,
                                            fa[2] * ca + fb[2] * cb, fa[3] * ca + fb[3] * cb};
      *reinterpret_cast<f32x4*>(op + 4) = f32x4{fa[4] * ca + fb[4] * cb, fa[5] * ca + fb[5] * cb,
                                                fa[6] * ca + fb[6] * cb, fa[7] * ca + fb[7] * cb};
    } else {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = pack2<E>(fa[2 * i] * ca + fb[2 * i] * cb, fa[2 * i + 1] * ca + fb[2 * i + 1] * cb);
      *reinterpret_cast<u32x4*>(op) = w;
    }
  }
}

// Work-groups of prefill_rows_kernel<T, D> resident at once on the current
// device (occupancy x CUs), queried once per device.
template <typename T, int D>
long long rows_resident() {
  static std::atomic<long long> slots[kMaxDevices];
  return resident_work_groups(slots, prefill_rows_kernel<T, D>, 256);
}

// First split query tile (rows_split) of a launch; nqt: no split.  One causal
// prompt with at least as many keys as queries, on a grid that leaves at
// least a quarter of the resident slots empty: there the last tile's chain of
// 2 nqt key steps sets the time while CUs holding short tiles (or none) idle,
// and the key halves of the longer half of the tiles spread that chain over
// more work-groups.  On a full grid the zig-zag already gives every CU the
// same work, and a CU's two work-groups together step only ~1.3x as fast as
// one alone (per-work-group clock stamps at L 2048, Hq 32: 2.1-3.0 us per
// 64-key step side by side, 1.6 alone), so the extra work-groups and the
// merge cost more than the shorter chain saves.  Measured (MI355X, fp16,
// head_dim 128, Hkv 8, split against whole tiles): L 2048 Hq 8 / 16 31.2 /
// 40.5 against 44.3 / 47.4 us, L 4096 Hq 8 58.4 against 82.6, L 3072 Hq 16
// 60.8 against 69.2, L 6144 Hq 8 95.6 against 124.9, L 4096 Hq 12 (Hkv 4)
// 72.2 against 86.0; slower where the split grid overflows the resident slots
// with short rows: L 2048 Hq 24 / 32 50.0 / 66.0 against 47.4 / 54.9, L 2560
// Hq 24 67.8 against 58.7.
template <typename T, int D>
int rows_split_from(const PrefillParams& p, int num_seqs) {
  const int nqt = (p.q_len + kRowsBM - 1) / kRowsBM;
  if (num_seqs != 1 || p.cu_q || p.kv_table || !p.causal || p.q_pos_offset != 0 || p.kv_len < p.q_len || nqt < 4)
    return nqt;
  const long long resident = rows_resident<T, D>(), heads = p.num_heads;
  const int split = nqt / 2;
  if (4 * heads * nqt > 3 * resident) return nqt;
  if (heads * (2 * nqt - split) > resident && nqt < 24) return nqt;
  return split;
}

// Workspace bytes of a split launch: both halves' rows (room for fp32 rows
// whatever the types, so the size depends on the shape only), then their
// (max, sum) pairs.
template <typename T, int D>
size_t rows_split_layout(const PrefillParams& p, int split, size_t& ml_offset) {
  const int nqt = (p.q_len + kRowsBM - 1) / kRowsBM;
  const size_t units = (size_t)p.num_heads * (nqt - split);
  ml_offset = units * 2 * kRowsBM * D * sizeof(float);
  return split >= nqt ? 0 : ml_offset + units * 2 * kRowsBM * 2 * sizeof(float);
}

template <typename T, int D>
size_t rows_workspace(const PrefillParams& p) {
  size_t ml_offset;
  return rows_split_layout<T, D>(p, rows_split_from<T, D>(p, 1), ml_offset);
}

template <typename T, int D>
void launch_rows(const PrefillParams& pp_in, int num_seqs, int max_q_len, void* workspace, hipStream_t stream) {
  PrefillParams pp = pp_in;
  const int nqt = (max_q_len + kRowsBM - 1) / kRowsBM;
  // the merge moves 16-byte pieces of the workspace and of out's rows
  const bool aligned16 = (uintptr_t)workspace % 16 == 0 && (uintptr_t)pp.out % 16 == 0 && pp.out_stride % 8 == 0;
  pp.rows_split = workspace && aligned16 ? rows_split_from<T, D>(pp, num_seqs) : nqt;
  if (pp.rows_split < nqt) {
    size_t ml_offset;
    rows_split_layout<T, D>(pp, pp.rows_split, ml_offset);
    pp.split_o = workspace;
    pp.split_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + ml_offset);
    pp.longest_first = 0;
    hipLaunchKernelGGL((prefill_rows_kernel<T, D>), dim3(pp.num_heads, 2 * nqt - pp.rows_split), dim3(256), 0,
                       stream, pp);
    const dim3 mgrid(pp.num_heads, nqt - pp.rows_split, kRowsMergeParts);
    using H = std::conditional_t<rows_split_f32<T>(ElemTraits<T>::kCode), float, T>;   // halves of a T output
    if (pp.out_dtype == kF32)
      hipLaunchKernelGGL((prefill_rows_merge_kernel<float, float, D>), mgrid, dim3(256), 0, stream, pp);
    else
      hipLaunchKernelGGL((prefill_rows_merge_kernel<H, T, D>), mgrid, dim3(256), 0, stream, pp);
    return;
  }
  const dim3 grid(pp.num_heads, nqt, num_seqs);
  pp.longest_first = (long long)grid.x * grid.y * grid.z > rows_resident<T, D>() ? 1 : 0;
  hipLaunchKernelGGL((prefill_rows_kernel<T, D>), grid, dim3(256), 0, stream, pp);
}

// Workspace of a one-prompt launch (0: no split, or a shape not handled here).
size_t prefill_rows_workspace_bytes(const PrefillParams& pp, int dtype) {
  if (!(dtype == kF16 || dtype == kBF16) || pp.head_dim != 128) return 0;
  return dtype == kF16 ? rows_workspace<_Float16, 128>(pp) : rows_workspace<__bf16, 128>(pp);
}

// Launch for one prompt (grid.z = 1) or several (cu_q set; grid.z = prompts).
// A one-prompt launch given a workspace of prefill_rows_workspace_bytes may
// split its longer query tiles.  Returns false when the shape is not handled
// here (only head_dim 128 is: at head_dim 64 the 64-row kernel of
// flash_prefill.hip is faster at every length measured).
bool launch_prefill_rows(const PrefillParams& pp, int dtype, int num_seqs, int max_q_len, void* workspace,
                         hipStream_t stream) {
  if (!(dtype == kF16 || dtype == kBF16) || pp.head_dim != 128) return false;
  if (dtype == kF16) launch_rows<_Float16, 128>(pp, num_seqs, max_q_len, workspace, stream);
  else launch_rows<__bf16, 128>(pp, num_seqs, max_q_len, workspace, stream);
  return true;
}

}  // namespace tv
