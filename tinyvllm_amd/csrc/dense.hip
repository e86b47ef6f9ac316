// Dense kernels of the batched decode step (gfx950): the weight-streaming
// products, RMSNorm with the residual add, RoPE with the K/V cache write, and
// greedy sampling.  Semantics follow tinyvllm/model/llama.py:
//   RMSNorm          x * rsqrt(mean(x^2) + eps) * w              llama.py:14-23
//   RoPE table       cos/sin(p * theta^(-2i/D))                  llama.py:26-31
//   RoPE             interleaved pairs (2i, 2i+1)                llama.py:34-55
//   SwiGLU           w2(silu(w1 x) * w3 x)                       llama.py:220-221
//   greedy sampling  argmax over the vocabulary (first maximum)  sampling.py:131-134
//
// linear_kernel computes Y = A W^T for a skinny A (the decode batch, M <= 64
// per work-group) against a weight matrix W [N, K] that is streamed from HBM
// exactly once.  Each of the 4 waves of a work-group owns 16 rows of W and all
// 64 rows of A; A is staged in LDS per 512-byte-wide K chunk (256 fp16/bf16 or
// 128 fp32 elements) and shared by the waves.  fp32 runs the same byte layout
// on v_mfma_f32_16x16x4_f32, four of them per 16-byte fragment pair.  W rows are the MFMA A operand (lane = output feature), A^T the B
// operand (lane = token), so a lane ends up holding 4 consecutive output
// features of one token: the layout the fused epilogues want.
#include "tv_common.h"
#include "tv_dense.h"

namespace tv {

// ---------------------------------------------------------------------------
// Y = A W^T
// ---------------------------------------------------------------------------

__device__ __forceinline__ unsigned long long argmax_key(float v, int n) {
  // order-preserving map of the float to an unsigned key; ties resolve to the
  // smallest index, as numpy / tinygrad argmax return the first maximum
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (0xFFFFFFFFu - (uint32_t)n);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// Two / four consecutive elements of T to and from floats.
template <typename T> __device__ __forceinline__ void store2(void* base, size_t idx, float a, float b) {
  *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(base) + idx) = pack2<T>(a, b);
}
template <> __device__ __forceinline__ void store2<float>(void* base, size_t idx, float a, float b) {
  *reinterpret_cast<float2*>(reinterpret_cast<float*>(base) + idx) = float2{a, b};
}
template <typename T> __device__ __forceinline__ void store4(void* base, size_t idx, f32x4 v) {
  *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(base) + idx) = u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
}
template <> __device__ __forceinline__ void store4<float>(void* base, size_t idx, f32x4 v) {
  *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(base) + idx) = v;
}
template <typename T> __device__ __forceinline__ f32x4 load4(const void* base, size_t idx) {
  const u32x2 e = *reinterpret_cast<const u32x2*>(reinterpret_cast<const T*>(base) + idx);
  float a, b, c, d;
  unpack2<T>(e[0], a, b);
  unpack2<T>(e[1], c, d);
  return f32x4{a, b, c, d};
}
template <> __device__ __forceinline__ f32x4 load4<float>(const void* base, size_t idx) {
  return *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + idx);
}

// acc += (16 rows of W) x (16 columns of A^T) over the k range of one pair of
// 16-byte fragments: one v_mfma_f32_16x16x32 for 16-bit T; for fp32 four
// v_mfma_f32_16x16x4_f32, step j taking element j of every lane's fragment
// (lane group g then holds k = 4 g + j in both operands, so the steps cover
// the fragment's 16 k once).
template <typename T> __device__ __forceinline__ f32x4 mfma_frag(u32x4 a, u32x4 b, f32x4 c) {
  return mfma16x16x32<T>(a, b, c);
}
template <> __device__ __forceinline__ f32x4 mfma_frag<float>(u32x4 a, u32x4 b, f32x4 c) {
#pragma unroll
  for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(u32_as_f32(a[j]), u32_as_f32(b[j]), c, 0, 0, 0);
  return c;
}

constexpr int kLinearMinBlocks = 1;    // occupancy hint of the product kernel
constexpr int kLinearWStages = 2;      // W chunks in registers: in flight + the one multiplied
// A chunks requested ahead of the one being multiplied.  Two ahead measured
// slower for every product of the TinyLlama batch-64 decode step (64-step
// graph: 1468 us/step at one ahead; two ahead for the SwiGLU product 1488, for
// the split-K partial products 1485, for both 1505), so one it is.
constexpr int kLinearAStages = 1;

constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }
constexpr int lcm3(int a, int b, int c) {
  const int ab = a / gcd_c(a, b) * b;
  return ab / gcd_c(ab, c) * c;
}

// Epilogue of the skinny product: lane (wave, g, col) holds acc[mb][i] =
// Y[m0 + 16 mb + col][n_wave + 4 g + i].  sk: 8 KB of LDS for the argmax
// exchange (logits), free to reuse once every wave reaches this point.
template <typename T, int EPI>
__device__ __forceinline__ void linear_epilogue(const LinearParams& p, const f32x4 (&acc)[4], int n_wave, int m0,
                                                int split, int ntile, int wave, int tid, unsigned long long* sk) {
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int col = lane & 15;
  const int n = n_wave + 4 * g;
  if constexpr (EPI == kEpiPartial) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int m = m0 + mb * 16 + col;
      if (m < p.M && n < p.N)
        *reinterpret_cast<f32x4*>(p.part + ((size_t)split * p.M + m) * p.N + n) = acc[mb];
    }
  } else if constexpr (EPI == kEpiSwiglu) {
    // rows 4j, 4j+1 of W are w1 rows 2j, 2j+1; rows 4j+2, 4j+3 the matching w3 rows
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int m = m0 + mb * 16 + col;
      if (m < p.M && n < p.N) {
        const f32x4 v = acc[mb];
        store2<T>(p.out, (size_t)m * p.ldo + (n >> 1), silu(v[0]) * v[2], silu(v[1]) * v[3]);
      }
    }
  } else {
    lds_barrier();   // sk reuses LDS of the main loop: [16 (wave, g)][64 rows]
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int m = m0 + mb * 16 + col;
      const f32x4 v = acc[mb];
      if (p.out && m < p.M && n < p.N)
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.out) + (size_t)m * p.ldo + n) = v;
      unsigned long long best = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + i < p.N) best = max(best, argmax_key(v[i], n + i));
      sk[(wave * 4 + g) * 64 + mb * 16 + col] = best;
    }
    lds_barrier();
    if (tid < 64 && p.keys && m0 + tid < p.M) {
      unsigned long long best = sk[tid];
#pragma unroll
      for (int j = 1; j < 16; ++j) best = max(best, sk[j * 64 + tid]);
      p.keys[(size_t)ntile * p.M + m0 + tid] = best;
    }
  }
}

template <typename T, int EPI>
__global__ void __launch_bounds__(256, kLinearMinBlocks) linear_kernel(const LinearParams p) {
  // LDS in 16-bit units; a chunk row is 512 bytes of K at a 544-byte pitch (an
  // odd multiple of 32 modulo 256: conflict-free 16-byte reads)
  constexpr int KP = 256 + 16;
  constexpr int KC = 512 / (int)sizeof(T);   // K elements per chunk
  constexpr int VE = 16 / (int)sizeof(T);    // K elements per 16-byte vector
  __shared__ __attribute__((aligned(16))) uint16_t sa[2][kLinBM * KP];   // A chunk, double-buffered

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: W resource in SGPRs
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int col = lane & 15;
  // grid (splits, n tiles, m tiles): consecutive work-groups take different
  // K splits of one n tile, and each n tile starts its chunk sequence at a
  // different chunk, so the work-groups in flight read different column
  // ranges of W.  (With the row pitch of W a power of two, work-groups that
  // march through the same columns in step all hit the same HBM channels.)
  const int split = blockIdx.x;
  const int ntile = blockIdx.y;
  const int n_wave = ntile * kLinBN + wave * 16;
  const int m0 = blockIdx.z * kLinBM;
  const int kb = split * p.k_split;
  const int ke = min(kb + p.k_split, p.K);
  const int nc = (ke - kb + KC - 1) / KC;
  const int rot = ntile % nc;
  auto chunk_of = [&](int i) { const int c = i + rot; return c < nc ? c : c - nc; };

  // Buffer loads: reads past the end of W (rows >= N) or of A (rows >= M)
  // return zero in hardware, so no address is clamped.  The row part of every
  // offset goes in the VGPR offset: the hardware range check covers the VGPR
  // and instruction offsets, not the scalar one.
  const long long w_rows = max(p.N - n_wave, 0);
  const __amdgpu_buffer_rsrc_t wres = make_rsrc(reinterpret_cast<const T*>(p.w) + (size_t)min(n_wave, p.N) * p.K,
                                                (unsigned long long)w_rows * p.K * sizeof(T));
  const __amdgpu_buffer_rsrc_t ares = make_rsrc(reinterpret_cast<const T*>(p.a) + (size_t)m0 * p.lda,
                                                (unsigned long long)max(p.M - m0, 0) * p.lda * sizeof(T));
  const int w_voff = (col * p.K + kb) * (int)sizeof(T) + 16 * g;
  const int a_voff = ((tid >> 5) * (int)p.lda + kb) * (int)sizeof(T) + 16 * (tid & 31);
  const int a_rows8 = 8 * (int)p.lda * (int)sizeof(T);   // byte step between the 8 rows a thread loads

  // W: lane (row col, k group g) reads 16 bytes per 64-byte k step.  Columns
  // past the split are multiplied by zero rows of A.
  // i is the position in this work-group's chunk sequence; positions past the
  // last chunk re-read it (W) or load zeros (A), so padding steps add nothing.
  auto loadW = [&](int i, u32x4 (&r)[8]) {
    const int off = w_voff + chunk_of(min(i, nc - 1)) * 512;
#pragma unroll
    for (int s = 0; s < 8; ++s) r[s] = buffer_load16(wres, off + 64 * s, 0);
  };
  // A chunk: 64 rows x 32 vectors of 16 bytes; thread tid loads vector
  // tid % 32 of rows tid / 32 + 8 i.  Columns past the split are zeroed when
  // stored to LDS (not at load time, so the loads stay in flight while the
  // previous chunk computes).
  auto loadA = [&](int i, u32x4 (&r)[8], bool& valid) {
    const int c = chunk_of(min(i, nc - 1));
    valid = i < nc && kb + c * KC + VE * (tid & 31) < ke;
    const int off = a_voff + c * 512;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = buffer_load16(ares, off + i * a_rows8, 0);   // row in the range-checked offset
  };
  auto storeA = [&](const u32x4 (&r)[8], bool valid, int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<u32x4*>(&sa[buf][((tid >> 5) + 8 * i) * KP + 8 * (tid & 31)]) = valid ? r[i] : u32x4{0, 0, 0, 0};
  };

  f32x4 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // All 8 k steps run even on a partial chunk: the A rows there are zero.
  // The B fragments of step s + 1 are read from LDS while step s multiplies.
  auto compute = [&](const u32x4 (&r)[8], int buf) {
    u32x4 b[2][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) b[0][mb] = *reinterpret_cast<const u32x4*>(&sa[buf][(mb * 16 + col) * KP + 8 * g]);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s + 1 < 8) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
          b[(s + 1) & 1][mb] = *reinterpret_cast<const u32x4*>(&sa[buf][(mb * 16 + col) * KP + 32 * (s + 1) + 8 * g]);
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) acc[mb] = mfma_frag<T>(r[s], b[s & 1][mb], acc[mb]);
    }
  };

  constexpr int NWS = kLinearWStages;
  constexpr int NAS = kLinearAStages;     // A chunks in flight in registers
  constexpr int U = lcm3(NWS, NAS, 2);     // loop unroll: every stage / buffer index compile-time
  u32x4 w[NWS][8], ar[NAS][8];
  bool av[NAS];
  if (nc == 1) {
    loadW(0, w[0]);
    loadA(0, ar[0], av[0]);
    storeA(ar[0], av[0], 0);
    lds_barrier();
    compute(w[0], 0);
  } else if (NWS >= 2 && nc == 2) {
    // both chunks requested at once, one in each LDS buffer: one round trip
    // instead of the pipeline's two (the Wqkv product of the decode step)
    u32x4 a1[8];
    bool v1;
    loadW(0, w[0]);
    loadW(1, w[1 % NWS]);
    loadA(0, ar[0], av[0]);
    loadA(1, a1, v1);
    storeA(ar[0], av[0], 0);
    storeA(a1, v1, 1);
    lds_barrier();
    compute(w[0], 0);
    compute(w[1 % NWS], 1);
  } else {
#pragma unroll
    for (int i = 0; i < NWS - 1; ++i) loadW(i, w[i]);
#pragma unroll
    for (int i = 0; i < NAS; ++i) loadA(i, ar[i], av[i]);
    // Step j multiplies chunk j: W of chunks j + 1 .. j + NWS - 1 and A of
    // chunks j + 1 .. j + NAS are in flight meanwhile.  A goes through two
    // LDS buffers, so one barrier per step orders both its store and the
    // reuse of the buffer two steps later.  The loads are unconditional and
    // the step count is padded to a multiple of U (padding steps multiply
    // zero A rows), so the loop body has no exit and the compiler waits for
    // exactly the chunk it needs.  (sched_barrier keeps each prefetch issued
    // before the waits that follow.)
    const int ncp = (nc + U - 1) / U * U;
    for (int c = 0; c < ncp; c += U) {
#pragma unroll
      for (int j = 0; j < U; ++j) {
        loadW(c + j + NWS - 1, w[(j + NWS - 1) % NWS]);
        __builtin_amdgcn_sched_barrier(0);
        storeA(ar[j % NAS], av[j % NAS], j & 1);
        lds_barrier();
        loadA(c + j + NAS, ar[j % NAS], av[j % NAS]);
        __builtin_amdgcn_sched_barrier(0);
        compute(w[j % NWS], j & 1);
      }
    }
  }

  linear_epilogue<T, EPI>(p, acc, n_wave, m0, split, ntile, wave, tid, reinterpret_cast<unsigned long long*>(&sa[0][0]));
}


#define TV_LINEAR_CASE(T)                                                                              \
  switch (epi) {                                                                                       \
    case kEpiPartial: hipLaunchKernelGGL((linear_kernel<T, kEpiPartial>), grid, dim3(256), 0, s, p); \
      break;                                                                                           \
    case kEpiSwiglu: hipLaunchKernelGGL((linear_kernel<T, kEpiSwiglu>), grid, dim3(256), 0, s, p);   \
      break;                                                                                           \
    default: hipLaunchKernelGGL((linear_kernel<T, kEpiLogits>), grid, dim3(256), 0, s, p);           \
  }

void launch_linear(const LinearParams& p, int epi, int dtype, hipStream_t s) {
  const dim3 grid((p.K + p.k_split - 1) / p.k_split, (p.N + kLinBN - 1) / kLinBN, (p.M + kLinBM - 1) / kLinBM);
  if (dtype == kF16) {
    TV_LINEAR_CASE(_Float16)
  } else if (dtype == kBF16) {
    TV_LINEAR_CASE(__bf16)
  } else {
    TV_LINEAR_CASE(float)
  }
}

// ---------------------------------------------------------------------------
// residual add + RMSNorm
// ---------------------------------------------------------------------------

// One work-group per row; thread t holds float4 vectors t + 256 i (VPT of
// them) in registers, so the row is read once: every load (weight, embedding
// or residual, split partials) is issued before the first add, one LDS
// reduction gives the mean square, and the normalised row is written from
// registers.
// MODE: kNormEmb (x = emb[tokens]), kNormPart (x += the split partials) or
// kNormPlain (x as it is).  One instantiation per mode keeps every load of the
// row in one basic block, so the weight, residual and first batch of partials
// are all requested before the first wait.
enum NormMode : int { kNormEmb = 0, kNormPart = 1, kNormPlain = 2 };

template <typename T, int VPT, int MODE>
__global__ void __launch_bounds__(256) norm_kernel(const NormParams p) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  float* x = p.x + (size_t)m * p.dim;
  // SB splits per batch of loads: all of a product's splits in one round trip
  // at the decode step's sizes; indexes past the last split re-read it and are
  // dropped
  constexpr int SB = VPT <= 2 ? 8 : 4;
  f32x4 v[VPT], w[VPT], t[MODE == kNormPart ? SB : 1][VPT];
  int tok = 0;
  if constexpr (MODE == kNormEmb) tok = min(max(p.tokens[m], 0), p.vocab - 1);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int k = min(4 * (threadIdx.x + 256 * i), p.dim - 4);   // clamped: lanes past dim re-read the last vector
    w[i] = *reinterpret_cast<const f32x4*>(p.weight + k);
    if constexpr (MODE == kNormEmb) {
      v[i] = load4<T>(p.emb, (size_t)tok * p.dim + k);
    } else {
      v[i] = *reinterpret_cast<const f32x4*>(x + k);
    }
    if constexpr (MODE == kNormPart) {
      if (p.splits == 1) {   // unsplit producer (prompt passes): one load, not SB copies of it
        t[0][i] = *reinterpret_cast<const f32x4*>(p.part + (size_t)m * p.dim + k);
      } else {
#pragma unroll
        for (int u = 0; u < SB; ++u)
          t[u][i] = *reinterpret_cast<const f32x4*>(p.part + ((size_t)min(u, p.splits - 1) * p.M + m) * p.dim + k);
      }
    }
  }
  if constexpr (MODE == kNormPart) {
#pragma unroll
    for (int u = 0; u < SB; ++u)
      if (u < p.splits) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) v[i] += t[u][i];
      }
    for (int s0 = SB; s0 < p.splits; s0 += SB) {
#pragma unroll
      for (int u = 0; u < SB; ++u)
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
          const int k = min(4 * (threadIdx.x + 256 * i), p.dim - 4);
          t[u][i] = *reinterpret_cast<const f32x4*>(p.part + ((size_t)min(s0 + u, p.splits - 1) * p.M + m) * p.dim + k);
        }
#pragma unroll
      for (int u = 0; u < SB; ++u)
        if (s0 + u < p.splits) {
#pragma unroll
          for (int i = 0; i < VPT; ++i) v[i] += t[u][i];
        }
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int k = 4 * (threadIdx.x + 256 * i);
    if (k < p.dim) {
      if constexpr (MODE != kNormPlain) *reinterpret_cast<f32x4*>(x + k) = v[i];
      ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
    }
  }
  ss = group_sum<64>(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  lds_barrier();
  const float r = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)p.dim + p.eps);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int k = 4 * (threadIdx.x + 256 * i);
    if (k < p.dim) {
      store4<T>(p.xh, (size_t)m * p.dim + k, v[i] * r * w[i]);
    }
  }
}

template <typename T, int VPT> void launch_norm_v(const NormParams& p, hipStream_t s) {
  if (p.emb) hipLaunchKernelGGL((norm_kernel<T, VPT, kNormEmb>), dim3(p.M), dim3(256), 0, s, p);
  else if (p.part) hipLaunchKernelGGL((norm_kernel<T, VPT, kNormPart>), dim3(p.M), dim3(256), 0, s, p);
  else hipLaunchKernelGGL((norm_kernel<T, VPT, kNormPlain>), dim3(p.M), dim3(256), 0, s, p);
}

template <typename T> void launch_norm_t(const NormParams& p, hipStream_t s) {
  const int vpt = (p.dim + 1023) / 1024;
  if (vpt <= 1) launch_norm_v<T, 1>(p, s);
  else if (vpt <= 2) launch_norm_v<T, 2>(p, s);
  else if (vpt <= 4) launch_norm_v<T, 4>(p, s);
  else launch_norm_v<T, 8>(p, s);
}

void launch_norm(const NormParams& p, int dtype, hipStream_t s) {
  if (dtype == kF16)
    launch_norm_t<_Float16>(p, s);
  else if (dtype == kBF16)
    launch_norm_t<__bf16>(p, s);
  else
    launch_norm_t<float>(p, s);
}

// ---------------------------------------------------------------------------
// QKV: split reduction, RoPE, q store, K/V cache write
// ---------------------------------------------------------------------------

template <typename T>
__global__ void __launch_bounds__(256) qkv_rope_kernel(const QKVParams p) {
  const int qn = p.Hq * p.D;
  const int kn = p.Hkv * p.D;
  const int N = qn + 2 * kn;
  const int half = N >> 1;
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)p.M * half) return;
  const int m = (int)(t / half);
  const int n = 2 * (int)(t - (long long)m * half);
  // SB split partials requested at once with the position (one round trip
  // for the usual split counts); indexes past the last split re-read it and
  // are dropped; the sum runs in split order
  constexpr int SB = 8;
  float2 pv[SB];
  if (p.splits == 1) {   // unsplit producer (prompt passes): one load, not SB copies of it
    pv[0] = *reinterpret_cast<const float2*>(p.part + (size_t)m * N + n);
  } else {
#pragma unroll
    for (int s = 0; s < SB; ++s)
      pv[s] = *reinterpret_cast<const float2*>(p.part + ((size_t)min(s, p.splits - 1) * p.M + m) * N + n);
  }
  const int pos = p.positions ? p.positions[m] : p.pos_base + m;
  float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
  for (int s = 0; s < SB; ++s)
    if (s < p.splits) {
      v0 += pv[s].x;
      v1 += pv[s].y;
    }
  for (int s0 = SB; s0 < p.splits; s0 += SB) {
#pragma unroll
    for (int s = 0; s < SB; ++s)
      pv[s] = *reinterpret_cast<const float2*>(p.part + ((size_t)min(s0 + s, p.splits - 1) * p.M + m) * N + n);
#pragma unroll
    for (int s = 0; s < SB; ++s)
      if (s0 + s < p.splits) {
        v0 += pv[s].x;
        v1 += pv[s].y;
      }
  }
  if (n < qn + kn) {
    const int i = (n % p.D) >> 1;
    const int pr = min(max(pos, 0), p.rope_len - 1);
    const float2 cs = *reinterpret_cast<const float2*>(p.rope + ((size_t)pr * (p.D >> 1) + i) * 2);
    const float a = v0 * cs.x - v1 * cs.y;
    const float b = v0 * cs.y + v1 * cs.x;
    v0 = a;
    v1 = b;
  }
  if (n < qn) {
    store2<T>(p.q, (size_t)m * qn + n, v0, v1);
    return;
  }
  const bool is_k = n < qn + kn;
  const int e = is_k ? n - qn : n - qn - kn;
  void* stage = is_k ? p.k_out : p.v_out;
  if (stage) store2<T>(stage, (size_t)m * kn + e, v0, v1);
  void* cache = is_k ? p.k_cache : p.v_cache;
  const bool report = is_k && e == 0;   // one thread per row reports the slot
  if (!p.block_tables || (!cache && !(report && (p.slots || p.err_count)))) return;
  long long slot = -1;
  if (pos >= 0 && pos / p.block_size < p.bt_width) {
    const int blk = p.block_tables[(size_t)m * p.bt_row_step + pos / p.block_size];
    if (blk >= 0 && blk < p.num_blocks) slot = (long long)blk * p.block_size + pos % p.block_size;
  }
  if (cache && slot >= 0) store2<T>(cache, (size_t)slot * kn + e, v0, v1);
  if (report) {
    if (p.slots) p.slots[m] = (int)slot;
    if (slot < 0 && p.err_count) atomicAdd(p.err_count, 1u);
  }
}

void launch_qkv_rope(const QKVParams& p, int dtype, hipStream_t s) {
  const long long pairs = (long long)p.M * ((p.Hq + 2 * p.Hkv) * p.D / 2);
  const dim3 grid((unsigned)((pairs + 255) / 256));
  if (dtype == kF16)
    hipLaunchKernelGGL(qkv_rope_kernel<_Float16>, grid, dim3(256), 0, s, p);
  else if (dtype == kBF16)
    hipLaunchKernelGGL(qkv_rope_kernel<__bf16>, grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(qkv_rope_kernel<float>, grid, dim3(256), 0, s, p);
}

__global__ void rope_table_kernel(float* table, int max_pos, int head_dim, float theta) {
  const int half = head_dim >> 1;
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)max_pos * half) return;
  const int pos = (int)(idx / half);
  const int i = (int)(idx - (long long)pos * half);
  const float freq = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
  const float ang = (float)pos * freq;
  table[2 * idx] = cosf(ang);
  table[2 * idx + 1] = sinf(ang);
}

void launch_rope_table(float* table, int max_pos, int head_dim, float theta, hipStream_t s) {
  const long long n = (long long)max_pos * (head_dim / 2);
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, table, max_pos,
                     head_dim, theta);
}

// ---------------------------------------------------------------------------
// greedy sampling + position advance
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(64) advance_kernel(const AdvanceParams p) {
  const int m = blockIdx.x;
  const int lane = threadIdx.x;
  unsigned long long best = 0;
  // U keys per lane requested at once (500 per sequence at a 32000 vocabulary:
  // one round trip); indexes past the last key re-read it, which max ignores
  constexpr int U = 8;
  for (int j0 = 0; j0 < p.nparts; j0 += 64 * U) {
    unsigned long long kv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) kv[u] = p.keys[(size_t)min(j0 + lane + 64 * u, p.nparts - 1) * p.M + m];
#pragma unroll
    for (int u = 0; u < U; ++u) best = max(best, kv[u]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute((lane ^ off) << 2, (int)(uint32_t)best);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute((lane ^ off) << 2, (int)(uint32_t)(best >> 32));
    best = max(best, ((unsigned long long)hi << 32) | lo);
  }
  if (lane != 0) return;
  const int tok = (int)(0xFFFFFFFFu - (uint32_t)best);
  p.tokens[m] = tok;
  if (p.positions) {
    const int pos = p.positions[m];
    if (p.history && pos >= 0 && pos + 1 < p.history_len) p.history[(size_t)m * p.history_len + pos + 1] = tok;
    p.positions[m] = pos + 1;
  }
  if (p.context_lens) p.context_lens[m] += 1;
}

void launch_advance(const AdvanceParams& p, hipStream_t s) {
  hipLaunchKernelGGL(advance_kernel, dim3(p.M), dim3(64), 0, s, p);
}

__global__ void __launch_bounds__(256) iota_kernel(int* out, int n, int base) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = base + i;
}

void launch_iota(int* out, int n, int base, hipStream_t s) {
  hipLaunchKernelGGL(iota_kernel, dim3((n + 255) / 256), dim3(256), 0, s, out, n, base);
}

}  // namespace tv
