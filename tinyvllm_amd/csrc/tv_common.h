// Shared device helpers for the tinyvllm MI355X (gfx950) attention kernels.
//
// Element types: float, _Float16, __bf16.  All global loads and stores of
// cache / activation rows go through 16-byte vectors (u32x4) so every lane
// issues one 128-bit access.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tv {

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

template <typename T> struct ElemTraits;
template <> struct ElemTraits<float> { static constexpr int kCode = kF32; };
template <> struct ElemTraits<_Float16> { static constexpr int kCode = kF16; };
template <> struct ElemTraits<__bf16> { static constexpr int kCode = kBF16; };

// ---- conversions on packed 32-bit words -----------------------------------

// Reinterpret a 32-bit word as float.  Takes the word by value: applying
// __builtin_bit_cast directly to an element of an ext_vector_type lvalue reads
// element 0 of the vector with this compiler.
__device__ __forceinline__ float u32_as_f32(uint32_t w) { return __builtin_bit_cast(float, w); }

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
__device__ __forceinline__ float f16_lo(uint32_t w) {
  return (float)__builtin_bit_cast(f16x2, w)[0];
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
  return (float)__builtin_bit_cast(f16x2, w)[1];
}

// Unpack the two elements of a 32-bit word of type T into floats.
template <typename T> __device__ __forceinline__ void unpack2(uint32_t w, float& a, float& b);
template <> __device__ __forceinline__ void unpack2<_Float16>(uint32_t w, float& a, float& b) {
  a = f16_lo(w); b = f16_hi(w);
}
template <> __device__ __forceinline__ void unpack2<__bf16>(uint32_t w, float& a, float& b) {
  a = bf16_lo(w); b = bf16_hi(w);
}

// Dot product of two packed pairs accumulated in fp32 (v_dot2_f32_{f16,bf16}).
template <typename T> __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c);
template <> __device__ __forceinline__ float dot2<_Float16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}
template <> __device__ __forceinline__ float dot2<__bf16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// Round a float to T (round-to-nearest-even) and back to raw bits.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <typename T> __device__ __forceinline__ T from_float(float f);
template <> __device__ __forceinline__ float from_float<float>(float f) { return f; }
template <> __device__ __forceinline__ _Float16 from_float<_Float16>(float f) { return (_Float16)f; }
template <> __device__ __forceinline__ __bf16 from_float<__bf16>(float f) {
  return __builtin_bit_cast(__bf16, f32_to_bf16_bits(f));
}

template <typename T> __device__ __forceinline__ float to_float(T x);
template <> __device__ __forceinline__ float to_float<float>(float x) { return x; }
template <> __device__ __forceinline__ float to_float<_Float16>(_Float16 x) { return (float)x; }
template <> __device__ __forceinline__ float to_float<__bf16>(__bf16 x) {
  return __builtin_bit_cast(float, (uint32_t)__builtin_bit_cast(uint16_t, x) << 16);
}

// Store one float as the output dtype selected at run time.
__device__ __forceinline__ void store_as(void* base, size_t idx, float v, int dtype) {
  if (dtype == kF32) {
    reinterpret_cast<float*>(base)[idx] = v;
  } else if (dtype == kF16) {
    reinterpret_cast<_Float16*>(base)[idx] = (_Float16)v;
  } else {
    reinterpret_cast<uint16_t*>(base)[idx] = f32_to_bf16_bits(v);
  }
}

// ---- MFMA ------------------------------------------------------------------
// v_mfma_f32_16x16x32_{f16,bf16}: D = A B + C with A 16x32, B 32x16.  Lane l
// supplies A[l % 16][8 (l / 16) + j] and B[8 (l / 16) + j][l % 16], j = 0..7, as
// eight packed elements; it receives D[4 (l / 16) + i][l % 16], i = 0..3.
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

// Eight packed 16-bit values each multiplied by c (fp32 product, rounded back).
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

// Where the softmax scale enters in the prefill kernels.  fp16: Q is
// pre-scaled by scale * log2(e) and rounded to fp16 once (a relative error of
// at most 2^-11 per element, comparable to the rounding of the fp16 inputs
// themselves), and the score accumulator starts at -m, so scores leave the
// matrix cores ready for exp2.  bf16: rounding q * scale to bf16 would add up
// to 2^-8 relative error to every score (scores of tens of units then move the
// softmax by several percent), so Q stays as given, the accumulator starts at 0
// and each score takes one fp32 fma, s * scale * log2(e) - m -- the
// reference's order, the scale applied after the product (llama.py:84).
template <typename T> inline constexpr bool kPreScaleQ = false;
template <> inline constexpr bool kPreScaleQ<_Float16> = true;

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

// ---- wave64 cross-lane helpers ---------------------------------------------
// DPP controls (GFX9 encoding): quad_perm, row_half_mirror, row_mirror.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within each 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within each 16

template <int CTRL> __device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float shfl_xor(float x, int mask) {
  int lane = __lane_id();
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __builtin_bit_cast(int, x)));
}

// Sum over aligned groups of N lanes (N a power of two <= 64); every lane of the
// group receives the total.  Groups of up to 16 use DPP only.
template <int N> __device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp<kDppXor1>(x);
  if constexpr (N >= 4) x += dpp<kDppXor2>(x);
  if constexpr (N >= 8) x += dpp<kDppHalfMirror>(x);
  if constexpr (N >= 16) x += dpp<kDppMirror>(x);
  if constexpr (N >= 32) x += shfl_xor(x, 16);
  if constexpr (N >= 64) x += shfl_xor(x, 32);
  return x;
}

template <int N> __device__ __forceinline__ float group_max(float x) {
  if constexpr (N >= 2) x = fmaxf(x, dpp<kDppXor1>(x));
  if constexpr (N >= 4) x = fmaxf(x, dpp<kDppXor2>(x));
  if constexpr (N >= 8) x = fmaxf(x, dpp<kDppHalfMirror>(x));
  if constexpr (N >= 16) x = fmaxf(x, dpp<kDppMirror>(x));
  if constexpr (N >= 32) x = fmaxf(x, shfl_xor(x, 16));
  if constexpr (N >= 64) x = fmaxf(x, shfl_xor(x, 32));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ds_read_b64_tr_b16 (gfx950): within each 16-lane row of the wave, lane i
// receives element i % 4 of the 64-bit words addressed by lanes 4 k + i / 4,
// k = 0..3.  With lane 4 k + q addressing row r_k, columns c + 4 q .. c + 4 q + 3
// of a row-major 16-bit matrix, lane i gets column c + i of rows r_0 .. r_3:
// a 4 x 16 block transposed into the MFMA operand layout.  ptr: LDS address.
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* ptr) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(ptr)));
}

// Raw buffer resource over [base, base + bytes) (gfx9 word 3: 32-bit dwords, no
// swizzle).  A load whose voffset lies at or past `bytes` returns zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned long long bytes) {
  // Clamp to 32 bits with a scalar compare of the high word.  Written as C the
  // compiler folds it into a 64-bit unsigned compare, which has no scalar form
  // and costs three VALU instructions per resource (bytes is wave-uniform at
  // every call, so both halves are scalars).
  unsigned n;
  asm("s_cmp_lg_u32 %1, 0\n\ts_cselect_b32 %0, -1, %2"
      : "=s"(n)
      : "s"((unsigned)(bytes >> 32)), "s"((unsigned)bytes)
      : "scc");
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Work-group barrier that orders LDS traffic only.  __syncthreads() also fences
// global memory, which makes every wave wait for all of its outstanding global
// loads (vmcnt(0)) -- including loads issued ahead as prefetch.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace tv
