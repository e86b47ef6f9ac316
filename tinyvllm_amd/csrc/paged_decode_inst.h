// Launch-side dispatch for the paged-decode kernel templates.  Each element
// type is instantiated in its own translation unit (paged_decode_{f32,f16,bf16}.hip)
// so the library builds in parallel.
#pragma once

#include "paged_decode.cuh"

namespace tv {

#ifndef TV_DECODE_WAVES
#define TV_DECODE_WAVES 4
#endif
constexpr int kDecodeWaves = TV_DECODE_WAVES;   // waves per work-group

// Launch the main kernel for element type T.  Returns false when (D, GT) has no
// instantiation.
template <typename T>
bool launch_paged_decode(const DecodeParams& p, int head_dim, int gt, dim3 grid, hipStream_t stream);

#define TV_DECODE_CASE(T, D, GT)                                                      \
  if (head_dim == D && gt == GT) {                                                    \
    hipLaunchKernelGGL((paged_decode_kernel<T, D, GT, kDecodeWaves>), grid,           \
                       dim3(64 * kDecodeWaves), 0, stream, p);                        \
    return true;                                                                      \
  }

#define TV_DECODE_ALL_GT(T, D) \
  TV_DECODE_CASE(T, D, 1)      \
  TV_DECODE_CASE(T, D, 2)      \
  TV_DECODE_CASE(T, D, 4)      \
  TV_DECODE_CASE(T, D, 8)

#define TV_DECODE_DEFINE(T)                                                                      \
  template <>                                                                                    \
  bool launch_paged_decode<T>(const DecodeParams& p, int head_dim, int gt, dim3 grid,            \
                              hipStream_t stream) {                                              \
    TV_DECODE_ALL_GT(T, 16)                                                                      \
    TV_DECODE_ALL_GT(T, 32)                                                                      \
    TV_DECODE_ALL_GT(T, 64)                                                                      \
    TV_DECODE_ALL_GT(T, 128)                                                                     \
    TV_DECODE_ALL_GT(T, 256)                                                                     \
    return false;                                                                                \
  }

}  // namespace tv
