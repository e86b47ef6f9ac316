// Launch-side dispatch for the paged-decode kernel templates.  Each element
// type is instantiated in its own translation unit (paged_decode_{f32,f16,bf16}.hip)
// so the library builds in parallel.
#pragma once

#include "paged_decode.cuh"
#include "tv_device_cache.h"

namespace tv {

constexpr int kDecodeWaves = 4;   // waves per work-group

// Small launches (at most one (sequence, KV head) pair per CU, contexts of at
// most kDecodeWideTokens): one unsplit launch of 8-wave work-groups, so a
// pair's tiles are spread over twice the waves (at most four 16-token tiles
// each) and no merge launch follows; the waves merge through LDS (64 GT D
// bytes).  The launcher also halves GQA chunks of 4+ heads when the doubled
// grid still fits the CUs (tv_api.hip), and waves with at most two tiles
// request both before consuming either (decode_range).  Eight waves cap a wave at 256 VGPRs: the shapes with a wide form,
// head_dim 64 or 128 with GQA chunks of 2+ heads, fit it without spills in all
// three element types (others -- head_dim 256, fp32 head_dim 32 with 8 heads,
// single heads of fp32 head_dim 128 -- would spill); sixteen waves (128 VGPRs)
// would spill the larger GQA groups.
constexpr int kDecodeWideWaves = 8;
constexpr int kDecodeWideTokens = 512;
template <int D, int GT> constexpr bool kDecodeWideOk = (D == 64 || D == 128) && GT >= 2;

// Work-groups of the paired scheduled kernel resident at once on the current
// device (occupancy x CUs), queried once per device and instantiation.
template <typename T, int D, int GT, bool UB>
int scheduled_pair_slots() {
  static std::atomic<long long> slots[kMaxDevices];
  return (int)resident_work_groups(slots, paged_decode_scheduled_kernel<T, D, GT, kDecodeWaves, 2, UB>,
                                   64 * kDecodeWaves);
}

// Work-groups of the partitioned kernel (uniform-tile form) resident at once on
// the current device (occupancy x CUs), queried once per device and instantiation.
template <typename T, int D, int GT>
int partitioned_slots() {
  static std::atomic<long long> slots[kMaxDevices];
  return (int)resident_work_groups(slots, paged_decode_kernel<T, D, GT, kDecodeWaves, true>, 64 * kDecodeWaves);
}

template <typename T>
int decode_partitioned_slots(int head_dim, int gt);

// Whether a scheduled launch may pair KV heads: Hkv even and at least 5/4
// paired items per resident work-group, so that the longest-first order still
// has short items left to fill the end of the launch (with fewer, pairing
// only idles CUs).  The length spread is checked on the device.
template <typename T, int D, int GT>
bool decode_pair_allowed(const DecodeParams& p) {
  if (p.num_kv_heads % 2 != 0) return false;
  const bool ub = decode_uniform_tiles<T, D, GT>(p.block_size, p.partition_size, p.num_kv_heads);
  const int slots = ub ? scheduled_pair_slots<T, D, GT, true>() : scheduled_pair_slots<T, D, GT, false>();
  const long long items = (long long)p.num_seqs * (p.num_kv_heads / 2) * p.head_chunks;
  return 4 * items >= 5LL * slots;
}

template <typename T>
bool decode_pair_allowed(const DecodeParams& p, int head_dim, int gt);

// Launch the decode kernel for element type T: the scheduled kernel when p.sched
// is set (pair: Hkv is even, so rows may take two KV heads; grid B x Hkv x
// head chunks, checked against 2^31 by the caller), else the partitioned
// kernel on `grid`.  Returns false when (D, GT) has no
// instantiation.
template <typename T>
bool launch_paged_decode(const DecodeParams& p, int head_dim, int gt, bool pair, bool wide, dim3 grid,
                         hipStream_t stream);

#define TV_DECODE_SCHEDULED(T, D, GT, HPW, UB)                                                    \
  {                                                                                               \
    hipLaunchKernelGGL((paged_decode_scheduled_kernel<T, D, GT, kDecodeWaves, HPW, UB>),          \
                       dim3(p.num_seqs * p.num_kv_heads * p.head_chunks), dim3(64 * kDecodeWaves), \
                       0, stream, p);                                                             \
    return true;                                                                                  \
  }

#define TV_DECODE_CASE(T, D, GT)                                                                  \
  if (head_dim == D && gt == GT) {                                                                \
    const bool ub = decode_uniform_tiles<T, D, GT>(p.block_size, p.partition_size, p.num_kv_heads); \
    if (p.sched) {                                                                                \
      if (pair && ub) TV_DECODE_SCHEDULED(T, D, GT, 2, true)                                         \
      if (pair) TV_DECODE_SCHEDULED(T, D, GT, 2, false)                                              \
      if (ub) TV_DECODE_SCHEDULED(T, D, GT, 1, true)                                                 \
      TV_DECODE_SCHEDULED(T, D, GT, 1, false)                                                        \
    }                                                                                             \
    if constexpr (kDecodeWideOk<D, GT>) {                                                         \
      if (wide) {                                                                                 \
        if (ub)                                                                                   \
          hipLaunchKernelGGL((paged_decode_kernel<T, D, GT, kDecodeWideWaves, true>), grid,       \
                             dim3(64 * kDecodeWideWaves), 0, stream, p);                          \
        else                                                                                      \
          hipLaunchKernelGGL((paged_decode_kernel<T, D, GT, kDecodeWideWaves, false>), grid,      \
                             dim3(64 * kDecodeWideWaves), 0, stream, p);                          \
        return true;                                                                              \
      }                                                                                           \
    }                                                                                             \
    if (ub)                                                                                       \
      hipLaunchKernelGGL((paged_decode_kernel<T, D, GT, kDecodeWaves, true>), grid,               \
                         dim3(64 * kDecodeWaves), 0, stream, p);                                  \
    else                                                                                          \
      hipLaunchKernelGGL((paged_decode_kernel<T, D, GT, kDecodeWaves, false>), grid,              \
                         dim3(64 * kDecodeWaves), 0, stream, p);                                  \
    return true;                                                                                  \
  }

#define TV_DECODE_ALL_GT(T, D) \
  TV_DECODE_CASE(T, D, 1)      \
  TV_DECODE_CASE(T, D, 2)      \
  TV_DECODE_CASE(T, D, 4)      \
  TV_DECODE_CASE(T, D, 8)

#define TV_DECODE_PAIR_CASE(T, D, GT) \
  if (head_dim == D && gt == GT) return decode_pair_allowed<T, D, GT>(p);
#define TV_DECODE_PAIR_ALL_GT(T, D) \
  TV_DECODE_PAIR_CASE(T, D, 1)      \
  TV_DECODE_PAIR_CASE(T, D, 2)      \
  TV_DECODE_PAIR_CASE(T, D, 4)      \
  TV_DECODE_PAIR_CASE(T, D, 8)

#define TV_DECODE_SLOTS_CASE(T, D, GT) \
  if (head_dim == D && gt == GT) return partitioned_slots<T, D, GT>();
#define TV_DECODE_SLOTS_ALL_GT(T, D) \
  TV_DECODE_SLOTS_CASE(T, D, 1)      \
  TV_DECODE_SLOTS_CASE(T, D, 2)      \
  TV_DECODE_SLOTS_CASE(T, D, 4)      \
  TV_DECODE_SLOTS_CASE(T, D, 8)

#define TV_DECODE_DEFINE(T)                                                                      \
  template <>                                                                                    \
  int decode_partitioned_slots<T>(int head_dim, int gt) {                                        \
    TV_DECODE_SLOTS_ALL_GT(T, 16)                                                                \
    TV_DECODE_SLOTS_ALL_GT(T, 32)                                                                \
    TV_DECODE_SLOTS_ALL_GT(T, 64)                                                                \
    TV_DECODE_SLOTS_ALL_GT(T, 128)                                                               \
    TV_DECODE_SLOTS_ALL_GT(T, 256)                                                               \
    return 0;                                                                                    \
  }                                                                                              \
  template <>                                                                                    \
  bool decode_pair_allowed<T>(const DecodeParams& p, int head_dim, int gt) {                     \
    TV_DECODE_PAIR_ALL_GT(T, 16)                                                                 \
    TV_DECODE_PAIR_ALL_GT(T, 32)                                                                 \
    TV_DECODE_PAIR_ALL_GT(T, 64)                                                                 \
    TV_DECODE_PAIR_ALL_GT(T, 128)                                                                \
    TV_DECODE_PAIR_ALL_GT(T, 256)                                                                \
    return false;                                                                                \
  }                                                                                              \
  template <>                                                                                    \
  bool launch_paged_decode<T>(const DecodeParams& p, int head_dim, int gt, bool pair, bool wide,  \
                              dim3 grid, hipStream_t stream) {                                   \
    TV_DECODE_ALL_GT(T, 16)                                                                      \
    TV_DECODE_ALL_GT(T, 32)                                                                      \
    TV_DECODE_ALL_GT(T, 64)                                                                      \
    TV_DECODE_ALL_GT(T, 128)                                                                     \
    TV_DECODE_ALL_GT(T, 256)                                                                     \
    return false;                                                                                \
  }

}  // namespace tv
