// Key / value tiles loaded straight into LDS (gfx950 LDS DMA) for the prefill
// kernels: buffer descriptors, the 16-byte-chunk permutation of tile rows, the
// load itself and the vmcnt wait that retires it.
#pragma once

#include "tv_common.h"

namespace tv {

// Chunk permutation of tile row r (16-byte chunks; 16 per row at head_dim 128,
// 8 at 64): distinct over any 16 consecutive rows for a fixed chunk (the K
// fragment reads of ds_read_b128), and keeps the chunk pairs {2u, 2u+1} of 4
// consecutive rows on distinct banks (the transposing V reads of
// ds_read_b64_tr_b16).  Depends on r & 15 only, so 16-row blocks of a tile share
// their offsets.
template <int D> __device__ __forceinline__ int tile_chunk_perm(int r) {
  if constexpr (D == 128) return ((r & 7) << 1) | ((r >> 3) & 1);
  else return (((r >> 1) & 3) << 1) | ((r >> 3) & 1);
}

// 16 bytes per lane from buffer `rsrc` at byte offset voff straight into LDS at
// lds_base + 16 * lane.  The compiler does not see these loads: callers retire
// them with wait_vmcnt before the barrier that publishes the tile.
__device__ __forceinline__ void load_lds16(u32x4 rsrc, uint32_t lds_base, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_base), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}

// Wait until at most N vector-memory operations of this wave are outstanding
// (gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ uint32_t sgpr(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// Raw buffer descriptor words over [base, base + bytes); the range is clamped to
// 32 bits with a scalar compare of the high word (as C the compiler makes it a
// 64-bit vector compare plus readfirstlane).  Loads at or past the range return
// zero, which is how tile rows past the last key arrive as zeros.
__device__ __forceinline__ u32x4 rsrc_words(const void* base, unsigned long long bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  uint32_t n;
  asm("s_cmp_lg_u32 %1, 0\n\ts_cselect_b32 %0, -1, %2"
      : "=s"(n)
      : "s"((uint32_t)(bytes >> 32)), "s"((uint32_t)bytes)
      : "scc");
  return u32x4{sgpr((uint32_t)a), sgpr((uint32_t)(a >> 32)), n, 0x00020000u};
}

}  // namespace tv
