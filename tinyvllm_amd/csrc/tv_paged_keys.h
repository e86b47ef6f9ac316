// Index arithmetic of the prefill kernels, shared by host and device.
//
// Key -> staged block-table slot mapping of the paged prefill kernel
// (prefill_fa_kernel<..., PAGED = true>, flash_prefill.hip).  A work-group
// stages the block ids of its key range [kbeg, stage_end) in LDS and reads
// every K / V row through that table -- padded rows of a partial tile and the
// clamped re-reads of the last tile included.  And the unit -> (query tile,
// key half) map of the 128-row kernel's split causal grids.  These functions
// are the kernels' own arithmetic; tests/paged_index_check.cpp runs them on
// the host over the tested shapes and checks that every slot stays inside the
// table and that the split units cover every query tile's keys exactly once.
#pragma once

#include <hip/hip_runtime.h>

namespace tv {

// Block ids a paged work-group can stage (keys of 65536 tokens at block size 16).
constexpr int kPagedTableMax = 4096;

// End of a query tile's key range: causal rows see keys j <= i + q_pos_offset.
__host__ __device__ inline int prefill_unit_key_end(bool causal, int klim, int qt, int rows, int q_pos_offset) {
  const int diag = (qt + 1) * rows + q_pos_offset;
  return causal ? (klim < diag ? klim : diag) : klim;
}

// Keys whose block ids are staged: [kbeg, paged_stage_end).  At least one key,
// so an empty range still stages a valid id.
__host__ __device__ inline int paged_stage_end(int kbeg, int kend) { return kend > kbeg + 1 ? kend : kbeg + 1; }

// Block ids staged for keys [kbeg, stage_end) at block size 2^lg.
__host__ __device__ inline int paged_staged_blocks(int kbeg, int stage_end, int lg) {
  return ((stage_end - 1) >> lg) - (kbeg >> lg) + 1;
}

// The key a load of tile row `row` reads: keys at or past the staged range
// (masked for every row of the unit) re-read the last staged key.
__host__ __device__ inline int paged_load_key(int kbeg, int stage_end, int tile, int tile_keys, int row) {
  const int key = kbeg + tile * tile_keys + row;
  const int hi = stage_end - 1;
  return key < kbeg ? kbeg : (key > hi ? hi : key);
}

// Tile that key group `grp` (of `groups`) loads at its step j: tiles
// grp, grp + groups, ...; steps past the last tile re-request the last tile.
__host__ __device__ inline int prefill_group_tile(int grp, int groups, int j, int ntiles) {
  const int t = grp + groups * j;
  return t < ntiles - 1 ? t : ntiles - 1;
}

// Slot of `key`'s block id in the staged table.
__host__ __device__ inline int paged_stage_slot(int key, int kbeg, int lg) { return (key >> lg) - (kbeg >> lg); }

// 128-row prefill kernel with split query tiles (prefill_rows_kernel,
// flash_prefill_rows.hip): tiles qt >= split run as two units over the key
// halves [0, 64 (qt + 1)) and [64 (qt + 1), kend), tiles below split as one
// unit.  Unit u of a head -> (qt, half), half -1 for an unsplit tile; units
// ordered by decreasing work: a half of tile qt walks qt + 1 pairs of 32-key
// tiles, an unsplit tile 2 (qt + 1).  Units per head: 2 nqt - split.
__host__ __device__ inline void rows_split_unit(int u, int nqt, int split, int& qt, int& half) {
  const int top = nqt > 2 * split ? nqt : 2 * split;
  for (int c = top; c >= 1; --c) {
    if (c - 1 >= split && c - 1 < nqt) {
      if (u < 2) {
        qt = c - 1;
        half = u;
        return;
      }
      u -= 2;
    }
    if ((c & 1) == 0 && c / 2 - 1 < split) {
      if (u == 0) {
        qt = c / 2 - 1;
        half = -1;
        return;
      }
      u -= 1;
    }
  }
  qt = -1;   // u >= 2 nqt - split
  half = -1;
}

// Key range [kbeg, kend) of a unit of the 128-row kernel; kfull is the
// tile's whole causal range.
__host__ __device__ inline void rows_unit_keys(int qt, int half, int kfull, int& kbeg, int& kend) {
  const int mid = (qt + 1) * 64;
  kbeg = half == 1 ? mid : 0;
  kend = half == 0 ? mid : kfull;
}

}  // namespace tv
