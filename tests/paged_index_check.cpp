// Host-side check of the paged prefill kernel's key -> staged-slot mapping,
// using the kernel's own functions (tinyvllm_amd/csrc/tv_paged_keys.h).
//
//   paged_index_check q_len start_pos block_size causal [planted]
//
// For every work unit (64-row query tile) and every kernel shape (1, 2 or 4
// key groups; 32- or 64-key tiles), enumerates the tiles the unit's loads
// request -- steps padded to even and two loads ahead, as the kernel's loop --
// and every row of each tile, maps the row to a key and the key to a staged
// slot, and checks 0 <= slot < staged blocks <= kPagedTableMax.  Prints
// "ok <loads checked>" or the first offending (unit, shape, key, slot) and
// exits 1.  `planted` replaces the clamp to the staged range by a clamp to the
// sequence's last key (a former bug) to show the check catches it.
//
//   paged_index_check split max_nqt [planted]
//
// For every tile count nqt <= max_nqt and first split tile 1 <= split <= nqt
// of the 128-row kernel (rows_split_unit / rows_unit_keys), checks that the
// 2 nqt - split units map to distinct (query tile, half) pairs covering every
// tile once (split tiles as halves 0 and 1), that units come in order of
// non-increasing work, that unit 2 nqt - split maps to no tile, and that the
// two halves of tile qt partition its keys [0, kend) at a multiple of 64 keys
// no later than the tile's first row (every row sees a key in both halves),
// for kend = 128 (qt + 1) and for a prompt whose keys end inside the tile.
// `planted` moves the second half's start 64 keys early (overlapping halves).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "tv_paged_keys.h"

static int check_split(int max_nqt, bool planted) {
  long long checked = 0;
  for (int nqt = 1; nqt <= max_nqt; ++nqt)
    for (int split = 1; split <= nqt; ++split) {
      std::vector<int> seen(2 * nqt, 0);   // [qt][half + 1 .. ] as qt * 2 + (half == 1)
      int prev_work = 1 << 30;
      const int units = 2 * nqt - split;
      for (int u = 0; u < units; ++u) {
        int qt, half;
        tv::rows_split_unit(u, nqt, split, qt, half);
        const bool ok_half = qt >= 0 && qt < nqt && (qt >= split ? (half == 0 || half == 1) : half == -1);
        if (!ok_half) {
          std::printf("nqt %d split %d unit %d -> tile %d half %d\n", nqt, split, u, qt, half);
          return 1;
        }
        const int slot = qt * 2 + (half == 1);
        if (seen[slot]++) {
          std::printf("nqt %d split %d: tile %d half %d dealt twice\n", nqt, split, qt, half);
          return 1;
        }
        const int work = half >= 0 ? qt + 1 : 2 * (qt + 1);
        if (work > prev_work) {
          std::printf("nqt %d split %d unit %d: work %d after %d\n", nqt, split, u, work, prev_work);
          return 1;
        }
        prev_work = work;
        for (int cut = 0; cut < 2; ++cut) {
          // the tile's keys: all 128 (qt + 1), or ending 1 past its first row
          const int kfull = cut ? qt * 128 + 1 : (qt + 1) * 128;
          if (half < 0) continue;
          int b0, e0, b1, e1;
          tv::rows_unit_keys(qt, 0, kfull, b0, e0);
          tv::rows_unit_keys(qt, 1, kfull, b1, e1);
          if (planted) b1 -= 64;
          ++checked;
          if (!(b0 == 0 && e0 == b1 && e1 == kfull && e0 % 64 == 0 && e0 > 0 && b1 <= qt * 128 && b1 < e1)) {
            std::printf("nqt %d split %d tile %d kend %d: halves [%d, %d) [%d, %d)\n", nqt, split, qt, kfull, b0, e0,
                        b1, e1);
            return 1;
          }
        }
      }
      for (int qt = 0; qt < nqt; ++qt)
        if (!seen[qt * 2] || (qt >= split) != (seen[qt * 2 + 1] == 1)) {
          std::printf("nqt %d split %d: tile %d not covered\n", nqt, split, qt);
          return 1;
        }
      int qt, half;
      tv::rows_split_unit(units, nqt, split, qt, half);
      if (qt != -1) {
        std::printf("nqt %d split %d: unit %d past the grid maps to tile %d\n", nqt, split, units, qt);
        return 1;
      }
    }
  std::printf("ok %lld\n", checked);
  return 0;
}

int main(int argc, char** argv) {
  if (argc >= 3 && std::strcmp(argv[1], "split") == 0) return check_split(std::atoi(argv[2]), argc > 3);
  if (argc < 5) {
    std::fprintf(stderr, "usage: %s q_len start_pos block_size causal [planted]\n", argv[0]);
    return 2;
  }
  const int q_len = std::atoi(argv[1]), start = std::atoi(argv[2]), bs = std::atoi(argv[3]);
  const bool causal = std::atoi(argv[4]) != 0, planted = argc > 5;
  int lg = 0;
  while ((1 << lg) < bs) ++lg;
  if ((1 << lg) != bs) return 2;
  const int kv_len = start + q_len, rows = 64, unit_keys = 64;
  const int shapes[][2] = {{1, 64}, {1, 32}, {2, 64}, {2, 32}, {4, 32}};   // (key groups, tile keys)
  long long checked = 0;
  for (int qt = 0; qt * rows < q_len; ++qt) {
    const int kend_full = tv::prefill_unit_key_end(causal, kv_len, qt, rows, start);
    const int nkt = (kend_full + unit_keys - 1) / unit_keys;
    const int kbeg = 0;
    const int klim = nkt * unit_keys < kv_len ? nkt * unit_keys : kv_len;
    const int kend = tv::prefill_unit_key_end(causal, klim, qt, rows, start);
    const int stage_end = tv::paged_stage_end(kbeg, kend);
    const int nblk = tv::paged_staged_blocks(kbeg, stage_end, lg);
    if (nblk > tv::kPagedTableMax) {
      std::printf("table of %d blocks exceeds %d (unit %d)\n", nblk, tv::kPagedTableMax, qt);
      return 1;
    }
    for (const auto& sh : shapes) {
      const int groups = sh[0], bn = sh[1];
      const int ntiles = (kend - kbeg + bn - 1) / bn;
      const int nsteps = (ntiles + groups - 1) / groups;
      const int nsteps2 = (nsteps + 1) & ~1;
      for (int grp = 0; grp < groups; ++grp)
        for (int j = 0; j <= nsteps2 + 2; ++j) {
          const int tile = tv::prefill_group_tile(grp, groups, j, ntiles);
          for (int row = 0; row < bn; ++row) {
            int key = tv::paged_load_key(kbeg, planted ? kv_len : stage_end, tile, bn, row);
            const int slot = tv::paged_stage_slot(key, kbeg, lg);
            ++checked;
            if (slot < 0 || slot >= nblk) {
              std::printf("unit %d groups %d tile_keys %d key %d slot %d of %d staged\n", qt, groups, bn, key, slot,
                          nblk);
              return 1;
            }
          }
        }
    }
  }
  std::printf("ok %lld\n", checked);
  return 0;
}
