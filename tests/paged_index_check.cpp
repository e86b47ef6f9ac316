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
#include <cstdio>
#include <cstdlib>

#include "tv_paged_keys.h"

int main(int argc, char** argv) {
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
