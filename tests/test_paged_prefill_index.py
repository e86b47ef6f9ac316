"""Index arithmetic of the paged prefill kernel, restated on the CPU.

`prefill_fa_kernel<..., PAGED = true>` (tinyvllm_amd/csrc/flash_prefill.hip)
stages the block ids of a work-group's key range [kbeg, kstage) in LDS and
maps every key a K/V load touches -- padded rows of a partial tile and the
unconditional prefetch of tiles past the last one included -- to a staged
slot.  This file restates that mapping and checks that every slot index stays
inside the staged range for the shapes the GPU tests and the bench launch,
for both key-tile widths (32 and 64).  The earlier clamp (to the last key of
the sequence instead of the last staged key) is planted and must fail.
"""

import pytest


def cdiv(a, b):
    return -(-a // b)


def staged_slots(q_len, start, bs, causal, bn, clamp_to_kv_len=False, rows=64):
    """Yield (slot index, staged count) for every key a work-group's K/V loads touch."""
    kv_len = start + q_len
    lg = bs.bit_length() - 1
    assert 1 << lg == bs
    for qt in range(cdiv(q_len, rows)):
        kend = min(kv_len, (qt + 1) * rows + start) if causal else kv_len
        kbeg = 0
        ntiles = cdiv(kend - kbeg, bn)
        kstage = max(kend, kbeg + 1)                 # keys whose block ids are staged: [kbeg, kstage)
        blk0 = kbeg >> lg
        nblk = ((kstage - 1) >> lg) - blk0 + 1
        hi = kv_len - 1 if clamp_to_kv_len else kstage - 1
        # tiles 0 .. ntiles-1, plus prefetches of later tiles that re-read the last one
        for t in list(range(ntiles)) + [ntiles - 1]:
            for row in range(bn):
                key = max(kbeg, min(kbeg + t * bn + row, hi))
                yield (key >> lg) - blk0, nblk


CASES = [
    # (q_len, start_pos, block_size, causal): the GPU tests' shapes and the bench's
    (100, 0, 16, True), (77, 300, 16, True), (256, 1000, 16, True), (64, 64, 4, True),
    (50, 200, 32, False), (512, 3584, 16, True), (16, 64, 16, True),
    (37, 0, 16, True), (50, 37, 16, True), (5, 87, 16, True), (33, 31, 128, True), (1, 4095, 1, True),
]


@pytest.mark.parametrize("bn", [32, 64])
@pytest.mark.parametrize("q_len,start,bs,causal", CASES)
def test_every_touched_key_maps_to_a_staged_slot(q_len, start, bs, causal, bn):
    for idx, nblk in staged_slots(q_len, start, bs, causal, bn):
        assert 0 <= idx < nblk
        assert nblk <= 4096      # the kernel's LDS table size


def test_the_old_clamp_reads_past_the_staged_table():
    bad = [(idx, nblk) for idx, nblk in staged_slots(77, 300, 16, True, 64, clamp_to_kv_len=True)
           if not 0 <= idx < nblk]
    assert bad, "the planted clamp should reach an unstaged slot"
