"""Write the small golden fixtures in this directory from the oracle.

The reference ships no golden vectors (its tests are unseeded), so these
fixtures record the oracle's float64 outputs on seeded inputs at tiny shapes,
plus the integer slot/table outputs of a scripted allocation.  They pin the
oracle and the GPU path against regressions; the oracle itself is pinned to
independent references in tests/test_oracle.py.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.attention import flash_prefill_ref, paged_decode_ref  # noqa: E402
from oracle.block_manager import (BlockManagerRef, prepare_batch_tensors_ref,  # noqa: E402
                                  slots_from_plan, write_kv_plan_ref)


def decode_case():
    rng = np.random.Generator(np.random.PCG64(2024))
    hq, hkv, d, bs = 8, 2, 16, 4
    ctx = np.array([17, 33], np.int32)
    nb = 20
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.zeros((2, 10), np.int32)
    bt[0, :5] = perm[:5]
    bt[1, :9] = perm[5:14]
    q = rng.standard_normal((2, 1, hq, d)).astype(np.float32)
    kc = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)
    out = paged_decode_ref(q, kc, vc, bt, ctx, hq, hkv, d, bs)
    np.savez_compressed(os.path.join(HERE, "paged_decode_b2.npz"), q=q, k_cache=kc, v_cache=vc,
                        block_tables=bt, context_lens=ctx, out=out,
                        shape=np.array([hq, hkv, d, bs], np.int32))


def prefill_case():
    rng = np.random.Generator(np.random.PCG64(2025))
    q = rng.standard_normal((1, 16, 4, 16)).astype(np.float32)
    k = rng.standard_normal((1, 16, 2, 16)).astype(np.float32)
    v = rng.standard_normal((1, 16, 2, 16)).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "prefill_l16.npz"), q=q, k=k, v=v,
                        out_causal=flash_prefill_ref(q, k, v, True),
                        out_full=flash_prefill_ref(q, k, v, False))


def slots_case():
    bm = BlockManagerRef(1, 24, 4)
    slots = {}
    for sid, (start, n) in enumerate([(0, 7), (0, 12), (0, 1)]):
        bm.register_sequence(sid)
        slots[f"prefill_{sid}"] = slots_from_plan(write_kv_plan_ref(bm, 0, sid, n, start), 4)
        for _ in range(n):
            bm.advance_position(sid)
    dec = []
    for sid in range(3):
        _, blk, off = bm.get_slot(sid)
        dec.append(blk * 4 + off)
    bt, ctx = prepare_batch_tensors_ref(bm, [0, 1, 2], [7, 12, 1], 4)
    np.savez_compressed(os.path.join(HERE, "slots_3seq.npz"), decode=np.array(dec, np.int32),
                        block_tables=bt, context_lens=ctx, **slots)


if __name__ == "__main__":
    decode_case()
    prefill_case()
    slots_case()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
