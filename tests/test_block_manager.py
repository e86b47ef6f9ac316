"""Host-side integer producers: bit-exact against the oracle's restatement.

Covers the slot mapping of prefill (llama.py:188-209), the decode-step slots
(llama.py:381-386), block tables / context lengths (engine.py:235-255,
llama.py:368-374) and the allocator itself (block_manager.py:6-92).
"""

import numpy as np
import pytest

from oracle.block_manager import (BlockManagerRef, pad_or_truncate_ref, prepare_batch_tensors_ref,
                                  slots_from_plan, write_kv_plan_ref)
from tinyvllm_amd.block_manager import BlockManager


def _state(bm):
    tables = {k: list(v) for k, v in bm.block_tables.items()}
    free = {g: list(v) for g, v in bm.free_blocks.items()}
    refs = {g: [int(bm.ref_counts[g][b]) for b in range(bm.blocks_per_gpu)] for g in bm.free_blocks}
    return tables, free, refs, dict(bm.seq_positions), dict(bm.seq_to_gpu)


def test_lifo_allocation_order():
    bm = BlockManager(1, 10, 4)
    bm.register_sequence(0)
    assert bm.ensure_block_for_position(0, 0) == 9
    assert bm.ensure_block_for_position(0, 9) == 7        # blocks 9, 8, 7 for positions 0..11
    assert bm.get_block_table(0) == [9, 8, 7]


def test_out_of_memory():
    bm = BlockManager(1, 2, 4)
    bm.register_sequence(0)
    bm.ensure_block_for_position(0, 7)
    with pytest.raises(RuntimeError, match="Out of KV cache memory"):
        bm.ensure_block_for_position(0, 8)


@pytest.mark.parametrize("seed", range(6))
def test_random_script_matches_reference(seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    nblk, bs = 40, int(rng.choice([1, 4, 16]))
    ref, new = BlockManagerRef(2, nblk, bs), BlockManager(2, nblk, bs)
    live, next_id = [], 0
    for _ in range(200):
        op = rng.integers(0, 6)
        try:
            if op == 0 or not live:
                gpu = int(rng.integers(0, 2))
                ref.register_sequence(next_id, gpu)
                new.register_sequence(next_id, gpu)
                live.append(next_id)
                next_id += 1
            elif op == 1:
                sid = live[rng.integers(len(live))]
                pos = int(rng.integers(0, 3 * bs + 1))
                r = ref.ensure_block_for_position(sid, pos)
                assert new.ensure_block_for_position(sid, pos) == r
            elif op == 2:
                sid = live[rng.integers(len(live))]
                assert new.get_slot(sid) == ref.get_slot(sid)
                ref.advance_position(sid)
                new.advance_position(sid)
            elif op == 3:
                sid = live.pop(rng.integers(len(live)))
                ref.free_sequence(sid)
                new.free_sequence(sid)
            elif op == 4:
                src = live[rng.integers(len(live))]
                ref.fork_sequence(src, next_id)
                new.fork_sequence(src, next_id)
                live.append(next_id)
                next_id += 1
            else:
                sid = live[rng.integers(len(live))]
                start = new.get_context_length(sid)
                n = int(rng.integers(1, 2 * bs + 2))
                err_ref = err_new = None
                try:
                    want = slots_from_plan(write_kv_plan_ref(ref, 0, sid, n, start), bs)
                except RuntimeError as e:
                    err_ref = str(e)
                try:
                    got = new.prefill_slot_mapping(sid, start, n, layer_idx=0)
                except RuntimeError as e:
                    err_new = str(e)
                assert err_ref == err_new
                if err_ref is not None:
                    raise RuntimeError(err_ref)
                assert got.dtype == np.int32 and np.array_equal(got, want)
                # later layers look the table up and must give the same slots
                want1 = slots_from_plan(write_kv_plan_ref(ref, 1, sid, n, start), bs)
                assert np.array_equal(new.prefill_slot_mapping(sid, start, n, layer_idx=1), want1)
        except RuntimeError as e:
            assert "Out of KV cache memory" in str(e)
            # both must have failed at the same point: replay the state comparison
        assert _state(new) == _state(ref)


def test_prefill_slots_match_chunk_loop_brute_force():
    """Every prompt token lands at table[p // bs] * bs + p % bs (llama.py:199-209)."""
    for bs in (1, 3, 4, 16):
        for start in (0, 1, bs - 1, bs, 2 * bs + 1):
            for n in (1, bs, bs + 1, 3 * bs + 2):
                ref, new = BlockManagerRef(1, 64, bs), BlockManager(1, 64, bs)
                ref.register_sequence(7)
                new.register_sequence(7)
                plan = write_kv_plan_ref(ref, 0, 7, n, start)
                got = new.prefill_slot_mapping(7, start, n)
                table = ref.get_block_table(7)
                brute = [table[p // bs] * bs + p % bs for p in range(start, start + n)]
                assert got.tolist() == brute == slots_from_plan(plan, bs).tolist()
                # every chunk of the plan stays inside one block
                for blk, off, _tok, cnt in plan:
                    assert 0 <= off and off + cnt <= bs


def test_decode_slots_match_get_slot():
    ref, new = BlockManagerRef(1, 50, 4), BlockManager(1, 50, 4)
    for sid, n in enumerate([3, 4, 9, 0]):
        for bm in (ref, new):
            bm.register_sequence(sid)
            if n:
                bm.ensure_block_for_position(sid, n - 1)
            for _ in range(n):
                bm.advance_position(sid)
    got = new.decode_slot_mapping([0, 1, 2, 3])
    want = []
    for sid in range(4):
        _, blk, off = ref.get_slot(sid)
        want.append(blk * 4 + off)
    assert got.dtype == np.int32 and got.tolist() == want
    assert _state(new) == _state(ref)


@pytest.mark.parametrize("max_blocks", [1, 3, 8, 64])
def test_prepare_batch_tensors_matches_engine(max_blocks):
    ref, new = BlockManagerRef(1, 200, 4), BlockManager(1, 200, 4)
    lens = [1, 5, 17, 33, 0]
    for sid, n in enumerate(lens):
        for bm in (ref, new):
            bm.register_sequence(sid)
            if n:
                bm.ensure_block_for_position(sid, n - 1)
    starts = [max(n - 1, 0) for n in lens]
    bt, ctx = new.prepare_batch_tensors(list(range(5)), starts, max_blocks)
    bt_r, ctx_r = prepare_batch_tensors_ref(ref, list(range(5)), starts, max_blocks)
    assert bt.dtype == np.int32 and ctx.dtype == np.int32
    assert np.array_equal(bt, bt_r) and np.array_equal(ctx, ctx_r)
    # Llama.decode's pad/truncate to the JIT width is idempotent on these tables
    assert np.array_equal(pad_or_truncate_ref(bt, max_blocks), bt)
    wider = pad_or_truncate_ref(bt, max_blocks + 3)
    assert wider.shape == (5, max_blocks + 3) and not wider[:, max_blocks:].any()


def _literal_script(cls):
    """10 blocks of 4 tokens, LIFO from list(range(10)) (block_manager.py:13-15,
    37): sequence 0 holds 6 tokens, 1 holds 1, 2 holds 13, 3 is registered
    with none."""
    bm = cls(1, 10, 4)
    for sid, n in enumerate([6, 1, 13, 0]):
        bm.register_sequence(sid)
        if n:
            bm.ensure_block_for_position(sid, n - 1)
    return bm


# Hand-enumerated from the reference's rules, not from either implementation:
# tables 0: [9, 8], 1: [7], 2: [6, 5, 4, 3], 3: []; rows zero-padded or
# truncated to max_blocks (engine.py:246-250); ctx = start + 1 (engine.py:251).
LITERAL_STARTS = [5, 0, 12, 0]
LITERAL_CTX = [6, 1, 13, 1]
LITERAL_BT = {
    3: [[9, 8, 0], [7, 0, 0], [6, 5, 4], [0, 0, 0]],                                 # sequence 2 truncated
    5: [[9, 8, 0, 0, 0], [7, 0, 0, 0, 0], [6, 5, 4, 3, 0], [0, 0, 0, 0, 0]],
    1: [[9], [7], [6], [0]],
}


@pytest.mark.parametrize("max_blocks", sorted(LITERAL_BT))
def test_prepare_batch_tensors_hand_enumerated(max_blocks):
    for cls in (BlockManager, BlockManagerRef):
        bm = _literal_script(cls)
        assert [bm.get_block_table(s) for s in range(4)] == [[9, 8], [7], [6, 5, 4, 3], []]
        if cls is BlockManager:
            bt, ctx = bm.prepare_batch_tensors([0, 1, 2, 3], LITERAL_STARTS, max_blocks)
        else:
            bt, ctx = prepare_batch_tensors_ref(bm, [0, 1, 2, 3], LITERAL_STARTS, max_blocks)
        assert bt.dtype == np.int32 and ctx.dtype == np.int32
        assert bt.tolist() == LITERAL_BT[max_blocks], cls
        assert ctx.tolist() == LITERAL_CTX, cls


def test_pad_or_truncate_hand_enumerated():
    # Llama.decode's pad / truncate to the JIT width (llama.py:368-374)
    bt = np.array(LITERAL_BT[5], np.int32)
    assert pad_or_truncate_ref(bt, 2).tolist() == [[9, 8], [7, 0], [6, 5], [0, 0]]
    assert pad_or_truncate_ref(bt, 7).tolist() == [[9, 8, 0, 0, 0, 0, 0], [7, 0, 0, 0, 0, 0, 0],
                                                   [6, 5, 4, 3, 0, 0, 0], [0, 0, 0, 0, 0, 0, 0]]
    assert pad_or_truncate_ref(bt, 5).tolist() == LITERAL_BT[5]


def test_slot_mapping_hand_enumerated():
    """slot = block_id * block_size + position % block_size (llama.py:199-209),
    worked out by hand for 6 blocks of 4 tokens, LIFO: a 6-token prompt takes
    blocks 5, 4; a 3-token prompt block 3; decode then writes position 6 of the
    first sequence at block 4 offset 2, and its position 8 opens block 2."""
    for cls in (BlockManager, BlockManagerRef):
        bm = cls(1, 6, 4)
        bm.register_sequence(0)
        bm.register_sequence(1)
        if cls is BlockManager:
            s0 = bm.prefill_slot_mapping(0, 0, 6).tolist()
            s1 = bm.prefill_slot_mapping(1, 0, 3).tolist()
        else:
            s0 = slots_from_plan(write_kv_plan_ref(bm, 0, 0, 6, 0), 4)   # layer 0, sequence 0, 6 tokens from 0
            s1 = slots_from_plan(write_kv_plan_ref(bm, 0, 1, 3, 0), 4)
        assert list(s0) == [20, 21, 22, 23, 16, 17], cls
        assert list(s1) == [12, 13, 14], cls
        for _ in range(6):
            bm.advance_position(0)
        for _ in range(3):
            bm.advance_position(1)
        _, blk, off = bm.get_slot(0)
        assert (blk, off) == (4, 2)
        bm.advance_position(0)
        bm.advance_position(0)
        _, blk, off = bm.get_slot(0)                      # position 8: a new block, popped LIFO
        assert (blk, off) == (2, 0)
        assert bm.get_block_table(0) == [5, 4, 2]
