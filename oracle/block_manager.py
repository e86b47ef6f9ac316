"""Restatement of the reference's slot / block-table producers (test infrastructure).

These are the integer contracts the GPU path consumes; they must be bit-exact.
"""

import numpy as np


class BlockManagerRef:
    """Restates ``BlockManager`` (tinyvllm/core/block_manager.py:6-92).

    Free list per GPU is ``list(range(blocks_per_gpu))`` and allocation pops from
    its end (LIFO), so the first block handed out is ``blocks_per_gpu - 1``
    (block_manager.py:13-15, 37); freed blocks are appended back (:71).
    """

    def __init__(self, num_gpus, blocks_per_gpu, block_size):
        self.num_gpus = num_gpus
        self.blocks_per_gpu = blocks_per_gpu
        self.block_size = block_size
        self.free_blocks = {g: list(range(blocks_per_gpu)) for g in range(num_gpus)}
        self.ref_counts = {g: {b: 0 for b in range(blocks_per_gpu)} for g in range(num_gpus)}
        self.seq_to_gpu = {}
        self.block_tables = {}
        self.seq_positions = {}

    def register_sequence(self, seq_id, gpu_id=0):
        self.seq_to_gpu[seq_id] = gpu_id
        self.block_tables[seq_id] = []
        self.seq_positions[seq_id] = 0

    def ensure_block_for_position(self, seq_id, pos):
        idx = pos // self.block_size
        while len(self.block_tables[seq_id]) <= idx:
            g = self.seq_to_gpu[seq_id]
            if not self.free_blocks[g]:
                raise RuntimeError("Out of KV cache memory!")
            b = self.free_blocks[g].pop()
            self.ref_counts[g][b] = 1
            self.block_tables[seq_id].append(b)
        return self.block_tables[seq_id][idx]

    def get_slot(self, seq_id):
        pos = self.seq_positions[seq_id]
        b = self.ensure_block_for_position(seq_id, pos)
        return (self.seq_to_gpu[seq_id], b, pos % self.block_size)

    def advance_position(self, seq_id):
        self.seq_positions[seq_id] += 1

    def get_block_table(self, seq_id):
        return self.block_tables[seq_id]

    def get_context_length(self, seq_id):
        return self.seq_positions[seq_id]

    def free_sequence(self, seq_id):
        g = self.seq_to_gpu[seq_id]
        for b in self.block_tables[seq_id]:
            self.ref_counts[g][b] -= 1
            if self.ref_counts[g][b] == 0:
                self.free_blocks[g].append(b)
        del self.seq_to_gpu[seq_id]
        del self.block_tables[seq_id]
        del self.seq_positions[seq_id]

    def get_num_free_blocks(self, gpu_id=None):
        if gpu_id is None:
            return sum(len(v) for v in self.free_blocks.values())
        return len(self.free_blocks[gpu_id])

    def fork_sequence(self, src, dst):
        g = self.seq_to_gpu[src]
        self.block_tables[dst] = self.block_tables[src].copy()
        self.seq_to_gpu[dst] = g
        self.seq_positions[dst] = self.seq_positions[src]
        for b in self.block_tables[src]:
            self.ref_counts[g][b] += 1


def write_kv_plan_ref(block_manager, layer_idx, seq_id, seq_len, start_pos):
    """Restates the chunk loop of ``Attention._write_kv_to_blocks`` (llama.py:188-209).

    Returns the list of (block_id, offset, token_start, n_tokens) write calls the
    reference would issue, allocating through the block manager at layer 0 only.
    """
    bs = block_manager.block_size
    calls = []
    token_idx, pos = 0, start_pos
    while token_idx < seq_len:
        offset = pos % bs
        n = min(bs - offset, seq_len - token_idx)
        if layer_idx == 0:
            blk = block_manager.ensure_block_for_position(seq_id, pos)
        else:
            blk = block_manager.get_block_table(seq_id)[pos // bs]
        calls.append((blk, offset, token_idx, n))
        token_idx += n
        pos += n
    return calls


def slots_from_plan(calls, block_size):
    """Flatten a write plan into per-token slots ``block_id*bs + offset + i``."""
    out = []
    for blk, offset, _tok, n in calls:
        out.extend(blk * block_size + offset + i for i in range(n))
    return np.asarray(out, dtype=np.int32)


def prepare_batch_tensors_ref(block_manager, seq_ids, start_positions, max_blocks):
    """Restates ``LLMEngine._prepare_batch_tensors`` (engine.py:235-255).

    bt[i, j] = table_i[j] for j < len(table_i), else 0, for j < max_blocks (longer
    tables are truncated); ctx[i] = start_pos_i + 1.
    """
    b = len(seq_ids)
    bt = np.zeros((b, max_blocks), dtype=np.int32)
    ctx = np.zeros((b,), dtype=np.int32)
    for i, (sid, sp) in enumerate(zip(seq_ids, start_positions)):
        table = block_manager.get_block_table(sid)
        for j in range(max_blocks):
            bt[i, j] = table[j] if j < len(table) else 0
        ctx[i] = sp + 1
    return bt, ctx


def pad_or_truncate_ref(block_tables, max_blocks):
    """Restates the pad/truncate in ``Llama.decode`` (llama.py:368-374)."""
    bt = np.asarray(block_tables, dtype=np.int32)
    cur = bt.shape[1]
    if cur < max_blocks:
        return np.concatenate([bt, np.zeros((bt.shape[0], max_blocks - cur), np.int32)], axis=1)
    return bt[:, :max_blocks]
