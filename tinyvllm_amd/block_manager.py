"""Host-side producers of the integer inputs of the attention path.

``BlockManager`` keeps the reference interface (tinyvllm/core/block_manager.py:6-92):
per-GPU LIFO free lists seeded with ``list(range(blocks_per_gpu))``, per-sequence
block tables grown on demand, reference counts for forks.  On top of it this
module builds, as int32 arrays, the three things the kernels consume:

* ``prefill_slot_mapping`` -- the flat slot ``block_id*bs + pos%bs`` of every
  prompt token, identical to the placement done by the per-chunk loop of
  ``Attention._write_kv_to_blocks`` (llama.py:188-209);
* ``decode_slot_mapping`` -- the slot of each sequence's next token, as obtained
  per sequence from ``get_slot`` in ``Llama.decode`` (llama.py:381-386);
* ``prepare_batch_tensors`` -- zero-padded / truncated block tables and
  ``context_len = start_pos + 1`` (engine.py:235-255, llama.py:368-374).

All three must be bit-exact with the reference logic; they are pure integer
host code with no device work.
"""

import numpy as np


class BlockManager:
    """KV-cache block allocator (reference interface, block_manager.py:6-92)."""

    def __init__(self, num_gpus, blocks_per_gpu, block_size):
        self.num_gpus = num_gpus
        self.blocks_per_gpu = blocks_per_gpu
        self.block_size = block_size
        # LIFO stacks: the next block handed out is the last element.
        self.free_blocks = {g: list(range(blocks_per_gpu)) for g in range(num_gpus)}
        self.ref_counts = {g: np.zeros(blocks_per_gpu, dtype=np.int64) for g in range(num_gpus)}
        self.seq_to_gpu = {}
        self.block_tables = {}
        self.seq_positions = {}

    def register_sequence(self, seq_id, gpu_id=0):
        """Register a sequence with an empty table; blocks are allocated on demand."""
        self.seq_to_gpu[seq_id] = gpu_id
        self.block_tables[seq_id] = []
        self.seq_positions[seq_id] = 0

    def _allocate_until(self, seq_id, n_blocks):
        table = self.block_tables[seq_id]
        gpu = self.seq_to_gpu[seq_id]
        free = self.free_blocks[gpu]
        refs = self.ref_counts[gpu]
        while len(table) < n_blocks:
            if not free:
                raise RuntimeError("Out of KV cache memory!")
            blk = free.pop()
            refs[blk] = 1
            table.append(blk)

    def ensure_block_for_position(self, seq_id, pos):
        """Allocate blocks up to the one holding ``pos``; returns its id."""
        idx = pos // self.block_size
        self._allocate_until(seq_id, idx + 1)
        return self.block_tables[seq_id][idx]

    def get_slot(self, seq_id):
        """(gpu_id, block_id, offset) of the next token to write; allocates if needed."""
        pos = self.seq_positions[seq_id]
        blk = self.ensure_block_for_position(seq_id, pos)
        return self.seq_to_gpu[seq_id], blk, pos % self.block_size

    def advance_position(self, seq_id):
        self.seq_positions[seq_id] += 1

    def get_block_table(self, seq_id):
        return self.block_tables[seq_id]

    def get_context_length(self, seq_id):
        return self.seq_positions[seq_id]

    def get_gpu_for_seq(self, seq_id):
        return self.seq_to_gpu[seq_id]

    def free_sequence(self, seq_id):
        """Drop a sequence; blocks whose count reaches 0 return to the free list in table order."""
        gpu = self.seq_to_gpu.pop(seq_id)
        refs = self.ref_counts[gpu]
        for blk in self.block_tables.pop(seq_id):
            refs[blk] -= 1
            if refs[blk] == 0:
                self.free_blocks[gpu].append(blk)
        del self.seq_positions[seq_id]

    def get_num_free_blocks(self, gpu_id=None):
        if gpu_id is None:
            return sum(len(f) for f in self.free_blocks.values())
        return len(self.free_blocks[gpu_id])

    def fork_sequence(self, src_seq_id, dst_seq_id):
        """Share the source's blocks with a new sequence (reference counted)."""
        gpu = self.seq_to_gpu[src_seq_id]
        self.block_tables[dst_seq_id] = list(self.block_tables[src_seq_id])
        self.seq_to_gpu[dst_seq_id] = gpu
        self.seq_positions[dst_seq_id] = self.seq_positions[src_seq_id]
        for blk in self.block_tables[src_seq_id]:
            self.ref_counts[gpu][blk] += 1

    # -- slot / table producers ------------------------------------------------
    def prefill_slot_mapping(self, seq_id, start_pos, num_tokens, layer_idx=0):
        """int32 [num_tokens]: slot of prompt token i at position start_pos + i.

        Layer 0 allocates the blocks the prompt needs (in position order, as the
        reference's chunk loop does); other layers only look the table up.
        """
        if num_tokens <= 0:
            return np.zeros((0,), dtype=np.int32)
        bs = self.block_size
        last = start_pos + num_tokens - 1
        if layer_idx == 0:
            self._allocate_until(seq_id, last // bs + 1)
        table = np.asarray(self.block_tables[seq_id], dtype=np.int64)
        if table.size <= last // bs:
            raise IndexError("block table does not cover the prompt (allocation happens at layer 0)")
        pos = np.arange(start_pos, last + 1, dtype=np.int64)
        return (table[pos // bs] * bs + pos % bs).astype(np.int32)

    def decode_slot_mapping(self, seq_ids):
        """int32 [B]: slot of each sequence's next token (allocates a block when needed)."""
        out = np.empty((len(seq_ids),), dtype=np.int32)
        for i, sid in enumerate(seq_ids):
            _, blk, off = self.get_slot(sid)
            out[i] = blk * self.block_size + off
        return out

    def prepare_batch_tensors(self, seq_ids, start_positions, max_blocks):
        """(block_tables [B, max_blocks] int32, context_lens [B] int32).

        Rows are the sequences' tables zero-padded or truncated to ``max_blocks``;
        ``context_lens[i] = start_positions[i] + 1``.
        """
        bt = np.zeros((len(seq_ids), max_blocks), dtype=np.int32)
        for i, sid in enumerate(seq_ids):
            table = self.block_tables[sid][:max_blocks]
            bt[i, :len(table)] = table
        ctx = np.asarray(start_positions, dtype=np.int64).reshape(-1) + 1
        return bt, ctx.astype(np.int32)
