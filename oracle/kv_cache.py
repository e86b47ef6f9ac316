"""numpy restatement of the reference KV cache (test infrastructure).

Layout (tinyvllm/core/kv_cache.py:14, 25-32): per layer one zero-initialised K
and one V array of shape [num_blocks, block_size, n_kv_heads, head_dim]; element
(blk, t, h, d) sits at flat index ((blk*bs + t)*Hkv + h)*D + d.
"""

import numpy as np


class KVCacheRef:
    """Restates ``KVCache`` (tinyvllm/core/kv_cache.py:13-61)."""

    def __init__(self, num_layers, num_blocks, block_size, n_kv_heads, head_dim, dtype):
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.dtype = np.dtype(dtype)
        shape = (num_blocks, block_size, n_kv_heads, head_dim)
        self.k_cache = [np.zeros(shape, self.dtype) for _ in range(num_layers)]
        self.v_cache = [np.zeros(shape, self.dtype) for _ in range(num_layers)]

    def write_kv(self, layer_idx, block_id, start_offset, k, v):
        """kv_cache.py:34-38 -- slice-assign ``k[T,Hkv,D]`` at [block_id, start:start+T]."""
        end = start_offset + k.shape[0]
        self.k_cache[layer_idx][block_id, start_offset:end] = k
        self.v_cache[layer_idx][block_id, start_offset:end] = v

    def read_kv_blocks(self, layer_idx, block_ids, context_len):
        """kv_cache.py:40-55 -- stack listed blocks, flatten, keep the first ``context_len``."""
        if not block_ids:
            z = np.zeros((0, self.n_kv_heads, self.head_dim), self.dtype)
            return z, z.copy()
        k = np.stack([self.k_cache[layer_idx][b] for b in block_ids])
        v = np.stack([self.v_cache[layer_idx][b] for b in block_ids])
        n = len(block_ids) * self.block_size
        k = k.reshape(n, self.n_kv_heads, self.head_dim)
        v = v.reshape(n, self.n_kv_heads, self.head_dim)
        return k[:context_len], v[:context_len]

    def get_memory_bytes(self):
        """kv_cache.py:57-61."""
        return (self.num_layers * self.num_blocks * self.block_size *
                self.n_kv_heads * self.head_dim * 2) * self.dtype.itemsize


def reshape_and_cache_ref(k_cache, v_cache, k, v, slot_mapping):
    """Write token t's K/V rows to flat slot ``slot_mapping[t]`` of the caches.

    The reference performs the same placement one block chunk at a time
    (kv_cache.py:34-38 called from llama.py:203-209 and per token from
    llama.py:382-386); here the per-token slots are explicit.  Slot s addresses
    block ``s // block_size`` row ``s % block_size``.  A negative slot marks a
    padding token and is skipped.  Mutates the caches in place.
    """
    bs = k_cache.shape[1]
    for t, slot in enumerate(np.asarray(slot_mapping).reshape(-1).tolist()):
        if slot < 0:
            continue
        blk, off = divmod(int(slot), bs)
        k_cache[blk, off] = k[t]
        v_cache[blk, off] = v[t]
