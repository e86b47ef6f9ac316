"""MI355X (gfx950) attention hot path for tinyvllm.

Drop-in entry points (reference signatures, tinyvllm/model/llama.py and
tinyvllm/core/kv_cache.py):

    from tinyvllm_amd.attention import paged_decode_attention, flash_prefill_attention
    from tinyvllm_amd.kv_cache import KVCache, reshape_and_cache
    from tinyvllm_amd.block_manager import BlockManager

The kernels live in libtvattn.so (built by ``python -m tinyvllm_amd.build``);
the ops raise if it is missing.
"""

__all__ = ["attention", "kv_cache", "block_manager", "workloads", "build"]
