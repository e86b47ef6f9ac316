"""Paged KV cache with the reference's interface (tinyvllm/core/kv_cache.py:13-61).

Storage per layer: one K and one V tensor [num_blocks, block_size, n_kv_heads,
head_dim], zero-initialised, dense, on a HIP device.  Element (blk, t, h, d)
sits at ((blk*bs + t)*Hkv + h)*D + d, the layout paged_decode_attention reads.
All writes and reads go through libtvattn.so kernels.
"""

import numpy as np
import torch

from . import _lib

_lib.load()

_DTYPES = {
    "float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
    "half": torch.float16, "float": torch.float32,
}


def as_torch_dtype(dtype):
    """Accept a torch dtype, a numpy dtype or a name ('float16', ...)."""
    if isinstance(dtype, torch.dtype):
        return dtype
    if isinstance(dtype, str):
        return _DTYPES[dtype]
    name = getattr(dtype, "name", None) or np.dtype(dtype).name
    return _DTYPES[name]


class KVCache:
    """Block-based KV cache.  Shape per layer: [num_blocks, block_size, n_kv_heads, head_dim]."""

    def __init__(self, num_layers, num_blocks, block_size, n_kv_heads, head_dim, dtype, device="cuda"):
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.dtype = as_torch_dtype(dtype)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("KVCache storage must be on a HIP device")
        shape = (num_blocks, block_size, n_kv_heads, head_dim)
        self.k_cache = [torch.zeros(shape, dtype=self.dtype, device=self.device) for _ in range(num_layers)]
        self.v_cache = [torch.zeros(shape, dtype=self.dtype, device=self.device) for _ in range(num_layers)]

    # -- helpers -------------------------------------------------------------
    def _rows(self, x, name):
        """View ``x`` as [T, Hkv*D] rows with a token stride; validates layout."""
        if x.dim() == 2:          # a single token [Hkv, D]
            x = x.unsqueeze(0)
        if x.dim() != 3 or tuple(x.shape[1:]) != (self.n_kv_heads, self.head_dim):
            raise ValueError(f"{name} must be [T, {self.n_kv_heads}, {self.head_dim}], got {tuple(x.shape)}")
        if x.dtype != self.dtype:
            raise ValueError(f"{name} dtype {x.dtype} differs from cache dtype {self.dtype}")
        if x.device != self.k_cache[0].device:
            raise ValueError(f"{name} must be on {self.k_cache[0].device}")
        if x.shape[0] > 1 and not (x.stride(2) == 1 and x.stride(1) == self.head_dim):
            raise ValueError(f"{name}: heads and head_dim must be contiguous")
        stride = x.stride(0) if x.shape[0] > 1 else self.n_kv_heads * self.head_dim
        return x, stride

    # -- reference API -------------------------------------------------------
    def write_kv(self, layer_idx, block_id, start_offset, k, v):
        """Write k/v [T, Hkv, D] to [block_id, start_offset:start_offset+T] (kv_cache.py:34-38)."""
        k, ks = self._rows(k, "k")
        v, vs = self._rows(v, "v")
        if k.shape[0] != v.shape[0]:
            raise ValueError("k and v must hold the same number of tokens")
        lib = _lib.load()
        rc = lib.tv_write_kv(
            self.k_cache[layer_idx].data_ptr(), self.v_cache[layer_idx].data_ptr(),
            k.data_ptr(), v.data_ptr(), int(block_id), int(start_offset), k.shape[0],
            self.n_kv_heads, self.head_dim, self.block_size, self.num_blocks, ks, vs,
            _lib.dtype_code(self.dtype), _lib.stream_ptr(self.device))
        _lib.check(rc, "KVCache.write_kv")

    def read_kv_blocks(self, layer_idx, block_ids, context_len):
        """Return (k, v) [context_len, Hkv, D] gathered from ``block_ids`` (kv_cache.py:40-55)."""
        shape = (0, self.n_kv_heads, self.head_dim)
        if not block_ids:
            return (torch.zeros(shape, dtype=self.dtype, device=self.device),
                    torch.zeros(shape, dtype=self.dtype, device=self.device))
        n = min(int(context_len), len(block_ids) * self.block_size)
        if n < 0:
            raise ValueError("context_len must be >= 0")
        k_out = torch.empty((n, self.n_kv_heads, self.head_dim), dtype=self.dtype, device=self.device)
        v_out = torch.empty_like(k_out)
        if n == 0:
            return k_out, v_out
        ids = torch.tensor(list(block_ids), dtype=torch.int32).to(self.device)
        lib = _lib.load()
        rc = lib.tv_read_kv_blocks(
            k_out.data_ptr(), v_out.data_ptr(),
            self.k_cache[layer_idx].data_ptr(), self.v_cache[layer_idx].data_ptr(),
            ids.data_ptr(), len(block_ids), n, self.n_kv_heads, self.head_dim, self.block_size,
            self.num_blocks, _lib.dtype_code(self.dtype), _lib.stream_ptr(self.device))
        _lib.check(rc, "KVCache.read_kv_blocks")
        return k_out, v_out

    def get_memory_bytes(self):
        """Total bytes of K and V storage over all layers (kv_cache.py:57-61)."""
        return (self.num_layers * self.num_blocks * self.block_size *
                self.n_kv_heads * self.head_dim * 2) * self.dtype.itemsize

    # -- fused path (no reference counterpart) --------------------------------
    def write_kv_slots(self, layer_idx, slot_mapping, k, v, err_count=None):
        """Write token t of k/v [T, Hkv, D] to flat slot ``slot_mapping[t]`` in one launch.

        Replaces the per-chunk ``write_kv`` loop of llama.py:199-209 and the
        per-token loop of llama.py:381-386.  ``slot_mapping`` is an int32 device
        tensor [T]; negative slots are skipped.  ``err_count`` (uint32/int32
        device scalar) counts tokens whose slot is past the cache.
        """
        return reshape_and_cache(self.k_cache[layer_idx], self.v_cache[layer_idx], k, v,
                                 slot_mapping, err_count=err_count)


def reshape_and_cache(k_cache, v_cache, k, v, slot_mapping, err_count=None):
    """Fused cache write: ``cache[slot // bs, slot % bs] = row`` for every token."""
    nb, bs, hkv, d = k_cache.shape
    if tuple(v_cache.shape) != (nb, bs, hkv, d) or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache / v_cache must be dense [NB, bs, Hkv, D] tensors of one shape")
    if k.dim() != 3 or tuple(k.shape[1:]) != (hkv, d) or tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"k/v must be [T, {hkv}, {d}]")
    if not (k.stride(2) == 1 and k.stride(1) == d and v.stride(2) == 1 and v.stride(1) == d):
        raise ValueError("k/v heads and head_dim must be contiguous")
    if k.dtype != k_cache.dtype or v.dtype != k_cache.dtype:
        raise ValueError("k/v dtype must match the cache dtype")
    if slot_mapping.dtype != torch.int32 or slot_mapping.numel() != k.shape[0]:
        raise ValueError("slot_mapping must be int32 with one entry per token")
    if not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be contiguous")
    dev = k_cache.device
    for t in (v_cache, k, v, slot_mapping):
        if t.device != dev:
            raise ValueError("all tensors must be on the cache's device")
    if err_count is not None and (err_count.device != dev or err_count.dtype not in (torch.int32, torch.uint32)):
        raise ValueError("err_count must be an int32/uint32 tensor on the cache's device")
    lib = _lib.load()
    t = k.shape[0]
    rc = lib.tv_reshape_and_cache(
        k_cache.data_ptr(), v_cache.data_ptr(), k.data_ptr(), v.data_ptr(), slot_mapping.data_ptr(),
        t, hkv, d, bs, nb, k.stride(0) if t > 1 else hkv * d, v.stride(0) if t > 1 else hkv * d,
        _lib.dtype_code(k_cache.dtype), err_count.data_ptr() if err_count is not None else None,
        _lib.stream_ptr(dev))
    _lib.check(rc, "reshape_and_cache")
