"""Drop-in attention entry points with the reference's signatures.

``paged_decode_attention`` and ``flash_prefill_attention`` keep the names,
positional order and keyword names of tinyvllm/model/llama.py:97-108 and
llama.py:58-63, so callers written against the reference (the JIT decode body,
Attention.__call__, the tests) can switch by import.  Tensors are PyTorch-ROCm
tensors on a HIP device; all arithmetic runs in libtvattn.so (no fallback).
"""

import math

import numpy as np
import torch

from . import _lib

_lib.load()

def _require(cond, msg):
    if not cond:
        raise ValueError(msg)


def _on_gpu(*tensors):
    dev = tensors[0].device
    _require(dev.type == "cuda", f"tensors must live on a HIP device (got {dev})")
    for t in tensors:
        _require(t.device == dev, "all tensors must be on the same device")
    return dev


def default_partition_size(num_seqs, n_heads, n_kv_heads, head_dim, max_blocks, block_size, dtype):
    """Tokens per decode work-group (multiple of 16) for this shape on the current device.

    With at least four (sequence, KV head) pairs per CU the work-groups already
    fill the GPU, and splitting only adds partial writes and a merge launch, so
    each pair gets one work-group over its whole context.  Otherwise contexts
    are split into as many partitions as make a full-width batch's work-groups
    fill the resident work-group slots once (occupancy x CUs, queried by the
    library): on MI355X 16 x 32768 bf16 runs 323 us with 5472-token partitions
    (768 work-groups, one round) against 342 us with 2048.
    """
    p = _lib.load().tv_paged_decode_partition_size(num_seqs, n_heads, n_kv_heads, head_dim, max_blocks,
                                                     block_size, _lib.dtype_code(dtype))
    _lib.check(0 if p > 0 else _lib.TV_EINVAL, "default_partition_size")
    return p


def paged_decode_attention(queries, k_cache, v_cache, block_tables, context_lens,
                           n_heads, n_kv_heads, head_dim, block_size, max_context_len=None,
                           *, partition_size=None, out_dtype=None):
    """Paged decode attention (tinyvllm/model/llama.py:97-144).

    queries [B,1,Hq,D]; k_cache/v_cache [NB,bs,Hkv,D] (same dtype as queries);
    block_tables [B,MB] int32 zero-padded; context_lens [B] int32.
    Returns [B,1,Hq,D] in ``out_dtype`` (default: the query dtype).
    ``max_context_len`` trims the table to ceil(max_context_len/bs) columns as in
    the reference.  ``partition_size`` (keyword-only, not in the reference)
    forces the split-context partition length in tokens.
    """
    lib = _lib.load()
    dev = _on_gpu(queries, k_cache, v_cache, block_tables, context_lens)
    _require(queries.dim() == 4 and queries.shape[1] == 1, f"queries must be [B,1,Hq,D], got {tuple(queries.shape)}")
    b, _, hq, d = queries.shape
    _require(hq == n_heads and d == head_dim, "queries shape does not match n_heads/head_dim")
    nb, bs, hkv, d2 = k_cache.shape
    _require(tuple(v_cache.shape) == (nb, bs, hkv, d2), "k_cache and v_cache shapes differ")
    _require(bs == block_size and hkv == n_kv_heads and d2 == head_dim,
             f"cache shape {tuple(k_cache.shape)} does not match block_size/n_kv_heads/head_dim")
    _require(n_heads % n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads")
    _require(queries.dtype == k_cache.dtype == v_cache.dtype, "queries and caches must share a dtype")
    _require(block_tables.dtype == torch.int32 and context_lens.dtype == torch.int32,
             "block_tables and context_lens must be int32")
    _require(block_tables.dim() == 2 and block_tables.shape[0] == b, "block_tables must be [B, max_blocks]")
    _require(context_lens.numel() == b, "context_lens must have B entries")
    for t in (queries, k_cache, v_cache, block_tables, context_lens):
        _require(t.is_contiguous(), "all inputs must be contiguous")

    mb = block_tables.shape[1]
    used = mb
    if max_context_len is not None:
        used = min((int(max_context_len) + block_size - 1) // block_size, mb)
    _require(used > 0, "no block table columns to attend over")
    width = used * block_size
    if partition_size is None:
        partition_size = default_partition_size(b, n_heads, n_kv_heads, head_dim, used, block_size, queries.dtype)
    out_dtype = queries.dtype if out_dtype is None else out_dtype
    out = torch.empty((b, 1, hq, d), dtype=out_dtype, device=dev)
    ws_bytes = lib.tv_paged_decode_workspace_bytes(b, hq, d, used, block_size, partition_size)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    rc = lib.tv_paged_decode(
        out.data_ptr(), queries.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        block_tables.data_ptr(), context_lens.data_ptr(),
        b, hq, n_kv_heads, d, block_size, nb, mb, used,
        1.0 / math.sqrt(head_dim), _lib.dtype_code(queries.dtype), _lib.dtype_code(out_dtype),
        int(partition_size), ws.data_ptr() if ws is not None else None, ws_bytes,
        _lib.stream_ptr(dev))
    _lib.check(rc, "paged_decode_attention")
    return out


def _token_rows(t, name):
    """[1, L, H, D] tensor whose (H, D) rows are dense; returns the token stride."""
    _require(t.dim() == 4 and t.shape[0] == 1, f"{name} must be [1, L, H, D] (batch 1, llama.py:65-67)")
    _require(t.stride(3) == 1 and t.stride(2) == t.shape[3], f"{name}: heads and head_dim must be contiguous")
    return t.stride(1)


def flash_prefill_attention(queries, keys, values, causal=True, *, out_dtype=None, chunk_tiles=0):
    """Prefill attention over one prompt (tinyvllm/model/llama.py:58-94).

    queries [1,Lq,Hq,D], keys [1,Lk,Hkv,D], values [1,Lk,Hkv,Dv] -> [1,Lq,Hq,Dv].
    ``causal`` masks key j for query i when j > i (top-left aligned).
    ``chunk_tiles`` (keyword-only, not in the reference): 64-key tiles per work
    unit when long causal rows are split; 0 picks it from the shape.
    """
    lib = _lib.load()
    dev = _on_gpu(queries, keys, values)
    qs = _token_rows(queries, "queries")
    ks = _token_rows(keys, "keys")
    vs = _token_rows(values, "values")
    _, lq, hq, d = queries.shape
    _, lk, hkv, dk = keys.shape
    _require(dk == d, "queries and keys must share head_dim")
    _require(values.shape[1] == lk and values.shape[2] == hkv, "keys and values must share [L, Hkv]")
    _require(hq % hkv == 0, "query heads must be a multiple of KV heads")
    _require(queries.dtype == keys.dtype == values.dtype, "queries, keys and values must share a dtype")
    dv = values.shape[3]
    out_dtype = queries.dtype if out_dtype is None else out_dtype
    out = torch.empty((1, lq, hq, dv), dtype=out_dtype, device=dev)
    code = _lib.dtype_code(queries.dtype)
    ws_bytes = lib.tv_flash_prefill_workspace_bytes(lq, lk, hq, d, dv, 1 if causal else 0, code, chunk_tiles)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    rc = lib.tv_flash_prefill(
        out.data_ptr(), queries.data_ptr(), keys.data_ptr(), values.data_ptr(),
        lq, lk, hq, hkv, d, dv, qs, ks, vs, hq * dv, 1 if causal else 0,
        1.0 / math.sqrt(d), code, _lib.dtype_code(out_dtype), chunk_tiles,
        ws.data_ptr() if ws is not None else None, ws_bytes, _lib.stream_ptr(dev))
    _lib.check(rc, "flash_prefill_attention")
    return out


def flash_prefill_paged(queries, k_cache, v_cache, block_table, start_pos, causal=True, *, out_dtype=None):
    """Prefill of one prompt chunk whose keys and values come from the paged cache
    (no counterpart in the reference: its chunk at start_pos > 0 attends within
    the chunk only, llama.py:184; chunked prefill is on its roadmap,
    ROADMAP.md:75-99).

    queries [1, n, Hq, D] (or [n, Hq, D]) are the chunk's rows at positions
    start_pos .. start_pos + n - 1; k_cache / v_cache [NB, bs, Hkv, D] already
    hold the K/V of positions 0 .. start_pos + n - 1 at the blocks listed in
    block_table (int32, one sequence, device).  Equals the last n rows of
    ``flash_prefill_attention`` over the whole sequence.  fp16 / bf16, head_dim
    64 or 128, power-of-two block size.  Returns [1, n, Hq, D].
    """
    lib = _lib.load()
    dev = _on_gpu(queries, k_cache, v_cache, block_table)
    q = queries[0] if queries.dim() == 4 else queries
    _require(queries.dim() in (3, 4) and (queries.dim() == 3 or queries.shape[0] == 1),
             "queries must be [1, n, Hq, D] or [n, Hq, D]")
    _require(q.stride(2) == 1 and q.stride(1) == q.shape[2], "queries: heads and head_dim must be contiguous")
    n, hq, d = q.shape
    nb, bs, hkv, d2 = k_cache.shape
    _require(tuple(v_cache.shape) == tuple(k_cache.shape) and d2 == d, "cache shape does not match the queries")
    _require(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    _require(hq % hkv == 0, "query heads must be a multiple of KV heads")
    _require(q.dtype == k_cache.dtype == v_cache.dtype, "queries and caches must share a dtype")
    _require(block_table.dtype == torch.int32 and block_table.is_contiguous(), "block_table must be contiguous int32")
    start_pos = int(start_pos)
    _require(start_pos >= 0 and n > 0, "start_pos must be >= 0 and the chunk non-empty")
    _require(block_table.numel() * bs >= start_pos + n, "block_table does not cover the sequence")
    out_dtype = q.dtype if out_dtype is None else out_dtype
    out = torch.empty((1, n, hq, d), dtype=out_dtype, device=dev)
    rc = lib.tv_flash_prefill_paged(out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                    block_table.data_ptr(), nb, bs, n, start_pos, hq, hkv, d, q.stride(0), hq * d,
                                    1 if causal else 0, 1.0 / math.sqrt(d), _lib.dtype_code(q.dtype),
                                    _lib.dtype_code(out_dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "flash_prefill_paged")
    return out


class VarlenPrefillPlan:
    """Several prompts in one prefill launch (no reference counterpart: the
    engine prefills one sequence per call, engine.py:125-132).

    queries [T, Hq, D], keys / values [T, Hkv, D] (or with a leading batch
    dimension of 1) hold the prompts back to back; ``seq_lens`` (host ints)
    are their lengths, summing to T.  Each prompt attends within itself exactly
    as ``flash_prefill_attention`` attends one prompt (``causal``: key j masked
    for query i when j > i).  fp16 / bf16 with head_dim 64 or 128.  The plan
    holds the output and the device offsets, so ``run()`` is one C call (HIP
    graph capture works); the inputs must stay alive while it is used.
    """

    def __init__(self, queries, keys, values, seq_lens, causal=True, *, out_dtype=None):
        self.lib = _lib.load()
        self.dev = _on_gpu(queries, keys, values)
        for t in (queries, keys, values):
            _require(t.dim() == 3 or (t.dim() == 4 and t.shape[0] == 1), "inputs must be [T, H, D] or [1, T, H, D]")
        q, k, v = (t[0] if t.dim() == 4 else t for t in (queries, keys, values))
        for t, name in ((q, "queries"), (k, "keys"), (v, "values")):
            _require(t.stride(2) == 1 and t.stride(1) == t.shape[2], f"{name}: heads and head_dim must be contiguous")
        tot, hq, d = q.shape
        _, hkv, dk = k.shape
        _require(dk == d and tuple(v.shape) == tuple(k.shape), "keys and values must be [T, Hkv, D] with the queries' D")
        _require(k.shape[0] == tot, "keys and values must hold the same tokens as the queries")
        _require(hq % hkv == 0, "query heads must be a multiple of KV heads")
        _require(q.dtype == k.dtype == v.dtype, "queries, keys and values must share a dtype")
        lens = [int(n) for n in seq_lens]
        _require(len(lens) > 0 and min(lens) > 0 and sum(lens) == tot, "seq_lens must be positive and sum to T")
        cu = np.zeros(len(lens) + 1, np.int32)
        cu[1:] = np.cumsum(lens)
        order = np.argsort(-np.asarray(lens), kind="stable").astype(np.int32)   # longest first
        self.cu = torch.from_numpy(cu).to(self.dev)
        self.order = torch.from_numpy(order).to(self.dev)
        out_dtype = q.dtype if out_dtype is None else out_dtype
        self.out = torch.empty((tot, hq, d), dtype=out_dtype, device=self.dev)
        self._inputs = (queries, keys, values)     # a captured launch reads them on every replay
        self._args = (self.out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), self.cu.data_ptr(),
                      self.cu.data_ptr(), self.order.data_ptr(), len(lens), max(lens), max(lens), tot, hq, hkv, d,
                      q.stride(0), k.stride(0), v.stride(0), hq * d, 1 if causal else 0, 1.0 / math.sqrt(d),
                      _lib.dtype_code(q.dtype), _lib.dtype_code(out_dtype))

    def run(self):
        rc = self.lib.tv_flash_prefill_varlen(*self._args, _lib.stream_ptr(self.dev))
        _lib.check(rc, "flash_prefill_varlen")
        return self.out


def flash_prefill_varlen(queries, keys, values, seq_lens, causal=True, *, out_dtype=None):
    """Prefill attention over several prompts in one launch; see VarlenPrefillPlan.
    Returns [T, Hq, D]."""
    return VarlenPrefillPlan(queries, keys, values, seq_lens, causal, out_dtype=out_dtype).run()


class PagedDecodePlan:
    """Pre-validated, pointer-stable paged decode for a fixed batch shape.

    Holds the output and split-context workspace so that ``run()`` is a single
    C call with no allocation -- the form a decode loop captures in a HIP graph
    (the analogue of the reference's TinyJit replay, llama.py:290-344).  The
    input tensors must stay alive and keep their storage while the plan is used.
    """

    def __init__(self, queries, k_cache, v_cache, block_tables, context_lens,
                 n_heads, n_kv_heads, head_dim, block_size, max_context_len=None,
                 *, partition_size=None, out_dtype=None):
        self.lib = _lib.load()
        self.dev = _on_gpu(queries, k_cache, v_cache, block_tables, context_lens)
        b = queries.shape[0]
        mb = block_tables.shape[1]
        used = mb if max_context_len is None else min((int(max_context_len) + block_size - 1) // block_size, mb)
        _require(used > 0, "no block table columns to attend over")
        if partition_size is None:
            partition_size = default_partition_size(b, n_heads, n_kv_heads, head_dim, used, block_size,
                                                    queries.dtype)
        self.partition_size = int(partition_size)
        out_dtype = queries.dtype if out_dtype is None else out_dtype
        # validate once through the functional path's checks
        _require(queries.shape == (b, 1, n_heads, head_dim), "queries must be [B,1,Hq,D]")
        _require(tuple(k_cache.shape[1:]) == (block_size, n_kv_heads, head_dim), "cache shape mismatch")
        _require(block_tables.dtype == torch.int32 and context_lens.dtype == torch.int32, "int32 tables required")
        for t in (queries, k_cache, v_cache, block_tables, context_lens):
            _require(t.is_contiguous(), "all inputs must be contiguous")
        self.out = torch.empty((b, 1, n_heads, head_dim), dtype=out_dtype, device=self.dev)
        self.ws_bytes = self.lib.tv_paged_decode_workspace_bytes(b, n_heads, head_dim, used, block_size,
                                                                 self.partition_size)
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=self.dev)
        self._inputs = (queries, k_cache, v_cache, block_tables, context_lens)
        self.args = (self.out.data_ptr(), queries.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                     block_tables.data_ptr(), context_lens.data_ptr(), b, n_heads, n_kv_heads, head_dim,
                     block_size, k_cache.shape[0], mb, used, 1.0 / math.sqrt(head_dim),
                     _lib.dtype_code(queries.dtype), _lib.dtype_code(out_dtype), self.partition_size,
                     self.ws.data_ptr(), self.ws_bytes)

    def run(self):
        _lib.check(self.lib.tv_paged_decode(*self.args, _lib.stream_ptr(self.dev)), "PagedDecodePlan.run")
        return self.out


class PrefillPlan:
    """Pre-validated, pointer-stable causal prefill for fixed [1, L, H, D] inputs."""

    def __init__(self, queries, keys, values, causal=True, *, out_dtype=None, chunk_tiles=0):
        self.lib = _lib.load()
        self.dev = _on_gpu(queries, keys, values)
        qs, ks, vs = _token_rows(queries, "queries"), _token_rows(keys, "keys"), _token_rows(values, "values")
        _, lq, hq, d = queries.shape
        _, lk, hkv, _ = keys.shape
        dv = values.shape[3]
        out_dtype = queries.dtype if out_dtype is None else out_dtype
        code = _lib.dtype_code(queries.dtype)
        self.out = torch.empty((1, lq, hq, dv), dtype=out_dtype, device=self.dev)
        self.ws_bytes = self.lib.tv_flash_prefill_workspace_bytes(lq, lk, hq, d, dv, 1 if causal else 0, code,
                                                                  chunk_tiles)
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=self.dev)
        self._inputs = (queries, keys, values)
        self.args = (self.out.data_ptr(), queries.data_ptr(), keys.data_ptr(), values.data_ptr(),
                     lq, lk, hq, hkv, d, dv, qs, ks, vs, hq * dv, 1 if causal else 0, 1.0 / math.sqrt(d),
                     code, _lib.dtype_code(out_dtype), chunk_tiles, self.ws.data_ptr(), self.ws_bytes)

    def run(self):
        _lib.check(self.lib.tv_flash_prefill(*self.args, _lib.stream_ptr(self.dev)), "PrefillPlan.run")
        return self.out
