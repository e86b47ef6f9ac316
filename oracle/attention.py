"""numpy restatement of the reference's two attention ops (test infrastructure).

Both functions follow the reference tensor expressions step by step, including
its quirks:

* the mask is an additive -1e9 computed in float32, not -inf
  (llama.py:89, 137-140);
* the scale is applied after the matmul, ``(q @ k^T) * scale`` (llama.py:84, 134-135);
* GQA maps query head h to KV head ``h // (Hq // Hkv)`` (llama.py:74-77, 124-128);
* decode gathers every block of the (possibly trimmed) table, padding included
  (llama.py:111-122), so a context of 0 yields the mean of the gathered V;
* prefill's causal mask is top-left aligned: key j is masked for query i when
  ``j > i`` (llama.py:86-90).

``acc`` selects the arithmetic type: float64 for parity goldens, float32 for the
timed CPU baseline.
"""

import math

import numpy as np

_MASK = np.float32(-1e9)


def _masked_scores(scores, valid):
    """Apply the reference's additive float32 mask to ``scores``.

    Valid positions keep their value.  Masked positions become
    ``float32(score) + float32(-1e9)`` rounded in float32, which is what
    tinygrad computes when an f32 mask meets f32 scores (llama.py:138-140);
    in f32 this rounds to -1e9 for any |score| < 32.
    """
    masked = (scores.astype(np.float32) + _MASK).astype(scores.dtype)
    return np.where(valid, scores, masked)


def _softmax(x):
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)


def paged_decode_ref(queries, k_cache, v_cache, block_tables, context_lens,
                     n_heads, n_kv_heads, head_dim, block_size,
                     max_context_len=None, acc=np.float64):
    """Restates ``paged_decode_attention`` (tinyvllm/model/llama.py:97-144).

    queries [B,1,Hq,D]; k_cache/v_cache [NB,bs,Hkv,D]; block_tables [B,MB] int;
    context_lens [B] int.  Returns [B,1,Hq,D] in ``acc``.
    """
    queries = np.asarray(queries)
    block_tables = np.asarray(block_tables)
    context_lens = np.asarray(context_lens).reshape(-1)
    batch = queries.shape[0]
    total_max_blocks = block_tables.shape[1]

    # llama.py:113-118 -- optional trim of the table width
    if max_context_len is not None:
        blocks_needed = min((max_context_len + block_size - 1) // block_size, total_max_blocks)
        max_context = blocks_needed * block_size
        block_tables = block_tables[:, :blocks_needed]
    else:
        max_context = total_max_blocks * block_size

    # llama.py:120-122 -- gather every listed block (padding rows included)
    idx = block_tables.reshape(-1).astype(np.int64)
    k_g = np.asarray(k_cache)[idx].astype(acc).reshape(batch, max_context, n_kv_heads, head_dim)
    v_g = np.asarray(v_cache)[idx].astype(acc).reshape(batch, max_context, n_kv_heads, head_dim)

    # llama.py:124-128 -- GQA expand: query head h reads KV head h // n_rep
    n_rep = n_heads // n_kv_heads
    if n_rep != 1:
        k_g = np.repeat(k_g, n_rep, axis=2)
        v_g = np.repeat(v_g, n_rep, axis=2)

    q = queries.astype(acc).transpose(0, 2, 1, 3)          # [B,Hq,1,D]
    k = k_g.transpose(0, 2, 1, 3)                          # [B,Hq,C,D]
    v = v_g.transpose(0, 2, 1, 3)

    scale = acc(1.0 / math.sqrt(head_dim))                 # llama.py:134
    scores = (q @ k.transpose(0, 1, 3, 2)) * scale         # [B,Hq,1,C]

    positions = np.arange(max_context).reshape(1, max_context)   # llama.py:137-140
    valid = positions < context_lens.reshape(batch, 1)
    scores = _masked_scores(scores, valid.reshape(batch, 1, 1, max_context))

    out = _softmax(scores) @ v                             # llama.py:142-143
    return out.transpose(0, 2, 1, 3)                       # [B,1,Hq,D]


def paged_decode_split_ref(queries, k_cache, v_cache, block_tables, context_lens,
                           n_heads, n_kv_heads, head_dim, block_size,
                           partition_size, max_context_len=None, acc=np.float64):
    """Split-context (flash-decoding) form of ``paged_decode_ref``.

    The reference has no partitioning (llama.py:97-144); this function restates
    the decomposition the GPU path uses so that its algebra is checked on the
    CPU: every partition of ``partition_size`` positions yields
    (max m_p, sum l_p = sum exp(s - m_p), o_p = sum exp(s - m_p) v / l_p) and the
    partitions are merged with weights ``l_p * exp(m_p - max_p m_p)``.
    Positions past the effective length are dropped; a context of 0 (or less)
    keeps the reference's all-masked behaviour over the whole gathered width.
    """
    queries = np.asarray(queries)
    block_tables = np.asarray(block_tables)
    context_lens = np.asarray(context_lens).reshape(-1)
    batch, _, _, _ = queries.shape
    mb = block_tables.shape[1]
    if max_context_len is not None:
        mb = min((max_context_len + block_size - 1) // block_size, mb)
    width = mb * block_size
    n_rep = n_heads // n_kv_heads
    scale = 1.0 / math.sqrt(head_dim)
    out = np.zeros((batch, 1, n_heads, head_dim), dtype=acc)
    for b in range(batch):
        ctx = int(context_lens[b])
        length = width if ctx <= 0 else min(ctx, width)
        pos = np.arange(length)
        blk = block_tables[b, pos // block_size].astype(np.int64)
        k = np.asarray(k_cache)[blk, pos % block_size].astype(acc)   # [len,Hkv,D]
        v = np.asarray(v_cache)[blk, pos % block_size].astype(acc)
        for h in range(n_heads):
            kh = h // n_rep
            s = (k[:, kh, :] @ queries[b, 0, h].astype(acc)) * scale
            if ctx <= 0:
                s = (s.astype(np.float32) + _MASK).astype(acc)
            parts = []
            for p0 in range(0, length, partition_size):
                sp = s[p0:p0 + partition_size]
                m = sp.max()
                e = np.exp(sp - m)
                l = e.sum()
                o = (e @ v[p0:p0 + partition_size, kh, :]) / l
                parts.append((m, l, o))
            gm = max(p[0] for p in parts)
            w = np.array([p[1] * np.exp(p[0] - gm) for p in parts])
            o = sum(wi * p[2] for wi, p in zip(w, parts)) / w.sum()
            out[b, 0, h] = o
    return out


def flash_prefill_ref(queries, keys, values, causal=True, acc=np.float64, q_offset=0):
    """Restates ``flash_prefill_attention`` (tinyvllm/model/llama.py:58-94).

    queries [1,Lq,Hq,D], keys [1,Lk,Hkv,D], values [1,Lk,Hkv,Dv] (batch must be
    1, llama.py:65-67).  Returns [1,Lq,Hq,Dv] in ``acc``.  ``q_offset`` (no
    reference counterpart; 0 is the reference) places query row i at position
    i + q_offset for the causal mask: a chunk after a cached prefix.
    """
    q = np.asarray(queries)
    k = np.asarray(keys)
    v = np.asarray(values)
    if q.shape[0] != 1 or k.shape[0] != 1 or v.shape[0] != 1:
        raise ValueError("flash_prefill_ref: batch must be 1 (llama.py:65-67)")
    q, k, v = q[0].astype(acc), k[0].astype(acc), v[0].astype(acc)
    q_len, n_heads, head_dim = q.shape
    kv_len, n_kv_heads, _ = k.shape
    scale = acc(1.0 / math.sqrt(head_dim))

    if n_kv_heads != n_heads:                                   # llama.py:74-77
        n_rep = n_heads // n_kv_heads
        k = np.repeat(k, n_rep, axis=1)
        v = np.repeat(v, n_rep, axis=1)

    qt, kt, vt = q.transpose(1, 0, 2), k.transpose(1, 0, 2), v.transpose(1, 0, 2)
    scores = (qt @ kt.transpose(0, 2, 1)) * scale               # llama.py:84
    if causal:                                                  # llama.py:86-90
        q_pos = np.arange(q_len).reshape(q_len, 1) + q_offset
        kv_pos = np.arange(kv_len).reshape(1, kv_len)
        scores = _masked_scores(scores, (kv_pos <= q_pos)[None])
    out = _softmax(scores) @ vt                                 # llama.py:92-93
    return out.transpose(1, 0, 2)[None]                         # llama.py:94
