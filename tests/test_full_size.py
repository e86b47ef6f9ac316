"""Paged decode at the benchmark's full sizes (tinyvllm/model/llama.py:97-144).

The two HBM-bound decode workloads run exactly as bench.py builds and launches
them: the Llama-3-8B head shape (B256, Hq32 Hkv8 D128, fp16 cache, context
lengths ~U[512, 4096], shuffled pool +10%; the scheduled launch with KV-head
pairs) and the split-context case (16 x 32768, bf16).  At these sizes the
float64 oracle runs on sampled sequences, whose blocks are gathered from the
device into a compact cache; the whole batch is checked through properties that
do not depend on size: repeated launches are bit-identical, and the split and
unsplit launches agree (the log-sum-exp merge is exact in real arithmetic, so
they differ by rounding only).  Tolerance: 2e-2 max-abs for fp16/bf16.
"""

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_ref

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _decode(wl, partition_size=None):
    from tinyvllm_amd.attention import paged_decode_attention
    out = paged_decode_attention(wl.q, wl.k_cache, wl.v_cache, wl.bt_dev, wl.ctx_dev, wl.num_heads,
                                 wl.num_kv_heads, wl.head_dim, wl.block_size, partition_size=partition_size)
    torch.cuda.synchronize()
    return out


def _check_sampled(wl, out, seqs):
    bs = wl.block_size
    for b in seqs:
        ctx = int(wl.context_lens[b])
        nb = (ctx + bs - 1) // bs
        ids = torch.from_numpy(wl.block_tables[b, :nb].astype(np.int64)).to(wl.k_cache.device)
        kc = wl.k_cache[ids].float().cpu().numpy()
        vc = wl.v_cache[ids].float().cpu().numpy()
        q = wl.q[b:b + 1].float().cpu().numpy()
        want = paged_decode_ref(q, kc, vc, np.arange(nb, dtype=np.int32)[None], np.array([ctx], np.int32),
                                wl.num_heads, wl.num_kv_heads, wl.head_dim, bs)
        err = np.abs(out[b:b + 1].float().cpu().numpy() - want).max()
        assert err <= TOL, f"sequence {b} (ctx {ctx}): max-abs {err}"


def test_llama3_8b_b256_full_size():
    from tinyvllm_amd import workloads
    wl = workloads.decode_llama3_8b_b256()
    try:
        out = _decode(wl)
        ctx = wl.context_lens
        rng = np.random.Generator(np.random.PCG64(5))
        seqs = sorted({int(np.argmax(ctx)), int(np.argmin(ctx)), *rng.choice(len(ctx), 6, replace=False).tolist()})
        _check_sampled(wl, out, seqs)
        assert torch.equal(_decode(wl), out)                 # repeat: bit-identical
        split = _decode(wl, partition_size=1024)            # 1-4 partitions per sequence + merge
        _check_sampled(wl, split, seqs[:3])
        diff = (split.float() - out.float()).abs().max().item()
        assert diff <= TOL, f"split vs unsplit over the batch: {diff}"
        assert torch.isfinite(out).all()
    finally:
        del wl
        torch.cuda.empty_cache()


def test_long_bf16_b16_full_size():
    from tinyvllm_amd import workloads
    wl = workloads.decode_long_bf16_b16()
    try:
        out = _decode(wl)                                   # the recommended split
        _check_sampled(wl, out, [0, 11])
        assert torch.equal(_decode(wl), out)
        whole = _decode(wl, partition_size=32768)           # one partition per sequence
        diff = (whole.float() - out.float()).abs().max().item()
        assert diff <= TOL, f"unsplit vs split over the batch: {diff}"
        assert torch.isfinite(out).all()
    finally:
        del wl
        torch.cuda.empty_cache()
