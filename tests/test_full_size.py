"""Paged decode and causal prefill at the benchmark's full sizes
(tinyvllm/model/llama.py:97-144, 58-94).

The two HBM-bound decode workloads run exactly as bench.py builds and launches
them: the Llama-3-8B head shape (B256, Hq32 Hkv8 D128, fp16 cache, context
lengths ~U[512, 4096], shuffled pool +10%; the scheduled launch with KV-head
pairs) and the split-context case (16 x 32768, bf16).  At these sizes the
float64 oracle runs on sampled sequences, whose blocks are gathered from the
device into a compact cache; the whole batch is checked through properties that
do not depend on size: repeated launches are bit-identical, and the split and
unsplit launches agree (the log-sum-exp merge is exact in real arithmetic, so
they differ by rounding only).  Prefill at the benchmark's long prompts
(Llama-3-8B heads at L 4096 / 8192, and the 4-way head shard whose longer
query tiles run as key halves plus a merge) is checked on sampled query rows:
row i of a causal prefill is the softmax attention of q_i over keys 0 .. i, so
the oracle runs on that one row with all heads.  Tolerance: 2e-2 max-abs for
fp16/bf16.
"""

import numpy as np
import pytest
import torch

from oracle.attention import flash_prefill_ref, paged_decode_ref

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


def _prefill_rows_check(L, hq, hkv, dtype, seed):
    """Bench-shaped causal prefill (inputs drawn as bench.py draws its long
    prompts); sampled rows against the float64 oracle, a repeat bit-identical."""
    from tinyvllm_amd.attention import flash_prefill_attention
    d = 128
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((1, L, hq, d), generator=g, device="cuda").to(dtype)
    k = torch.randn((1, L, hkv, d), generator=g, device="cuda").to(dtype)
    v = torch.randn((1, L, hkv, d), generator=g, device="cuda").to(dtype)
    out = flash_prefill_attention(q, k, v, True)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    rng = np.random.Generator(np.random.PCG64(seed + 1))
    # first rows, both sides of 128-row tile and key-half boundaries, the last rows, random rows
    rows = sorted({0, 1, 127, 128, 2047, 2048, L // 2 + 63, L // 2 + 64, L - 2, L - 1,
                   *rng.choice(L, 6, replace=False).tolist()})
    qh, kh, vh = q[0].float().cpu().numpy(), k[0].float().cpu().numpy(), v[0].float().cpu().numpy()
    got = out[0].float().cpu().numpy()
    for i in rows:
        want = flash_prefill_ref(qh[None, i:i + 1], kh[None, :i + 1], vh[None, :i + 1], causal=False)[0, 0]
        err = np.abs(got[i] - want).max()
        assert err <= TOL, f"L {L} Hq {hq} row {i}: max-abs {err}"
    again = flash_prefill_attention(q, k, v, True)
    torch.cuda.synchronize()
    assert torch.equal(again, out)


@pytest.mark.parametrize("L,hq,hkv,dtype", [(4096, 32, 8, torch.float16), (8192, 32, 8, torch.float16),
                                             (4096, 32, 8, torch.bfloat16), (4096, 8, 2, torch.float16)])
def test_prefill_long_prompts_full_size(L, hq, hkv, dtype):
    try:
        _prefill_rows_check(L, hq, hkv, dtype, seed=0)
    finally:
        torch.cuda.empty_cache()
