"""Committed golden fixtures (tests/golden/*.npz, written by make_golden.py).

CPU: the oracle and the host-side producers reproduce the fixtures.
GPU: the HIP path matches them within 1e-4 (fp32) / 2e-2 (fp16, bf16) max-abs.
"""

import os

import numpy as np
import pytest

from oracle.attention import flash_prefill_ref, paged_decode_ref
from tinyvllm_amd.block_manager import BlockManager

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def test_oracle_reproduces_decode_fixture():
    g = load("paged_decode_b2.npz")
    hq, hkv, d, bs = g["shape"].tolist()
    out = paged_decode_ref(g["q"], g["k_cache"], g["v_cache"], g["block_tables"], g["context_lens"],
                           hq, hkv, d, bs)
    assert np.abs(out - g["out"]).max() < 1e-12


def test_oracle_reproduces_prefill_fixture():
    g = load("prefill_l16.npz")
    assert np.abs(flash_prefill_ref(g["q"], g["k"], g["v"], True) - g["out_causal"]).max() < 1e-12
    assert np.abs(flash_prefill_ref(g["q"], g["k"], g["v"], False) - g["out_full"]).max() < 1e-12


def test_block_manager_reproduces_slot_fixture():
    g = load("slots_3seq.npz")
    bm = BlockManager(1, 24, 4)
    for sid, (start, n) in enumerate([(0, 7), (0, 12), (0, 1)]):
        bm.register_sequence(sid)
        assert np.array_equal(bm.prefill_slot_mapping(sid, start, n), g[f"prefill_{sid}"])
        for _ in range(n):
            bm.advance_position(sid)
    assert np.array_equal(bm.decode_slot_mapping([0, 1, 2]), g["decode"])
    bt, ctx = bm.prepare_batch_tensors([0, 1, 2], [7, 12, 1], 4)
    assert np.array_equal(bt, g["block_tables"]) and np.array_equal(ctx, g["context_lens"])


@pytest.mark.gpu
def test_gpu_decode_matches_fixture():
    import torch
    from tinyvllm_amd.attention import paged_decode_attention
    g = load("paged_decode_b2.npz")
    hq, hkv, d, bs = g["shape"].tolist()
    t = {k: torch.from_numpy(g[k]).cuda() for k in ("q", "k_cache", "v_cache", "block_tables", "context_lens")}
    for ps in (16, 512):
        out = paged_decode_attention(t["q"], t["k_cache"], t["v_cache"], t["block_tables"], t["context_lens"],
                                     hq, hkv, d, bs, partition_size=ps)
        assert np.abs(out.cpu().numpy() - g["out"]).max() <= 1e-4


@pytest.mark.gpu
def test_gpu_prefill_matches_fixture():
    import torch
    from tinyvllm_amd.attention import flash_prefill_attention
    g = load("prefill_l16.npz")
    q, k, v = (torch.from_numpy(g[n]).cuda() for n in ("q", "k", "v"))
    assert np.abs(flash_prefill_attention(q, k, v, True).cpu().numpy() - g["out_causal"]).max() <= 1e-4
    assert np.abs(flash_prefill_attention(q, k, v, False).cpu().numpy() - g["out_full"]).max() <= 1e-4
    for dt in (torch.float16, torch.bfloat16):
        # generic kernel at head_dim 16 in half precision, against the oracle on the rounded inputs
        qh, kh, vh = q.to(dt), k.to(dt), v.to(dt)
        out = flash_prefill_attention(qh, kh, vh, True).float().cpu().numpy()
        want = flash_prefill_ref(*(x.float().cpu().numpy() for x in (qh, kh, vh)), True)
        assert np.abs(out - want).max() <= 2e-2
