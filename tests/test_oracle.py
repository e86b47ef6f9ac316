"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each oracle function is checked against something independent of its own
formula: torch's scaled_dot_product_attention (a library routine) on the
contiguous K/V, scalar brute force, closed forms, the reference tests' known
answers, and invariants.  Planted mistakes (in the oracle, on the CPU) show the
checks are sensitive to the errors they are meant to catch.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle.attention import flash_prefill_ref, paged_decode_ref, paged_decode_split_ref
from oracle.kv_cache import KVCacheRef, reshape_and_cache_ref


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def make_paged(rng, ctx_list, hq, hkv, d, bs, spare=5, shuffle=True, width=None):
    """Paged cache + zero-padded tables + the contiguous K/V each sequence sees."""
    need = [(c + bs - 1) // bs for c in ctx_list]
    nb = sum(need) + spare
    ids = rng.permutation(nb) if shuffle else np.arange(nb)
    mb = max(need) if width is None else width
    bt = np.zeros((len(ctx_list), mb), np.int32)
    cur = 0
    for i, n in enumerate(need):
        bt[i, :n] = ids[cur:cur + n]
        cur += n
    kc = rng.standard_normal((nb, bs, hkv, d))
    vc = rng.standard_normal((nb, bs, hkv, d))
    q = rng.standard_normal((len(ctx_list), 1, hq, d))
    contig = []
    for i, c in enumerate(ctx_list):
        blocks = bt[i, :need[i]]
        contig.append((kc[blocks].reshape(-1, hkv, d)[:c], vc[blocks].reshape(-1, hkv, d)[:c]))
    return q, kc, vc, bt, np.asarray(ctx_list, np.int32), contig


def sdpa_decode(q, contig, hq, hkv):
    """torch SDPA (float64, CPU) per sequence over its contiguous K/V."""
    outs = []
    for i, (k, v) in enumerate(contig):
        qt = torch.from_numpy(q[i]).permute(1, 0, 2)[None]          # [1,Hq,1,D]
        kt = torch.from_numpy(k).permute(1, 0, 2)[None]             # [1,Hkv,C,D]
        vt = torch.from_numpy(v).permute(1, 0, 2)[None]
        o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, enable_gqa=(hq != hkv))
        outs.append(o[0].permute(1, 0, 2).numpy())                  # [1,Hq,D]
    return np.stack(outs)


DECODE_CASES = [
    # ctx list, Hq, Hkv, D, bs
    ([32], 4, 4, 32, 16),
    ([32, 32], 8, 8, 64, 16),
    ([32], 32, 8, 64, 16),
    ([64], 32, 4, 64, 16),
    ([17, 64, 128, 250], 32, 4, 64, 16),
    ([25], 4, 4, 32, 16),
    ([5, 9, 1], 6, 2, 16, 4),
    ([40, 3], 8, 1, 8, 8),
]


@pytest.mark.parametrize("ctx,hq,hkv,d,bs", DECODE_CASES)
def test_paged_decode_vs_sdpa(ctx, hq, hkv, d, bs):
    rng = _rng(1)
    q, kc, vc, bt, cl, contig = make_paged(rng, ctx, hq, hkv, d, bs)
    got = paged_decode_ref(q, kc, vc, bt, cl, hq, hkv, d, bs)
    ref = sdpa_decode(q, contig, hq, hkv)
    assert got.shape == (len(ctx), 1, hq, d)
    assert np.abs(got - ref).max() < 1e-12


def test_paged_decode_brute_force():
    """Scalar loops with math.exp on a tiny case."""
    rng = _rng(2)
    ctx, hq, hkv, d, bs = [3, 6], 4, 2, 3, 2
    q, kc, vc, bt, cl, _ = make_paged(rng, ctx, hq, hkv, d, bs, width=4)
    got = paged_decode_ref(q, kc, vc, bt, cl, hq, hkv, d, bs)
    for b, c in enumerate(ctx):
        for h in range(hq):
            kh = h // (hq // hkv)
            rows = [(bt[b, j // bs], j % bs) for j in range(c)]
            s = [sum(q[b, 0, h, e] * kc[blk, off, kh, e] for e in range(d)) / math.sqrt(d) for blk, off in rows]
            mx = max(s)
            w = [math.exp(x - mx) for x in s]
            tot = sum(w)
            for e in range(d):
                val = sum(wi * vc[blk, off, kh, e] for wi, (blk, off) in zip(w, rows)) / tot
                assert abs(got[b, 0, h, e] - val) < 1e-12


def test_paged_decode_closed_forms():
    rng = _rng(3)
    hq, hkv, d, bs = 8, 2, 16, 4
    q, kc, vc, bt, cl, contig = make_paged(rng, [1, 7, 12], hq, hkv, d, bs)
    out = paged_decode_ref(q, kc, vc, bt, cl, hq, hkv, d, bs)
    # ctx = 1: the only weight is 1, output is that V row
    for h in range(hq):
        assert np.array_equal(out[0, 0, h], vc[bt[0, 0], 0, h // 4])
    # K = 0: uniform weights, output is the mean of V over the context
    out0 = paged_decode_ref(q, np.zeros_like(kc), vc, bt, cl, hq, hkv, d, bs)
    for b, (_, v) in enumerate(contig):
        for h in range(hq):
            assert np.abs(out0[b, 0, h] - v[:, h // 4].mean(axis=0)).max() < 1e-12


def test_paged_decode_ctx_zero_quirk():
    """ctx = 0: every gathered position is masked (-1e9 in f32) -> mean of the padded gather."""
    rng = _rng(4)
    hq, hkv, d, bs = 4, 4, 8, 4
    q, kc, vc, bt, cl, _ = make_paged(rng, [6, 9], hq, hkv, d, bs)
    q *= 0.1                                                  # |scores| << 32
    cl = np.array([0, 9], np.int32)
    out = paged_decode_ref(q, kc, vc, bt, cl, hq, hkv, d, bs)
    gathered = vc[bt[0]].reshape(-1, hkv, d)                  # all MB*bs rows incl. padding block 0
    assert np.abs(out[0, 0] - gathered.mean(axis=0)).max() < 1e-12


def test_paged_decode_invariants():
    rng = _rng(5)
    hq, hkv, d, bs = 8, 4, 16, 4
    q, kc, vc, bt, cl, _ = make_paged(rng, [5, 11, 16], hq, hkv, d, bs, spare=3)
    base = paged_decode_ref(q, kc, vc, bt, cl, hq, hkv, d, bs)
    # relabel blocks consistently
    perm = rng.permutation(kc.shape[0])
    kc2, vc2 = np.empty_like(kc), np.empty_like(vc)
    kc2[perm], vc2[perm] = kc, vc
    assert np.abs(paged_decode_ref(q, kc2, vc2, perm[bt].astype(np.int32), cl, hq, hkv, d, bs) - base).max() < 1e-12
    # contents of padding / unused blocks do not matter
    used = set()
    for i, c in enumerate(cl):
        used |= set(bt[i, :(c + bs - 1) // bs].tolist())
    kc3, vc3 = kc.copy(), vc.copy()
    for blk in range(kc.shape[0]):
        if blk not in used:
            kc3[blk] = 1e3
            vc3[blk] = -1e3
    # the last row of a partial block is beyond ctx and must not matter either
    blk_last = bt[0, (cl[0] - 1) // bs]
    kc3[blk_last, cl[0] % bs:] = 77.0
    assert np.abs(paged_decode_ref(q, kc3, vc3, bt, cl, hq, hkv, d, bs) - base).max() < 1e-12


def test_paged_decode_max_context_len_trims_table():
    rng = _rng(6)
    hq, hkv, d, bs = 4, 2, 8, 4
    q, kc, vc, bt, cl, _ = make_paged(rng, [9, 12], hq, hkv, d, bs, width=6)
    a = paged_decode_ref(q, kc, vc, bt, cl, hq, hkv, d, bs, max_context_len=10)
    b = paged_decode_ref(q, kc, vc, bt[:, :3], cl, hq, hkv, d, bs)
    assert np.array_equal(a, b)
    # context beyond the used width is truncated to the width (reference gathers only MB*bs rows)
    c = paged_decode_ref(q, kc, vc, bt[:, :2], np.array([9, 12], np.int32), hq, hkv, d, bs)
    d_ = paged_decode_ref(q, kc, vc, bt[:, :2], np.array([8, 8], np.int32), hq, hkv, d, bs)
    assert np.array_equal(c, d_)


@pytest.mark.parametrize("psize", [1, 3, 4, 16, 64, 1000])
def test_split_merge_equals_single_pass(psize):
    rng = _rng(7)
    hq, hkv, d, bs = 8, 2, 16, 4
    q, kc, vc, bt, cl, _ = make_paged(rng, [1, 7, 33, 50], hq, hkv, d, bs)
    a = paged_decode_ref(q, kc, vc, bt, cl, hq, hkv, d, bs)
    b = paged_decode_split_ref(q, kc, vc, bt, cl, hq, hkv, d, bs, psize)
    assert np.abs(a - b).max() < 1e-12
    # the all-masked quirk survives splitting
    q2 = q * 0.1
    cl0 = np.array([0, 7, 33, 0], np.int32)
    a0 = paged_decode_ref(q2, kc, vc, bt, cl0, hq, hkv, d, bs)
    b0 = paged_decode_split_ref(q2, kc, vc, bt, cl0, hq, hkv, d, bs, psize)
    assert np.abs(a0 - b0).max() < 1e-12


def test_planted_gqa_mapping_error_is_caught(monkeypatch):
    """A wrong GQA mapping (h % Hkv instead of h // g) planted in the oracle fails the SDPA pin."""
    rng = _rng(8)
    hq, hkv, d, bs = 8, 2, 16, 4
    q, kc, vc, bt, cl, contig = make_paged(rng, [9, 13], hq, hkv, d, bs)
    ref = sdpa_decode(q, contig, hq, hkv)
    monkeypatch.setattr(oa.np, "repeat", lambda a, n, axis: np.tile(a, [n if i == axis else 1 for i in range(a.ndim)]))
    bad = paged_decode_ref(q, kc, vc, bt, cl, hq, hkv, d, bs)
    assert np.abs(bad - ref).max() > 1e-3


def test_planted_mask_boundary_error_is_caught():
    """Attending one position too far (ctx+1) is caught by the SDPA pin."""
    rng = _rng(9)
    hq, hkv, d, bs = 4, 4, 16, 4
    q, kc, vc, bt, cl, contig = make_paged(rng, [9, 13], hq, hkv, d, bs)
    ref = sdpa_decode(q, contig, hq, hkv)
    bad = paged_decode_ref(q, kc, vc, bt, cl + 1, hq, hkv, d, bs)
    assert np.abs(bad - ref).max() > 1e-3


# ---- prefill -------------------------------------------------------------------

def sdpa_prefill(q, k, v, causal):
    qt = torch.from_numpy(q[0]).permute(1, 0, 2)[None]
    kt = torch.from_numpy(k[0]).permute(1, 0, 2)[None]
    vt = torch.from_numpy(v[0]).permute(1, 0, 2)[None]
    lq, lk = q.shape[1], k.shape[1]
    mask = None
    if causal:
        mask = torch.ones(lq, lk, dtype=torch.bool).tril(0)   # key j allowed for query i iff j <= i
    o = torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, attn_mask=mask, enable_gqa=(q.shape[2] != k.shape[2]))
    return o[0].permute(1, 0, 2)[None].numpy()


@pytest.mark.parametrize("lq,hq,hkv,d,causal", [
    (1, 8, 8, 64, True), (2, 4, 4, 32, True), (7, 4, 4, 32, True), (16, 8, 4, 32, True),
    (33, 32, 8, 64, True), (64, 32, 4, 64, True), (16, 4, 4, 32, False), (31, 8, 2, 16, False),
])
def test_prefill_vs_sdpa(lq, hq, hkv, d, causal):
    rng = _rng(10)
    q = rng.standard_normal((1, lq, hq, d))
    k = rng.standard_normal((1, lq, hkv, d))
    v = rng.standard_normal((1, lq, hkv, d))
    got = flash_prefill_ref(q, k, v, causal)
    assert np.abs(got - sdpa_prefill(q, k, v, causal)).max() < 1e-12


def test_prefill_top_left_alignment_for_unequal_lengths():
    rng = _rng(11)
    q = rng.standard_normal((1, 5, 4, 8))
    k = rng.standard_normal((1, 9, 2, 8))
    v = rng.standard_normal((1, 9, 2, 8))
    got = flash_prefill_ref(q, k, v, True)
    assert np.abs(got - sdpa_prefill(q, k, v, True)).max() < 1e-12
    # query 0 sees only key 0 -> equals V[0]
    assert np.abs(got[0, 0] - np.repeat(v[0, 0], 2, axis=0)).max() < 1e-12


@pytest.mark.parametrize("start,n", [(0, 9), (5, 4), (12, 1), (3, 13)])
def test_prefill_query_offset_equals_last_rows_of_whole_prompt(start, n):
    """q_offset = s (a chunk after s cached positions) gives exactly the last n
    rows of causal attention over the whole sequence (torch SDPA, float64) --
    and differs from the top-left aligned chunk when s > 0 (the offset matters)."""
    rng = _rng(14)
    total = start + n
    q = rng.standard_normal((1, total, 4, 8))
    k = rng.standard_normal((1, total, 2, 8))
    v = rng.standard_normal((1, total, 2, 8))
    got = flash_prefill_ref(q[:, start:], k, v, True, q_offset=start)
    assert np.abs(got - sdpa_prefill(q, k, v, True)[:, start:]).max() < 1e-12
    if start > 0:
        assert np.abs(got - flash_prefill_ref(q[:, start:], k, v, True)).max() > 1e-3


def test_prefill_reference_known_answers():
    """test_flash_attention.py:123-139, restated."""
    rng = _rng(12)
    # first token attends only to itself; V = I (head_dim_v 8 != head_dim 16)
    q = np.zeros((1, 8, 2, 16))
    q[0, 0] = 1.0
    k = rng.standard_normal((1, 8, 2, 16))
    v = np.broadcast_to(np.eye(8)[:, None, :], (8, 2, 8))[None].copy()
    out = flash_prefill_ref(q, k, v, True)
    assert out[0, 0, 0, 0] > 0.5
    assert out[0, 0, 0, 0] == 1.0
    # K = 0: last row uniform over all 8 keys -> mean(0..7) = 3.5
    q = np.ones((1, 8, 2, 16))
    k = np.zeros((1, 8, 2, 16))
    v = np.broadcast_to(np.arange(8.0).reshape(8, 1, 1), (8, 2, 16))[None].copy()
    out = flash_prefill_ref(q, k, v, True)
    assert abs(out[0, -1, 0, 0] - 3.5) < 1e-12
    # L = 1 -> output is V
    q, k, v = (rng.standard_normal((1, 1, 4, 8)) for _ in range(3))
    assert np.abs(flash_prefill_ref(q, k, v, True)[0, 0] - v[0, 0]).max() < 1e-15


def test_planted_scale_error_is_caught(monkeypatch):
    """Dropping the 1/sqrt(D) scale in the oracle is caught by the SDPA pin."""
    rng = _rng(13)
    q, k, v = (rng.standard_normal((1, 12, 4, 16)) for _ in range(3))
    ref = sdpa_prefill(q, k, v, True)
    monkeypatch.setattr(oa.math, "sqrt", lambda x: 1.0)
    assert np.abs(flash_prefill_ref(q, k, v, True) - ref).max() > 1e-3


# ---- KV cache ------------------------------------------------------------------

def test_kv_cache_reference_known_answers():
    """test_kv_cache.py:143-365 sums, restated on the oracle."""
    c = KVCacheRef(2, 4, 16, 2, 4, np.float32)
    c.write_kv(0, 0, 0, np.ones((5, 2, 4)), np.ones((5, 2, 4)) * 2)
    for i in range(5):
        assert c.k_cache[0][0, i].sum() == 8
    c.write_kv(0, 0, 5, np.ones((3, 2, 4)) * 5, np.ones((3, 2, 4)) * 5)
    for i in range(5, 8):
        assert c.k_cache[0][0, i].sum() == 40
    c = KVCacheRef(1, 4, 4, 2, 4, np.float32)
    for blk, base in ((0, 1), (1, 5), (2, 9)):
        n = 4 if blk < 2 else 2
        rows = np.stack([np.ones((2, 4)) * (base + i) for i in range(n)])
        c.write_kv(0, blk, 0, rows, rows)
    k, v = c.read_kv_blocks(0, [0, 1, 2], 10)
    assert k.shape == (10, 2, 4)
    for pos in range(10):
        assert k[pos].sum() == (pos + 1) * 8
    k, v = c.read_kv_blocks(0, [], 0)
    assert k.shape == (0, 2, 4) and v.shape == (0, 2, 4)
    assert KVCacheRef(2, 10, 16, 4, 64, np.float32).get_memory_bytes() == 2 * 10 * 16 * 4 * 64 * 2 * 4


def test_reshape_and_cache_ref_placement():
    rng = _rng(14)
    nb, bs, hkv, d = 6, 4, 2, 3
    kc = np.zeros((nb, bs, hkv, d))
    vc = np.zeros((nb, bs, hkv, d))
    k = rng.standard_normal((7, hkv, d))
    v = rng.standard_normal((7, hkv, d))
    slots = np.array([0, 5, 23, -1, 9, 10, 4], np.int32)
    reshape_and_cache_ref(kc, vc, k, v, slots)
    flat_k = kc.reshape(nb * bs, hkv, d)
    for t, s in enumerate(slots):
        if s >= 0:
            assert np.array_equal(flat_k[s], k[t])
    written = {int(s) for s in slots if s >= 0}
    for s in range(nb * bs):
        if s not in written:
            assert not flat_k[s].any()
