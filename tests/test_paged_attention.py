"""Paged decode attention on the GPU vs the oracle (tinyvllm/model/llama.py:97-144).

Restates tests/test_paged_attention.py of the reference (consecutive-block
fixture, GQA 4x/8x, batching, context lengths, non-multiple context) and adds
parity on shuffled pools for every supported dtype / head_dim / group size,
the split-context path, and the reference's edge semantics.
Tolerances (max-abs vs the float64 oracle): fp32 1e-4, fp16/bf16 2e-2.
"""

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_ref
from tests.random_cases import case_count, case_seed

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _ops():
    from tinyvllm_amd.attention import paged_decode_attention
    return paged_decode_attention


def build_case(seed, ctx_list, hq, hkv, d, bs, dtype, spare=5, shuffle=True, width=None):
    rng = np.random.Generator(np.random.PCG64(seed))
    need = [(max(c, 1) + bs - 1) // bs for c in ctx_list]
    nb = sum(need) + spare
    ids = rng.permutation(nb) if shuffle else np.arange(nb)
    mb = max(need) if width is None else width
    bt = np.zeros((len(ctx_list), mb), np.int32)
    cur = 0
    for i, n in enumerate(need):
        bt[i, :min(n, mb)] = ids[cur:cur + n][:mb]
        cur += n
    q = torch.from_numpy(rng.standard_normal((len(ctx_list), 1, hq, d), dtype=np.float32)).to(dtype)
    kc = torch.from_numpy(rng.standard_normal((nb, bs, hkv, d), dtype=np.float32)).to(dtype)
    vc = torch.from_numpy(rng.standard_normal((nb, bs, hkv, d), dtype=np.float32)).to(dtype)
    return q, kc, vc, bt, np.asarray(ctx_list, np.int32)


def run(q, kc, vc, bt, cl, hq, hkv, d, bs, **kw):
    dev = "cuda"
    out = _ops()(q.to(dev), kc.to(dev), vc.to(dev), torch.from_numpy(bt).to(dev),
                 torch.from_numpy(cl).to(dev), hq, hkv, d, bs, **kw)
    torch.cuda.synchronize()
    return out


def oracle(q, kc, vc, bt, cl, hq, hkv, d, bs, **kw):
    return paged_decode_ref(q.float().numpy(), kc.float().numpy(), vc.float().numpy(), bt, cl,
                            hq, hkv, d, bs, **kw)


def check(case, hq, hkv, d, bs, dtype, **kw):
    q, kc, vc, bt, cl = case
    got = run(q, kc, vc, bt, cl, hq, hkv, d, bs, **kw)
    assert got.shape == (len(cl), 1, hq, d) and got.dtype == dtype
    okw = {k: v for k, v in kw.items() if k == "max_context_len"}
    want = oracle(q, kc, vc, bt, cl, hq, hkv, d, bs, **okw)
    err = np.abs(got.float().cpu().numpy() - want).max()
    assert err <= TOL[dtype], f"max-abs {err} > {TOL[dtype]}"
    return got


# ---- restated reference tests (consecutive blocks, fp32) ---------------------------

@pytest.mark.parametrize("batch,hq,hkv,d,ctx", [
    (2, 8, 8, 64, 32),      # test_output_shape
    (1, 4, 4, 32, 32),      # test_matches_standard_attention
    (1, 32, 8, 64, 32),     # test_gqa_4x
    (1, 32, 4, 64, 64),     # test_gqa_8x (TinyLlama)
    (4, 8, 8, 32, 32),      # test_batch_size_4
    (1, 4, 4, 32, 16), (1, 4, 4, 32, 64), (1, 4, 4, 32, 128),   # test_various_context_lengths
])
def test_reference_cases(batch, hq, hkv, d, ctx):
    case = build_case(1, [ctx] * batch, hq, hkv, d, 16, torch.float32, shuffle=False)
    check(case, hq, hkv, d, 16, torch.float32)


def test_context_not_multiple_of_block_size():
    case = build_case(2, [25], 4, 4, 32, 16, torch.float32, shuffle=False)
    out = check(case, 4, 4, 32, 16, torch.float32)
    assert not torch.isnan(out).any() and not torch.isinf(out).any()


# ---- parity on shuffled pools ------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
def test_head_dims_and_dtypes(dtype, d):
    case = build_case(3, [1, 17, 100, 250], 8, 2, d, 16, dtype)
    check(case, 8, 2, d, 16, dtype)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (16, 4), (32, 4), (32, 2), (24, 8), (12, 2), (6, 1)])
def test_group_sizes(hq, hkv):
    case = build_case(4, [5, 40, 77], hq, hkv, 64, 16, torch.float16)
    check(case, hq, hkv, 64, 16, torch.float16)


@pytest.mark.parametrize("bs", [1, 4, 8, 12, 32])
def test_block_sizes(bs):
    case = build_case(5, [3, 31, 65], 8, 2, 64, bs, torch.float32)
    check(case, 8, 2, 64, bs, torch.float32)


@pytest.mark.parametrize("psize", [16, 48, 64, 512, 4096])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_split_context_partitions(psize, dtype):
    case = build_case(6, [1, 15, 16, 17, 300, 1000], 16, 4, 128, 16, dtype)
    check(case, 16, 4, 128, 16, dtype, partition_size=psize)


def test_tinyllama_b4_fp32_workload():
    """TinyLlama layer, fp32, B4, ctx {17,64,128,250}, shuffled 64-block pool."""
    from tinyvllm_amd.workloads import decode_tinyllama_f32_b4
    wl = decode_tinyllama_f32_b4(device="cuda")
    out = _ops()(wl.q, wl.k_cache, wl.v_cache, wl.bt_dev, wl.ctx_dev, 32, 4, 64, 16)
    want = paged_decode_ref(wl.host["q"], wl.host["k_cache"], wl.host["v_cache"], wl.block_tables,
                            wl.context_lens, 32, 4, 64, 16)
    assert np.abs(out.cpu().numpy() - want).max() <= 1e-4


# ---- reference edge semantics --------------------------------------------------------

def test_max_context_len_trims_table():
    case = build_case(7, [20, 64], 8, 4, 64, 16, torch.float32, width=8)
    check(case, 8, 4, 64, 16, torch.float32, max_context_len=40)


def test_context_beyond_table_is_truncated():
    q, kc, vc, bt, cl = build_case(8, [30, 64], 8, 4, 64, 16, torch.float32)
    cl = np.array([30, 1000], np.int32)           # seq 1 claims more than its 4 blocks
    check((q, kc, vc, bt, cl), 8, 4, 64, 16, torch.float32)


def test_context_zero_reproduces_reference_mean():
    q, kc, vc, bt, cl = build_case(9, [20, 33], 8, 2, 64, 16, torch.float32)
    q = q * 0.05
    cl = np.array([0, 33], np.int32)
    check((q, kc, vc, bt, cl), 8, 2, 64, 16, torch.float32)


def test_invalid_block_id_gives_nan_not_fault():
    q, kc, vc, bt, cl = build_case(10, [20, 33], 8, 2, 64, 16, torch.float32)
    bt = bt.copy()
    bt[1, 1] = kc.shape[0] + 1000                 # outside the cache
    out = run(q, kc, vc, bt, cl, 8, 2, 64, 16).cpu().numpy()
    assert np.isnan(out[1]).all()
    want = oracle(q[:1], kc, vc, bt[:1], cl[:1], 8, 2, 64, 16)
    assert np.abs(out[:1] - want).max() <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_large_batch_runs_longest_first(dtype):
    """48 sequences of mixed lengths in one partition: the launch is scheduled
    longest first through the workspace; results stay per sequence, including
    ties, a context of 0 (whole padded width) and contexts beyond the table."""
    rng = np.random.Generator(np.random.PCG64(11))
    ctx = rng.integers(1, 200, 48).astype(np.int32)
    ctx[[3, 17, 30]] = 150           # ties
    ctx[5] = 0                        # reference all-masked mean of the padded gather
    case = build_case(12, ctx.tolist(), 16, 4, 128, 16, dtype, width=13)
    q, kc, vc, bt, cl = case
    cl = cl.copy()
    cl[9] = 100000                    # beyond the table: truncated to its width
    check((q, kc, vc, bt, cl), 16, 4, 128, 16, dtype, partition_size=4096)


@pytest.mark.parametrize("spread", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_scheduled_launch_many_sequences(spread, dtype):
    """256 sequences x 8 KV heads in one partition: the scheduled launch, with
    KV head pairs per work-group when the lengths are spread (longest >= 3x
    shortest) and single heads when they are alike; also a context of 0 and
    one beyond the table."""
    rng = np.random.Generator(np.random.PCG64(21))
    ctx = rng.integers(1, 200, 256) if spread else rng.integers(150, 200, 256)
    ctx = ctx.astype(np.int32)
    if spread:
        ctx[7] = 0
    case = build_case(22, ctx.tolist(), 32, 8, 128, 16, dtype, width=13)
    q, kc, vc, bt, cl = case
    cl = cl.copy()
    cl[40] = 100000
    check((q, kc, vc, bt, cl), 32, 8, 128, 16, dtype)


@pytest.mark.parametrize("hq,hkv,d,dtype", [(32, 4, 64, torch.float16), (16, 2, 128, torch.float16),
                                            (24, 6, 64, torch.float16), (32, 4, 64, torch.float32),
                                            (32, 8, 128, torch.bfloat16)])
def test_scheduled_launch_group_shapes(hq, hkv, d, dtype):
    """Scheduled launches over several GQA shapes and dtypes (Hkv / 2 pairs per
    sequence when the item count and the length spread allow it)."""
    rng = np.random.Generator(np.random.PCG64(23))
    ctx = rng.integers(1, 120, 900).astype(np.int32)
    case = build_case(24, ctx.tolist(), hq, hkv, d, 16, dtype, width=8)
    check(case, hq, hkv, d, 16, dtype)


def test_partition_size_recommendation():
    """tv_paged_decode_partition_size: whole context when the batch fills the
    GPU, and for small launches (at most one (sequence, KV head) pair per CU,
    contexts of at most 512 tokens, one launch of wide work-groups); else
    partitions that make a full-width batch's work-groups fill the resident
    work-group slots once; a multiple of 16, at least 64."""
    from tinyvllm_amd.attention import default_partition_size
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    whole = default_partition_size(4 * cus // 8, 32, 8, 128, 256, 16, torch.float16)
    assert whole == 4096
    p = default_partition_size(16, 32, 8, 128, 2048, 16, torch.bfloat16)
    assert p % 16 == 0 and 64 <= p < 32768
    parts = -(-32768 // p)
    assert 16 * 8 * parts >= cus                    # at least one work-group per CU
    assert default_partition_size(4, 32, 4, 64, 16, 16, torch.float32) == 256       # config 1: one launch
    p = default_partition_size(4, 32, 4, 64, 64, 16, torch.float32)                 # 1024-token width: split
    assert p % 16 == 0 and 64 <= p < 1024
    with pytest.raises(ValueError):
        default_partition_size(4, 30, 4, 64, 16, 16, torch.float32)


def test_scheduled_launch_in_graph():
    """The scheduled launch (schedule kernel + paired decode) captured in a HIP
    graph on its first use: every replay, with eager work and synchronisation
    between replays, matches the eager result and the oracle."""
    from tinyvllm_amd.attention import PagedDecodePlan
    rng = np.random.Generator(np.random.PCG64(31))
    ctx = rng.integers(1, 150, 256).astype(np.int32)
    q, kc, vc, bt, cl = build_case(32, ctx.tolist(), 32, 8, 64, 16, torch.float16, width=10)
    dev = "cuda"
    args = [q.to(dev), kc.to(dev), vc.to(dev), torch.from_numpy(bt).to(dev), torch.from_numpy(cl).to(dev)]
    plan = PagedDecodePlan(*args, 32, 8, 64, 16)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            plan.run()
    torch.cuda.synchronize()
    want = oracle(q, kc, vc, bt, cl, 32, 8, 64, 16)
    eager = PagedDecodePlan(*args, 32, 8, 64, 16).run().clone()
    torch.cuda.synchronize()
    assert np.abs(eager.float().cpu().numpy() - want).max() <= 2e-2
    for _ in range(3):
        plan.out.zero_()
        junk = torch.randn(1 << 20, device=dev).sum()    # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(plan.out, eager)
        del junk


def test_deterministic():
    case = build_case(11, [100, 700, 3], 32, 8, 128, 16, torch.float16)
    a = run(*case, 32, 8, 128, 16, partition_size=128)
    b = run(*case, 32, 8, 128, 16, partition_size=128)
    assert torch.equal(a, b)


def test_fp32_output_for_half_inputs():
    case = build_case(12, [50, 9], 8, 8, 64, 16, torch.float16)
    q, kc, vc, bt, cl = case
    out = run(q, kc, vc, bt, cl, 8, 8, 64, 16, out_dtype=torch.float32)
    assert out.dtype == torch.float32
    assert np.abs(out.cpu().numpy() - oracle(*case, 8, 8, 64, 16)).max() <= 2e-2


def test_rejects_bad_arguments():
    q, kc, vc, bt, cl = build_case(13, [10], 8, 2, 64, 16, torch.float32)
    dev = "cuda"
    with pytest.raises(ValueError):
        _ops()(q.to(dev), kc.to(dev), vc.to(dev), torch.from_numpy(bt).long().to(dev),
               torch.from_numpy(cl).to(dev), 8, 2, 64, 16)
    with pytest.raises(ValueError):
        _ops()(q.to(dev), kc.to(dev), vc.to(dev), torch.from_numpy(bt).to(dev),
               torch.from_numpy(cl).to(dev), 8, 4, 64, 16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d", [(32, 4, 64), (32, 8, 128), (16, 4, 64), (8, 4, 128), (12, 2, 64)])
def test_small_launch_wide_work_groups(dtype, hq, hkv, d):
    """Small batches with contexts of at most 512 tokens take one launch of
    8-wave work-groups: GQA groups of 8 / 4 / 6 / 2 heads (groups of 4+ are
    served in chunks of half the heads), waves with one or two 16-token tiles
    (both requested before either is consumed), a partial last block, and a
    zero-length context."""
    ctx = [17, 64, 250, 512, 1, 0]
    case = build_case(2100 + hq + d, [max(c, 1) for c in ctx], hq, hkv, d, 16, dtype)
    q, kc, vc, bt, _ = case
    check((q, kc, vc, bt, np.asarray(ctx, np.int32)), hq, hkv, d, 16, dtype)


# ---- seeded random shapes -------------------------------------------------------------

def _random_decode_cases(n=None, seed=81):
    n = case_count(24) if n is None else n
    rng = np.random.Generator(np.random.PCG64(case_seed(seed)))
    cases = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 4, 8]))
        hq = hkv * int(rng.choice([1, 2, 3, 4, 8]))
        d = int(rng.choice([16, 32, 64, 128, 256]))
        bs = int(rng.choice([16, 16, 32, 8, 1, 12]))
        b = int(rng.choice([1, 3, 17, 40, 64, 300]))
        width = int(rng.integers(1, 40))            # table columns
        while b > 1 and b * width * bs * hkv * d > (8 << 20):   # keeps the float64 oracle small
            b //= 2
        ctx = rng.integers(0, width * bs + 40, b)   # zero, short, past the table
        dtype = [torch.float16, torch.bfloat16, torch.float32][int(rng.integers(0, 3))]
        psize = [None, None, 16, 64, 512][int(rng.integers(0, 5))]
        cases.append((i, hq, hkv, d, bs, width, ctx.astype(np.int32), dtype, psize))
    return cases


@pytest.mark.parametrize("i,hq,hkv,d,bs,width,ctx,dtype,psize", _random_decode_cases())
def test_random_shapes(i, hq, hkv, d, bs, width, ctx, dtype, psize):
    """Seeded random batches, GQA shapes, head dims, block sizes, table widths,
    context lengths (0 and past the table included), dtypes and partition
    sizes against the oracle."""
    q, kc, vc, bt, _ = build_case(600 + i, [max(1, min(int(c), width * bs)) for c in ctx], hq, hkv, d, bs,
                                  dtype, width=width)
    kw = {} if psize is None else {"partition_size": psize}
    check((q, kc, vc, bt, ctx), hq, hkv, d, bs, dtype, **kw)


def test_shared_table_row_stride_zero():
    """block_table_stride 0: every query row reads table row 0 (the query rows of
    one prompt chunk over its sequence's table); equals the same table repeated."""
    from tinyvllm_amd import _lib
    ctx = [5, 16, 17, 40, 64]
    q, kc, vc, bt, _ = build_case(42, [64] * len(ctx), 8, 2, 64, 16, torch.float16)
    row = bt[:1].copy()
    cl = np.asarray(ctx, np.int32)
    dev = "cuda"
    out = torch.empty((len(ctx), 1, 8, 64), dtype=torch.float16, device=dev)
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    row_d, cl_d = torch.from_numpy(row).to(dev), torch.from_numpy(cl).to(dev)
    rc = _lib.load().tv_paged_decode(out.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), row_d.data_ptr(),
                                     cl_d.data_ptr(), len(ctx), 8, 2, 64, 16, kc.shape[0], 0, row.shape[1],
                                     0.125, _lib.TV_F16, _lib.TV_F16, 64 * 16, None, 0, None)
    _lib.check(rc, "tv_paged_decode")
    torch.cuda.synchronize()
    want = oracle(q, kc, vc, np.repeat(row, len(ctx), 0), cl, 8, 2, 64, 16)
    assert np.abs(out.float().cpu().numpy() - want).max() <= TOL[torch.float16]
