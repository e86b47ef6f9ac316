"""Prefill attention on the GPU vs the oracle (tinyvllm/model/llama.py:58-94).

Restates tests/test_flash_attention.py of the reference (shapes, GQA, causal
known answers, sequence lengths, head dims, dtypes, TinyLlama shapes) and adds
MFMA-path parity for fp16/bf16 at the benchmark shapes.
Tolerances (max-abs vs the float64 oracle): fp32 1e-4, fp16/bf16 2e-2.
"""

import numpy as np
import pytest
import torch

from oracle.attention import flash_prefill_ref
from tests.random_cases import case_count, case_seed

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _op():
    from tinyvllm_amd.attention import flash_prefill_attention
    return flash_prefill_attention


def flash(q, k, v, causal=True):
    """[L, H, D] wrapper like the reference test's (adds and removes the batch dim)."""
    out = _op()(q.unsqueeze(0).cuda(), k.unsqueeze(0).cuda(), v.unsqueeze(0).cuda(), causal)
    torch.cuda.synchronize()
    return out.squeeze(0)


def randn(seed, *shape, dtype=torch.float32):
    rng = np.random.Generator(np.random.PCG64(seed))
    return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dtype)


def check(q, k, v, causal=True, tol=None):
    out = flash(q, k, v, causal)
    want = flash_prefill_ref(q.float().numpy()[None], k.float().numpy()[None], v.float().numpy()[None], causal)[0]
    err = np.abs(out.float().cpu().numpy() - want).max()
    tol = TOL[q.dtype] if tol is None else tol
    assert err <= tol, f"max-abs {err} > {tol}"
    return out


# ---- restated reference tests ------------------------------------------------------

def test_output_shape():
    out = flash(randn(0, 16, 8, 64), randn(1, 16, 8, 64), randn(2, 16, 8, 64))
    assert out.shape == (16, 8, 64)


@pytest.mark.parametrize("lq,hq,hkv,d", [(32, 4, 4, 32), (32, 32, 8, 64), (16, 8, 4, 32), (16, 32, 8, 64),
                                          (16, 32, 4, 64), (64, 32, 8, 64), (256, 32, 8, 64)])
def test_matches_standard_attention(lq, hq, hkv, d):
    check(randn(3, lq, hq, d), randn(4, lq, hkv, d), randn(5, lq, hkv, d))


def test_non_causal():
    check(randn(6, 16, 4, 32), randn(7, 16, 4, 32), randn(8, 16, 4, 32), causal=False)


def test_causal_mask_first_token():
    q = torch.zeros(8, 2, 16)
    q[0] = 1.0
    k = randn(9, 8, 2, 16)
    v = torch.eye(8).unsqueeze(1).expand(8, 2, 8).contiguous()     # head_dim_v 8 != head_dim 16
    out = check(q, k, v)
    assert out[0, 0, 0].item() > 0.5


def test_last_token_attends_to_all():
    q = torch.ones(8, 2, 16)
    k = torch.zeros(8, 2, 16)
    v = torch.arange(8).reshape(8, 1, 1).expand(8, 2, 16).float().contiguous()
    out = flash(q, k, v)
    assert abs(out[-1, 0, 0].item() - 3.5) < 1e-2


@pytest.mark.parametrize("q_len", [1, 2, 7, 8, 15, 16, 31, 32, 63, 64, 128])
def test_various_lengths(q_len):
    check(randn(10, q_len, 4, 32), randn(11, q_len, 4, 32), randn(12, q_len, 4, 32))


@pytest.mark.parametrize("head_dim", [32, 64, 128])
def test_various_head_dims(head_dim):
    check(randn(13, 16, 4, head_dim), randn(14, 16, 4, head_dim), randn(15, 16, 4, head_dim))


def test_float16_finite():
    q, k, v = (randn(16 + i, 32, 4, 32, dtype=torch.float16) for i in range(3))
    out = check(q, k, v)
    assert out.shape == (32, 4, 32) and torch.isfinite(out).all()


def test_float32_dtype():
    out = flash(randn(19, 32, 4, 32), randn(20, 32, 4, 32), randn(21, 32, 4, 32))
    assert out.dtype == torch.float32 and out.shape == (32, 4, 32)


# ---- MFMA path (fp16 / bf16, head_dim 64 / 128) --------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("lq", [1, 15, 64, 65, 200])
@pytest.mark.parametrize("causal", [True, False])
def test_mfma_path(dtype, d, lq, causal):
    hq, hkv = 8, 2
    check(randn(22, lq, hq, d, dtype=dtype), randn(23, lq, hkv, d, dtype=dtype),
          randn(24, lq, hkv, d, dtype=dtype), causal)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("lq,hq,hkv", [(300, 8, 2), (1024, 32, 8)])
def test_peaked_softmax(dtype, d, causal, lq, hq, hkv):
    """q, k ~ N(0, 3^2): scores of tens of units, nearly one-hot softmax rows,
    where any rounding of the scores (or of q * scale) before the softmax shows
    up in the output.  The reference scales after the product (llama.py:84), in
    fp32 here; bar: 2e-2 max-abs against the float64 oracle."""
    q = randn(90, lq, hq, d) * 3
    k = randn(91, lq, hkv, d) * 3
    v = randn(92, lq, hkv, d)
    check(q.to(dtype), k.to(dtype), v.to(dtype), causal)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("lq,lk,scale", [(2048, 2048, 1.0), (2100, 2100, 3.0), (2048, 2500, 1.0)])
def test_long_prompts_head_dim_128(dtype, causal, lq, lk, scale):
    """Prompts of 2048+ rows at head_dim 128 take the 128-row kernel with
    LDS-DMA tiles (flash_prefill_rows.hip): full and partial last query and key
    tiles, Lq != Lk (top-left causal), and peaked scores (q, k ~ N(0, 3^2))."""
    q = randn(93, lq, 8, 128) * scale
    k = randn(94, lk, 2, 128) * scale
    v = randn(95, lk, 2, 128)
    check(q.to(dtype), k.to(dtype), v.to(dtype), causal)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("out_dtype", [None, torch.float32])
def test_split_key_halves_workspace_and_fp32_output(dtype, out_dtype):
    """A causal L 2100 prompt at Hq 8 (17 query tiles of 128 rows, all resident
    at once) runs tiles 8-16 as two key halves each, merged by a second kernel
    (flash_prefill_rows.hip): the workspace is sized for the halves, and the
    merged rows match the oracle in the input type and in fp32."""
    from tinyvllm_amd import _lib
    lib = _lib.load()
    lq = 2100
    assert lib.tv_flash_prefill_workspace_bytes(lq, lq, 8, 128, 128, 1, _lib.dtype_code(dtype), 0) > 0
    assert lib.tv_flash_prefill_workspace_bytes(lq, lq, 8, 128, 128, 0, _lib.dtype_code(dtype), 0) == 0
    q = randn(96, lq, 8, 128).to(dtype)
    k = randn(97, lq, 2, 128).to(dtype)
    v = randn(98, lq, 2, 128).to(dtype)
    out = _op()(q.unsqueeze(0).cuda(), k.unsqueeze(0).cuda(), v.unsqueeze(0).cuda(), True, out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert out.dtype == (dtype if out_dtype is None else out_dtype)
    want = flash_prefill_ref(q.float().numpy()[None], k.float().numpy()[None], v.float().numpy()[None], True)[0]
    err = np.abs(out[0].float().cpu().numpy() - want).max()
    assert err <= TOL[dtype], err


def test_split_key_halves_replay_in_graph():
    """The split launch (halves + merge) captured in a HIP graph: replays, with
    eager work between them, equal the eager launch bit for bit."""
    from tinyvllm_amd.attention import PrefillPlan
    q, k, v = (randn(99 + i, 2048, h, 128, dtype=torch.float16).cuda().unsqueeze(0) for i, h in enumerate((8, 2, 2)))
    plan = PrefillPlan(q, k, v)
    assert plan.ws_bytes > 0
    eager = plan.run().clone()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            plan.run()
    torch.cuda.synchronize()
    for _ in range(3):
        plan.out.zero_()
        junk = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(plan.out, eager)
        del junk


def test_split_shape_without_workspace_runs_unsplit():
    """A prompt that would split its key halves, given no workspace through the
    C ABI, runs unsplit and still matches the oracle; a workspace smaller than
    tv_flash_prefill_workspace_bytes asks for is rejected."""
    import math
    from tinyvllm_amd import _lib
    lib = _lib.load()
    lq, hq, hkv, d = 2048, 8, 2, 128
    q, k, v = (randn(110 + i, lq, h, d, dtype=torch.float16) for i, h in enumerate((hq, hkv, hkv)))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    need = lib.tv_flash_prefill_workspace_bytes(lq, lq, hq, d, d, 1, _lib.TV_F16, 0)
    assert need > 0
    out = torch.empty((lq, hq, d), dtype=torch.float16, device="cuda")
    stream = _lib.stream_ptr(torch.device("cuda"))
    args = (out.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), lq, lq, hq, hkv, d, d, hq * d, hkv * d,
            hkv * d, hq * d, 1, 1.0 / math.sqrt(d), _lib.TV_F16, _lib.TV_F16, 0)
    assert lib.tv_flash_prefill(*args, None, 0, stream) == 0
    torch.cuda.synchronize()
    _check_heads(out, q, k, v, True, [0, hkv - 1], torch.float16)
    small = torch.empty(256, dtype=torch.uint8, device="cuda")
    assert lib.tv_flash_prefill(*args, small.data_ptr(), 256, stream) == _lib.TV_EINVAL
    assert b"workspace" in lib.tv_last_error()


def _check_heads(out, q, k, v, causal, groups, dtype):
    """Oracle rows of the query heads of the listed KV groups only (the float64
    oracle over every head of a large grid would take minutes)."""
    hq, hkv = q.shape[1], k.shape[1]
    g = hq // hkv
    for kvh in groups:
        hs = slice(kvh * g, (kvh + 1) * g)
        want = flash_prefill_ref(q[:, hs].float().numpy()[None], k[:, kvh:kvh + 1].float().numpy()[None],
                                 v[:, kvh:kvh + 1].float().numpy()[None], causal)[0]
        err = np.abs(out[:, hs].float().cpu().numpy() - want).max()
        assert err <= TOL[dtype], (kvh, err)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
def test_long_prompt_grid_larger_than_resident(dtype, causal):
    """Hq 48 / Hkv 8 at L 2100: 816 work-groups of the 128-row kernel, more
    than are resident at once, so query tiles are dealt longest first (an odd
    tile count and a partial last tile); rows of two KV groups' query heads
    against the oracle -- the tile order is the same for every head."""
    lq = 2100
    q = randn(140, lq, 48, 128).to(dtype)
    k = randn(141, lq, 8, 128).to(dtype)
    v = randn(142, lq, 8, 128).to(dtype)
    out = flash(q, k, v, causal)
    _check_heads(out, q, k, v, causal, [0, 7], dtype)


def test_varlen_long_prompts_grid_larger_than_resident():
    """Two long prompts packed (Hq 32: grid 32 x 18 x 2 = 1152 work-groups of
    the 128-row kernel, longest-first tiles within each prompt)."""
    from tinyvllm_amd.attention import flash_prefill_varlen
    lens = [2300, 2048]
    tot = sum(lens)
    q, k, v = (randn(143 + i, tot, 32 if i == 0 else 8, 128, dtype=torch.float16) for i in range(3))
    out = flash_prefill_varlen(q.cuda(), k.cuda(), v.cuda(), lens, True)
    torch.cuda.synchronize()
    s = 0
    for n in lens:
        sl = slice(s, s + n)
        _check_heads(out[sl], q[sl], k[sl], v[sl], True, [0, 5], torch.float16)
        s += n


@pytest.mark.parametrize("length", [512, 1024])
def test_tinyllama_prefill_shape(length):
    """TinyLlama prefill shape: Hq 32, Hkv 4, D 64, fp16 inputs, causal."""
    q, k, v = (randn(30 + i, length, 32 if i == 0 else 4, 64, dtype=torch.float16) for i in range(3))
    check(q, k, v)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("lq,lk,causal", [(600, 600, False), (520, 520, True), (500, 700, True), (480, 900, False)])
def test_key_split_work_groups(dtype, lq, lk, causal, d):
    """Grids of at most one work-group per CU with rows of 8+ key tiles run two
    key groups per work-group and merge them in LDS."""
    q = randn(70, lq, 8, d, dtype=dtype)
    k = randn(71, lk, 2, d, dtype=dtype)
    v = randn(72, lk, 2, d, dtype=dtype)
    check(q, k, v, causal)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("lq,lk,causal", [(600, 600, False), (700, 900, True)])
def test_key_split_short_tiles(dtype, lq, lk, causal, d):
    """Between one and four work-groups per CU (Hq 32) with long rows: two key
    groups of 32-key tiles per work-group."""
    q = randn(73, lq, 32, d, dtype=dtype)
    k = randn(74, lk, 4, d, dtype=dtype)
    v = randn(75, lk, 4, d, dtype=dtype)
    check(q, k, v, causal)


@pytest.mark.parametrize("length", [512, 2048])
def test_llama3_8b_head_prefill(length):
    """Llama-3-8B head shape (Hq 32, Hkv 8, head_dim 128), fp16, causal."""
    q, k, v = (randn(80 + i, length, 32 if i == 0 else 8, 128, dtype=torch.float16) for i in range(3))
    check(q, k, v)


def test_unequal_lengths_top_left_causal():
    q = randn(40, 40, 8, 64, dtype=torch.float16)
    k = randn(41, 100, 2, 64, dtype=torch.float16)
    v = randn(42, 100, 2, 64, dtype=torch.float16)
    check(q, k, v, True)
    q32 = randn(43, 10, 4, 32)
    check(q32, randn(44, 30, 4, 32), randn(45, 30, 4, 32), True)


def test_strided_inputs_from_fused_qkv():
    """q/k/v as views into one [L, (Hq+2Hkv)*D] projection output."""
    L, hq, hkv, d = 96, 8, 2, 64
    qkv = randn(46, L, (hq + 2 * hkv) * d, dtype=torch.float16).cuda()
    q = qkv[:, :hq * d].view(L, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(L, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(L, hkv, d)
    out = _op()(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), True)[0]
    want = flash_prefill_ref(q.float().cpu().numpy()[None], k.float().cpu().numpy()[None],
                             v.float().cpu().numpy()[None], True)[0]
    assert np.abs(out.float().cpu().numpy() - want).max() <= 2e-2


def test_rejects_batch_above_one():
    q = randn(47, 2, 8, 4, 32).cuda()
    with pytest.raises(ValueError, match="batch 1"):
        _op()(q, q[:, :, :4], q[:, :, :4], True)


@pytest.mark.parametrize("chunk_tiles", [1, 2, 3, 5])
@pytest.mark.parametrize("lq,causal", [(130, True), (500, True), (200, False)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mfma_split_rows_merge(chunk_tiles, lq, causal, dtype):
    """Long rows split into key chunks on separate work-groups, merged by a second kernel."""
    q, k, v = (randn(60 + i, lq, 8 if i == 0 else 2, 64, dtype=dtype) for i in range(3))
    out = _op()(q.unsqueeze(0).cuda(), k.unsqueeze(0).cuda(), v.unsqueeze(0).cuda(), causal,
                chunk_tiles=chunk_tiles)[0]
    want = flash_prefill_ref(q.float().numpy()[None], k.float().numpy()[None], v.float().numpy()[None], causal)[0]
    assert np.abs(out.float().cpu().numpy() - want).max() <= 2e-2


# ---- seeded random shapes -------------------------------------------------------------

def _random_prefill_cases(n=None, seed=71):
    n = case_count(24) if n is None else n
    rng = np.random.Generator(np.random.PCG64(case_seed(seed)))
    cases = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 4, 8]))
        hq = hkv * int(rng.choice([1, 2, 4, 8]))
        d = int(rng.choice([64, 128, 64, 128, 32, 80]))
        lq = int(rng.integers(1, 700))
        lk = lq if rng.random() < 0.7 else int(rng.integers(1, 700))
        causal = bool(rng.random() < 0.7)
        dtype = [torch.float16, torch.bfloat16, torch.float32][int(rng.integers(0, 3))]
        chunk = int(rng.choice([0, 0, 0, 1, 2, 4]))
        cases.append((i, hq, hkv, d, lq, lk, causal, dtype, chunk))
    return cases


@pytest.mark.parametrize("i,hq,hkv,d,lq,lk,causal,dtype,chunk", _random_prefill_cases())
def test_random_shapes(i, hq, hkv, d, lq, lk, causal, dtype, chunk):
    """Seeded random head counts, head dims (MFMA and generic), lengths
    (Lq != Lk included), masks, dtypes and key-chunk splits against the oracle."""
    q = randn(300 + i, lq, hq, d, dtype=dtype)
    k = randn(400 + i, lk, hkv, d, dtype=dtype)
    v = randn(500 + i, lk, hkv, d, dtype=dtype)
    out = _op()(q.unsqueeze(0).cuda(), k.unsqueeze(0).cuda(), v.unsqueeze(0).cuda(), causal,
                chunk_tiles=chunk)[0]
    torch.cuda.synchronize()
    want = flash_prefill_ref(q.float().numpy()[None], k.float().numpy()[None], v.float().numpy()[None], causal)[0]
    assert np.abs(out.float().cpu().numpy() - want).max() <= TOL[dtype]


def _random_split_cases(n=None, seed=83):
    n = case_count(6) if n is None else n
    rng = np.random.Generator(np.random.PCG64(case_seed(seed)))
    cases = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 4]))
        hq = hkv * int(rng.choice([2, 4, 8]))
        hq = min(hq, 16)
        lq = int(rng.integers(2048, 3300 if hq <= 8 else 2560))   # grids that leave resident slots free
        lk = lq if rng.random() < 0.6 else lq + int(rng.integers(1, 500))
        dtype = [torch.float16, torch.bfloat16][int(rng.integers(0, 2))]
        out_f32 = bool(rng.random() < 0.3)
        scale = 3.0 if rng.random() < 0.3 else 1.0
        cases.append((i, hq, hkv, lq, lk, dtype, out_f32, scale))
    return cases


@pytest.mark.parametrize("i,hq,hkv,lq,lk,dtype,out_f32,scale", _random_split_cases())
def test_random_split_key_halves(i, hq, hkv, lq, lk, dtype, out_f32, scale):
    """Seeded random causal prompts of 2048+ rows at head_dim 128 with few heads
    (1-16 query heads over 1-4 KV heads), so the 128-row kernel runs the longer
    query tiles as two key halves and merges them: Lk >= Lq, fp16 / bf16,
    outputs in the input type or fp32, and peaked scores; rows of the first and
    last KV groups' query heads against the oracle."""
    from tinyvllm_amd import _lib
    lib = _lib.load()
    assert lib.tv_flash_prefill_workspace_bytes(lq, lk, hq, 128, 128, 1, _lib.dtype_code(dtype), 0) > 0
    q = (randn(600 + i, lq, hq, 128) * scale).to(dtype)
    k = (randn(700 + i, lk, hkv, 128) * scale).to(dtype)
    v = randn(800 + i, lk, hkv, 128).to(dtype)
    out = _op()(q.unsqueeze(0).cuda(), k.unsqueeze(0).cuda(), v.unsqueeze(0).cuda(), True,
                out_dtype=torch.float32 if out_f32 else None)[0]
    torch.cuda.synchronize()
    _check_heads(out, q, k, v, True, sorted({0, hkv - 1}), dtype)


# ---- several prompts per launch (no reference counterpart) ------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("lens,hq,hkv,d,causal", [
    ([512, 1024], 32, 4, 64, True),            # the TinyLlama prompts of the benchmark in one launch
    ([1, 17, 64, 300, 65], 8, 2, 64, True),    # ragged, single-token and tile-boundary prompts
    ([129, 7, 1000], 16, 8, 128, True),
    ([33, 200, 64], 8, 8, 64, False),
    ([300, 41, 512], 8, 2, 64, True),          # <= 256 work-groups with long rows: two key groups + LDS merge
    ([300, 41, 512], 8, 2, 128, True),
    ([2048, 300, 2200], 8, 2, 128, True),      # longest prompt >= 2048 at head_dim 128: the 128-row kernel
])
def test_varlen_matches_per_prompt(lens, hq, hkv, d, causal, dtype):
    """Every prompt of a packed batch equals the oracle on that prompt alone and
    the single-prompt launch (each within the fp16/bf16 bar)."""
    from tinyvllm_amd.attention import flash_prefill_varlen
    tot = sum(lens)
    q, k, v = randn(60, tot, hq, d, dtype=dtype), randn(61, tot, hkv, d, dtype=dtype), randn(62, tot, hkv, d, dtype=dtype)
    out = flash_prefill_varlen(q.cuda(), k.cuda(), v.cuda(), lens, causal)
    torch.cuda.synchronize()
    assert out.shape == (tot, hq, d) and out.dtype == dtype
    got = out.float().cpu().numpy()
    s = 0
    for n in lens:
        sl = slice(s, s + n)
        want = flash_prefill_ref(q[sl].float().numpy()[None], k[sl].float().numpy()[None],
                                 v[sl].float().numpy()[None], causal)[0]
        assert np.abs(got[sl] - want).max() <= TOL[dtype], (n, s)
        single = flash(q[sl], k[sl], v[sl], causal).float().cpu().numpy()
        assert np.abs(got[sl] - single).max() <= TOL[dtype], (n, s)
        s += n


def _random_varlen_cases(n=None, seed=73):
    n = case_count(8) if n is None else n
    rng = np.random.Generator(np.random.PCG64(case_seed(seed)))
    cases = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 4, 8]))
        hq = hkv * int(rng.choice([1, 2, 4, 8]))
        d = int(rng.choice([64, 128]))
        lens = [int(x) for x in rng.integers(1, 700, int(rng.integers(1, 6)))]
        causal = bool(rng.random() < 0.7)
        dtype = [torch.float16, torch.bfloat16][int(rng.integers(0, 2))]
        cases.append((i, lens, hq, hkv, d, causal, dtype))
    return cases


@pytest.mark.parametrize("i,lens,hq,hkv,d,causal,dtype", _random_varlen_cases())
def test_random_varlen(i, lens, hq, hkv, d, causal, dtype):
    """Seeded random packs of 1-5 prompts (lengths 1-699), GQA shapes, head
    dims, masks and dtypes: every prompt equals the oracle and its own launch."""
    test_varlen_matches_per_prompt(lens, hq, hkv, d, causal, dtype)


def test_varlen_fp32_output_and_strided_inputs():
    """fp32 output, and q/k/v as views into one fused [T, (Hq + 2 Hkv) * D] buffer."""
    from tinyvllm_amd.attention import flash_prefill_varlen
    lens = [70, 3, 130]
    tot, hq, hkv, d = sum(lens), 8, 2, 64
    fused = randn(70, tot, (hq + 2 * hkv) * d, dtype=torch.bfloat16).cuda()
    q = fused[:, :hq * d].view(tot, hq, d)
    k = fused[:, hq * d:(hq + hkv) * d].view(tot, hkv, d)
    v = fused[:, (hq + hkv) * d:].view(tot, hkv, d)
    out = flash_prefill_varlen(q, k, v, lens, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    s = 0
    for n in lens:
        sl = slice(s, s + n)
        want = flash_prefill_ref(q[sl].float().cpu().numpy()[None], k[sl].float().cpu().numpy()[None],
                                 v[sl].float().cpu().numpy()[None], True)[0]
        assert np.abs(out[sl].cpu().numpy() - want).max() <= TOL[torch.bfloat16], n
        s += n


def test_varlen_plan_replays_in_graph():
    """The plan captured in a HIP graph: replays (with eager work between them)
    equal the eager launch."""
    from tinyvllm_amd.attention import VarlenPrefillPlan
    lens = [300, 41, 512]
    tot = sum(lens)
    q, k, v = (randn(63 + i, tot, h, 64, dtype=torch.float16).cuda() for i, h in enumerate((8, 2, 2)))
    plan = VarlenPrefillPlan(q, k, v, lens)
    eager = plan.run().clone()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            plan.run()
    torch.cuda.synchronize()
    for _ in range(3):
        plan.out.zero_()
        junk = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(plan.out, eager)
        del junk


def test_varlen_rejects_bad_arguments():
    from tinyvllm_amd.attention import flash_prefill_varlen
    q = torch.zeros((10, 4, 64), dtype=torch.float16, device="cuda")
    k = torch.zeros((10, 2, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        flash_prefill_varlen(q, k, k, [4, 5])                  # lengths do not sum to T
    with pytest.raises(ValueError):
        flash_prefill_varlen(q, k, k, [10, 0])                 # empty prompt
    with pytest.raises(RuntimeError, match="head_dim 64 or 128"):
        flash_prefill_varlen(q.float(), k.float(), k.float(), [10])   # fp32: MFMA path only


# ---- a chunk attending through the paged cache (no reference counterpart) -----------------

def _paged_case(seed, total, hkv, d, bs, dtype, spare=5):
    """A sequence of `total` tokens' K/V scattered over a shuffled block pool."""
    rng = np.random.Generator(np.random.PCG64(seed))
    nblk = -(-total // bs)
    pool = nblk + spare
    table = rng.permutation(pool)[:nblk].astype(np.int32)
    k = randn(seed + 1, total, hkv, d, dtype=dtype)
    v = randn(seed + 2, total, hkv, d, dtype=dtype)
    kc = torch.zeros((pool, bs, hkv, d), dtype=dtype)
    vc = torch.zeros_like(kc)
    pos = np.arange(total)
    kc.view(pool * bs, hkv, d)[torch.from_numpy(table[pos // bs] * bs + pos % bs).long()] = k
    vc.view(pool * bs, hkv, d)[torch.from_numpy(table[pos // bs] * bs + pos % bs).long()] = v
    return k, v, kc, vc, table


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d,hq,hkv", [(64, 32, 4), (128, 8, 2)])
@pytest.mark.parametrize("start,n,bs,causal", [(0, 100, 16, True), (300, 77, 16, True), (1000, 256, 16, True),
                                               (64, 64, 4, True), (200, 50, 32, False), (3584, 512, 16, True)])
def test_paged_prefill_equals_last_rows_of_whole_prompt(dtype, d, hq, hkv, start, n, bs, causal):
    """flash_prefill_paged: a chunk at start_pos reading K/V through a shuffled
    block table equals the last n rows of prefill attention over the whole
    sequence (the oracle on the contiguous rows; causal bottom-right aligned,
    key j <= start + i), for block sizes 4, 16 and 32."""
    from tinyvllm_amd.attention import flash_prefill_paged
    total = start + n
    k, v, kc, vc, table = _paged_case(200 + start + n, total, hkv, d, bs, dtype)
    q = randn(97, total, hq, d, dtype=dtype)
    out = flash_prefill_paged(q[start:].cuda(), kc.cuda(), vc.cuda(), torch.from_numpy(table).cuda(), start, causal)
    torch.cuda.synchronize()
    want = flash_prefill_ref(q[start:].float().numpy()[None], k.float().numpy()[None], v.float().numpy()[None],
                             causal, q_offset=start)[0]
    assert np.abs(out[0].float().cpu().numpy() - want).max() <= TOL[dtype]


def _random_paged_prefill_cases(n=None, seed=77):
    n = case_count(8) if n is None else n
    rng = np.random.Generator(np.random.PCG64(case_seed(seed)))
    cases = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 4, 8]))
        hq = hkv * int(rng.choice([1, 2, 4, 8]))
        d = int(rng.choice([64, 128]))
        bs = int(rng.choice([4, 8, 16, 16, 32]))
        start = int(rng.integers(0, 1500))
        n_rows = int(rng.integers(1, 400))
        causal = bool(rng.random() < 0.8)
        dtype = [torch.float16, torch.bfloat16][int(rng.integers(0, 2))]
        cases.append((i, dtype, d, hq, hkv, start, n_rows, bs, causal))
    return cases


@pytest.mark.parametrize("i,dtype,d,hq,hkv,start,n,bs,causal", _random_paged_prefill_cases())
def test_random_paged_prefill(i, dtype, d, hq, hkv, start, n, bs, causal):
    """Seeded random chunks (start 0-1499, 1-399 rows) over shuffled block pools
    of block size 4-32: the chunk equals the last rows of the whole prompt."""
    test_paged_prefill_equals_last_rows_of_whole_prompt(dtype, d, hq, hkv, start, n, bs, causal)


@pytest.mark.parametrize("dtype,out_dtype", [(torch.float16, None), (torch.bfloat16, None),
                                             (torch.float16, torch.float32), (torch.bfloat16, torch.float32)])
def test_paged_prefill_invalid_block_id_gives_nan(dtype, out_dtype):
    # the NaNs are written as bit patterns (the kernel has no NaN arithmetic):
    # every element of the head's rows is a quiet NaN of the output type
    from tinyvllm_amd.attention import flash_prefill_paged
    k, v, kc, vc, table = _paged_case(5, 80, 2, 64, 16, dtype)
    table[2] = kc.shape[0] + 7
    q = randn(98, 16, 8, 64, dtype=dtype)
    out = flash_prefill_paged(q.cuda(), kc.cuda(), vc.cuda(), torch.from_numpy(table).cuda(), 64, True,
                              out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert out.dtype == (dtype if out_dtype is None else out_dtype)
    assert torch.isnan(out.float()).all()


def test_paged_prefill_rejects_bad_arguments():
    from tinyvllm_amd.attention import flash_prefill_paged
    kc = torch.zeros((4, 16, 2, 64), dtype=torch.float16, device="cuda")
    q = torch.zeros((8, 4, 64), dtype=torch.float16, device="cuda")
    table = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):
        flash_prefill_paged(q, kc, kc, table, 30)                      # table covers 32 positions, needs 38
    kc3 = torch.zeros((4, 12, 2, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="power of two"):
        flash_prefill_paged(q, kc3, kc3, table, 0)
