"""Decode-step kernels and the LLaMA model on the GPU vs the oracle (oracle/llama.py).

Kernel level (through the C ABI, include/tv_llama.h): the skinny MFMA product
with its three epilogues against numpy, RMSNorm + residual, RoPE + K/V cache
write (slot placement bit-exact), greedy sampling / advance.
Model level: prefill and batched decode of small configs (fp16 and fp32, the
reference's default model dtype) and of the TinyLlama 1.1B shape against the
float32 oracle (logits <= 2e-2 max-abs for fp16, 1e-4 for fp32),
the reference's K/V order, graph replay vs eager launches (bit-identical, the
reference's determinism test, test_jit_decode.py:138-171), and the
device-resident multi-step loop.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle.llama import LlamaRef, apply_rope_ref, greedy_ref, rms_norm_ref, rope_tables_ref
from tests.random_cases import case_count, case_seed

pytestmark = pytest.mark.gpu

TOL = 2e-2


def lib():
    from tinyvllm_amd import _lib
    return _lib.load()


def check(rc, what):
    from tinyvllm_amd import _lib
    _lib.check(rc, what)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def gen(seed, *shape, dtype=torch.float16, scale=1.0):
    rng = np.random.default_rng(seed)
    return torch.from_numpy((scale * rng.standard_normal(shape)).astype(np.float32)).to(dtype).cuda()


def f64(t):
    return t.double().cpu().numpy()


# ---- linear -----------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K,ks", [(1, 64, 32, 32), (5, 100, 96, 32), (64, 2560, 2048, 256),
                                      (70, 132, 320, 64), (130, 64, 512, 512), (64, 2048, 5632, 768),
                                      (3, 40, 800, 800),
                                      # whole 256-wide chunks (direct-to-LDS A): ragged N and M, 1-5 chunks
                                      # per split, padded pipeline steps, a short last split
                                      (33, 100, 1024, 512), (64, 2048, 5632, 1024), (17, 84, 1280, 1280),
                                      (64, 148, 2560, 768)])
def test_linear_partial(dtype, M, N, K, ks):
    from tinyvllm_amd._lib import dtype_code
    a = gen(1, M, K, dtype=dtype)
    w = gen(2, N, K, dtype=dtype, scale=0.05)
    splits = -(-K // ks)
    part = torch.full((splits, M, N), float("nan"), dtype=torch.float32, device="cuda")
    check(lib().tv_linear(ptr(part), ptr(a), ptr(w), M, N, K, K, 0, ks, 0, None, dtype_code(dtype), None), "linear")
    torch.cuda.synchronize()
    A, W, P = f64(a), f64(w), part.double().cpu().numpy()
    for s in range(splits):
        want = A[:, s * ks:(s + 1) * ks] @ W[:, s * ks:(s + 1) * ks].T
        assert np.abs(P[s] - want).max() < 1e-4 * max(1.0, np.abs(want).max()), s


@pytest.mark.parametrize("K,lda,ks", [(96, 160, 96), (512, 776, 256)])
def test_linear_strided_a(K, lda, ks):
    """A rows at a stride larger than K (a view into a wider activation buffer)."""
    from tinyvllm_amd._lib import TV_F16
    big = gen(3, 9, lda)
    a = big[:, :K]
    w = gen(4, 64, K, scale=0.05)
    splits = -(-K // ks)
    part = torch.empty((splits, 9, 64), dtype=torch.float32, device="cuda")
    check(lib().tv_linear(ptr(part), ptr(a), ptr(w), 9, 64, K, lda, 0, ks, 0, None, TV_F16, None), "linear")
    torch.cuda.synchronize()
    want = f64(a) @ f64(w).T
    assert np.abs(part.sum(0).double().cpu().numpy() - want).max() < 1e-4 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,H,K", [(4, 48, 64), (64, 5632, 2048), (65, 96, 256), (16, 40, 4096)])
def test_linear_swiglu(dtype, M, H, K):
    from tinyvllm_amd._lib import dtype_code
    a = gen(5, M, K, dtype=dtype)
    w1 = gen(6, H, K, dtype=dtype, scale=0.04)
    w3 = gen(7, H, K, dtype=dtype, scale=0.04)
    w13 = torch.stack([w1.view(H // 2, 2, K), w3.view(H // 2, 2, K)], 1).reshape(2 * H, K).contiguous()
    out = torch.full((M, H), float("nan"), dtype=dtype, device="cuda")
    check(lib().tv_linear(ptr(out), ptr(a), ptr(w13), M, 2 * H, K, K, H, K, 1, None, dtype_code(dtype), None),
          "swiglu")
    torch.cuda.synchronize()
    g, u = f64(a) @ f64(w1).T, f64(a) @ f64(w3).T
    want = g / (1 + np.exp(-g)) * u
    tol = 1e-5 if dtype == torch.float32 else TOL
    assert np.abs(out.double().cpu().numpy() - want).max() < tol * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(3, 100, 64), (64, 32000, 2048), (70, 260, 96), (70, 260, 768)])
def test_linear_logits_and_greedy(M, N, K, dtype):
    from tinyvllm_amd._lib import dtype_code
    a = gen(8, M, K, dtype=dtype)
    w = gen(9, N, K, dtype=dtype, scale=0.05)
    logits = torch.empty((M, N), dtype=torch.float32, device="cuda")
    nparts = -(-N // 64)
    keys = torch.zeros((nparts, M), dtype=torch.int64, device="cuda")
    check(lib().tv_linear(ptr(logits), ptr(a), ptr(w), M, N, K, K, N, K, 2, ptr(keys), dtype_code(dtype), None),
          "logits")
    toks = torch.zeros(M, dtype=torch.int32, device="cuda")
    check(lib().tv_argmax_advance(ptr(toks), None, None, None, 0, ptr(keys), nparts, M, None), "argmax")
    torch.cuda.synchronize()
    L = logits.double().cpu().numpy()
    want = f64(a) @ f64(w).T
    assert np.abs(L - want).max() < 1e-4 * max(1.0, np.abs(want).max())
    # the sampled token is the first maximum of the very values written
    assert np.array_equal(toks.cpu().numpy(), np.argmax(logits.cpu().numpy(), axis=1))


def test_greedy_tie_resolves_to_first_index():
    """Two identical, dominant rows in different work-group tiles (5 and 70): every
    token ties between them and must take 5 (numpy / tinygrad argmax semantics)."""
    from tinyvllm_amd._lib import TV_F16
    M, N, K = 7, 128, 64
    a = gen(30, M, K).abs()
    w = gen(31, N, K, scale=0.01)
    w[5] = 0.5
    w[70] = 0.5
    keys = torch.zeros((2, M), dtype=torch.int64, device="cuda")
    check(lib().tv_linear(None, ptr(a), ptr(w), M, N, K, K, N, K, 2, ptr(keys), TV_F16, None), "logits")
    toks = torch.zeros(M, dtype=torch.int32, device="cuda")
    check(lib().tv_argmax_advance(ptr(toks), None, None, None, 0, ptr(keys), 2, M, None), "argmax")
    torch.cuda.synchronize()
    assert toks.cpu().tolist() == [5] * M


def test_argmax_advance_updates_state():
    from tinyvllm_amd._lib import TV_F16
    M, N, K = 4, 128, 32
    a, w = gen(10, M, K), gen(11, N, K)
    keys = torch.zeros((2, M), dtype=torch.int64, device="cuda")
    check(lib().tv_linear(None, ptr(a), ptr(w), M, N, K, K, N, K, 2, ptr(keys), TV_F16, None), "logits")
    toks = torch.zeros(M, dtype=torch.int32, device="cuda")
    pos = torch.tensor([0, 5, 9, 3], dtype=torch.int32, device="cuda")
    ctx = pos + 1
    hist = torch.full((M, 8), -1, dtype=torch.int32, device="cuda")
    check(lib().tv_argmax_advance(ptr(toks), ptr(pos), ptr(ctx), ptr(hist), 8, ptr(keys), 2, M, None), "adv")
    torch.cuda.synchronize()
    want = np.argmax(f64(a) @ f64(w).T, axis=1)
    assert np.array_equal(toks.cpu().numpy(), want)
    assert pos.tolist() == [1, 6, 10, 4] and ctx.tolist() == [2, 7, 11, 5]
    h = hist.cpu().numpy()
    assert h[0, 1] == want[0] and h[1, 6] == want[1] and h[3, 4] == want[3]
    assert (h[2] == -1).all()                  # position 9 + 1 is past the history width: not written
    assert (h == -1).sum() == 4 * 8 - 3


# ---- norm / rope --------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_rms_norm_residual_embed_and_add(dtype):
    from tinyvllm_amd._lib import dtype_code
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    M, dim, V = 6, 256, 50
    emb = gen(12, V, dim, dtype=dtype)
    w = gen(13, dim, dtype=torch.float32, scale=0.3) + 1
    toks = torch.tensor([0, 7, 49, 3, 3, 22], dtype=torch.int32, device="cuda")
    x = torch.empty((M, dim), dtype=torch.float32, device="cuda")
    xh = torch.empty((M, dim), dtype=dtype, device="cuda")
    check(lib().tv_rms_norm_residual(ptr(x), ptr(xh), None, 0, ptr(emb), ptr(toks), V, ptr(w), M, dim, 1e-5,
                                     dtype_code(dtype), None), "embed")
    torch.cuda.synchronize()
    X = emb.float().cpu().numpy()[toks.cpu().numpy()]
    assert np.array_equal(x.cpu().numpy(), X)
    want = rms_norm_ref(X, w.cpu().numpy())
    assert np.abs(xh.float().cpu().numpy() - want).max() < tol * np.abs(want).max()
    part = gen(14, 3, M, dim, dtype=torch.float32)
    check(lib().tv_rms_norm_residual(ptr(x), ptr(xh), ptr(part), 3, None, None, 0, ptr(w), M, dim, 1e-5,
                                     dtype_code(dtype), None), "residual")
    torch.cuda.synchronize()
    P = part.cpu().numpy()
    X2 = ((X + P[0]) + P[1]) + P[2]
    assert np.abs(x.cpu().numpy() - X2).max() < 1e-6
    want = rms_norm_ref(X2, w.cpu().numpy())
    assert np.abs(xh.float().cpu().numpy() - want).max() < tol * np.abs(want).max()


def test_rope_table_matches_oracle():
    """Table vs the float64 closed form.  The reference computes the angles in
    float32 (llama.py:28-30), so an ulp of a frequency grows with the position:
    the bound is 4 ulps of the float32 angle (plus cos/sin rounding); the oracle's
    own float32 table obeys the same bound."""
    P, D = 512, 64
    t = torch.empty((P, D // 2, 2), dtype=torch.float32, device="cuda")
    check(lib().tv_rope_table(ptr(t), P, D, 10000.0, None), "rope_table")
    torch.cuda.synchronize()
    ang = np.arange(P)[:, None] * (10000.0 ** (-np.arange(0, D, 2) / D))[None]
    bound = 4 * np.spacing(ang.astype(np.float32)).astype(np.float64) + 2e-7
    T = t.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(T[..., 0] - np.cos(ang)) <= bound) and np.all(np.abs(T[..., 1] - np.sin(ang)) <= bound)
    cos, sin = rope_tables_ref(D, P)
    assert np.all(np.abs(cos - np.cos(ang)) <= bound) and np.all(np.abs(sin - np.sin(ang)) <= bound)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("write_cache", [True, False])
def test_qkv_rope_cache(write_cache, dtype):
    from tinyvllm_amd._lib import dtype_code
    tol = 1e-5 if dtype == torch.float32 else 4e-3
    M, Hq, Hkv, D, bs, NB, splits = 5, 4, 2, 32, 4, 12, 3
    N = (Hq + 2 * Hkv) * D
    part = gen(15, splits, M, N, dtype=torch.float32)
    rope = torch.empty((64, D // 2, 2), dtype=torch.float32, device="cuda")
    check(lib().tv_rope_table(ptr(rope), 64, D, 10000.0, None), "rope")
    pos = torch.tensor([0, 3, 9, 14, 40], dtype=torch.int32, device="cuda")
    bt_np = np.array([[5, 1, 0, 0], [2, 0, 0, 0], [7, 9, 11, 0], [3, 4, 6, 8], [10, 0, 0, 0]], dtype=np.int32)
    bt_np[1, 0] = 99                          # row 1's block is outside the cache: not written, counted
    bt = torch.from_numpy(bt_np).cuda()        # row 4's position 40 is past its table (4 blocks of 4): counted
    q = torch.empty((M, Hq * D), dtype=dtype, device="cuda")
    ko = torch.empty((M, Hkv * D), dtype=dtype, device="cuda")
    vo = torch.empty_like(ko)
    kc = torch.zeros((NB, bs, Hkv, D), dtype=dtype, device="cuda")
    vc = torch.zeros_like(kc)
    slots = torch.full((M,), 123, dtype=torch.int32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    check(lib().tv_qkv_rope_cache(ptr(q), ptr(ko), ptr(vo), ptr(kc) if write_cache else None,
                                  ptr(vc) if write_cache else None, ptr(part), splits, ptr(pos), 0, ptr(rope), 64,
                                  ptr(bt), 4, 4, bs, NB, M, Hq, Hkv, D, dtype_code(dtype), ptr(slots), ptr(err),
                                  None), "qkv")
    torch.cuda.synchronize()
    S = part.cpu().numpy().sum(0)
    P = pos.cpu().numpy()
    cos, sin = rope_tables_ref(D, 64)
    c, s = cos[P][:, None], sin[P][:, None]
    wq = apply_rope_ref(S[:, :Hq * D].reshape(M, Hq, D), c, s)
    wk = apply_rope_ref(S[:, Hq * D:(Hq + Hkv) * D].reshape(M, Hkv, D), c, s)
    wv = S[:, (Hq + Hkv) * D:].reshape(M, Hkv, D)
    assert np.abs(q.float().cpu().numpy().reshape(M, Hq, D) - wq).max() < tol * np.abs(wq).max()
    assert np.abs(ko.float().cpu().numpy().reshape(M, Hkv, D) - wk).max() < tol * np.abs(wk).max()
    assert np.abs(vo.float().cpu().numpy().reshape(M, Hkv, D) - wv).max() < tol * np.abs(wv).max()
    want_slots = [5 * 4 + 0, -1, 11 * 4 + 1, 8 * 4 + 2, -1]
    assert slots.cpu().tolist() == want_slots and err.item() == 2
    K, Vc = kc.cpu().numpy().reshape(NB * bs, Hkv, D), vc.cpu().numpy().reshape(NB * bs, Hkv, D)
    if write_cache:
        written = {sl: m for m, sl in enumerate(want_slots) if sl >= 0}
        for sl in range(NB * bs):
            if sl in written:
                m = written[sl]
                assert np.array_equal(K[sl], ko.cpu().numpy().reshape(M, Hkv, D)[m])
                assert np.array_equal(Vc[sl], vo.cpu().numpy().reshape(M, Hkv, D)[m])
            else:
                assert not K[sl].any() and not Vc[sl].any()
    else:
        assert not K.any() and not Vc.any()


# ---- model ------------------------------------------------------------------------------------

def small_config(**kw):
    from tinyvllm_amd.llama import LlamaConfig
    args = dict(dim=128, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=512, hidden_dim=256, max_seq_len=128,
                dtype="float16")
    args.update(kw)
    return LlamaConfig(**args)


def numpy_weights(weights):
    return {k: v.float().cpu().numpy() for k, v in weights.items()}


def build(cfg, seed=0, std=0.05, write_before_attend=True, num_blocks=64, block_size=16, act_rounding=False):
    from tinyvllm_amd.block_manager import BlockManager
    from tinyvllm_amd.kv_cache import KVCache
    from tinyvllm_amd.llama import Llama, random_weights
    weights = random_weights(cfg, seed=seed, std=std)
    # non-trivial norm weights so the norm weight path is exercised
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    for k in list(weights):
        if k.endswith("norm.weight"):
            weights[k] = 1 + 0.2 * torch.randn(weights[k].shape, generator=g, device="cuda")
    model = Llama(cfg, weights, write_before_attend=write_before_attend)
    kv = KVCache(cfg.n_layers, num_blocks, block_size, cfg.n_kv_heads, cfg.head_dim, cfg.dtype)
    bm = BlockManager(1, num_blocks, block_size)
    cache_dtype = {torch.float32: np.float32, torch.float16: np.float16, torch.bfloat16: "bfloat16"}[cfg.dtype]
    ref = LlamaRef(cfg, numpy_weights(weights), cache_dtype=cache_dtype,
                   act_dtype=cache_dtype if act_rounding else None)
    shape = (num_blocks, block_size, cfg.n_kv_heads, cfg.head_dim)
    rk = [np.zeros(shape, np.float32) for _ in range(cfg.n_layers)]
    rv = [np.zeros(shape, np.float32) for _ in range(cfg.n_layers)]
    return model, kv, bm, ref, rk, rv


def max_err(got, want):
    return float(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)).max())


def check_caches(kv, rk, rv):
    """Caches vs the oracle's: a few 16-bit ulps of the largest entry for fp16 /
    bf16 (layer-0 rounding differences propagate into the later layers' k/v),
    the fp32 bar of 1e-4 relative for fp32 (summation order differs from numpy's)."""
    rel = {torch.float32: 1e-4, torch.float16: 4e-3, torch.bfloat16: 2e-2}[kv.dtype]
    for layer, (k, v) in enumerate(zip(rk, rv)):
        for got, want in ((kv.k_cache[layer], k), (kv.v_cache[layer], v)):
            bound = rel * max(1.0, float(np.abs(want).max()))
            assert max_err(got.float().cpu().numpy(), want) < bound, layer


# fp16 / bf16 logits within 2e-2 of the float32 oracle (the 16-bit bar); fp32
# models (the reference's default dtype, weights.py:32) within 1e-4
LOGIT_TOL = {"float16": TOL, "bfloat16": TOL, "float32": 1e-4}
# bf16 models against the oracle that rounds their stored activations to bf16
# too (act_rounding): the two still round at different points and sum in
# different orders, and with 8 significant bits one bf16 step of a logit-sized
# value (|logit| <= 3 in these models) is 1.6e-2 -- a fixed absolute bound
BF16_MODEL_TOL = 3e-2


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_prefill_matches_oracle(dtype):
    cfg = small_config(dtype=dtype)
    model, kv, bm, ref, rk, rv = build(cfg)
    rng = np.random.default_rng(20)
    for sid, n in enumerate([5, 17, 33]):
        bm.register_sequence(sid)
        toks = rng.integers(0, cfg.vocab_size, n)
        logits = model.prefill(toks, kv, bm, sid)[0].cpu().numpy()
        want = ref.prefill(toks, rk, rv, np.array(bm.get_block_table(sid)), 0, 16)
        assert max_err(logits, want) < LOGIT_TOL[dtype], sid
        assert bm.get_context_length(sid) == n
    check_caches(kv, rk, rv)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("dim,heads", [(128, 4), (256, 4)])
def test_chunked_prefill_attends_to_prefix(dtype, dim, heads):
    """attend_prefix=True (no reference counterpart: the reference's chunk at
    start_pos > 0 ignores the cached prefix, llama.py:184): a prompt prefilled
    in chunks of 37, 50 and 5 rows gives each chunk the logits of one prefill of
    the whole prompt (oracle); the default still attends within the chunk only.
    16-bit models at head_dim 64 read the prefix through the block table on
    MFMA (tv_flash_prefill_paged); head_dim 32 and fp32 models take one paged
    decode query per row."""
    cfg = small_config(dim=dim, n_heads=heads, dtype=dtype)
    bf16 = dtype == "bfloat16"           # the oracle stores activations in bf16 where the model does
    model, kv, bm, ref, rk, rv = build(cfg, seed=8, act_rounding=bf16)
    rng = np.random.default_rng(25)
    chunks = [rng.integers(0, cfg.vocab_size, n) for n in (37, 50, 5)]
    bm.register_sequence(0)
    model.prefill(chunks[0], kv, bm, 0, logits=None)
    got = [model.prefill(chunks[1], kv, bm, 0, 37, attend_prefix=True)[0].cpu().numpy(),
           model.prefill(chunks[2], kv, bm, 0, 87, attend_prefix=True)[0].cpu().numpy()]
    table = np.array(bm.get_block_table(0))
    full = ref.prefill(np.concatenate(chunks), rk, rv, table, 0, 16)
    tol = BF16_MODEL_TOL if bf16 else LOGIT_TOL[dtype]
    assert max_err(got[0], full[37:87]) < tol
    assert max_err(got[1], full[87:]) < tol
    # the reference's behaviour (chunk only) is unchanged by default
    model2, kv2, bm2, ref2, rk2, rv2 = build(cfg, seed=8, act_rounding=bf16)
    bm2.register_sequence(0)
    model2.prefill(chunks[0], kv2, bm2, 0, logits=None)
    ref2.prefill(chunks[0], rk2, rv2, np.array(bm2.get_block_table(0)), 0, 16)
    own = model2.prefill(chunks[1], kv2, bm2, 0, 37)[0].cpu().numpy()
    want = ref2.prefill(chunks[1], rk2, rv2, np.array(bm2.get_block_table(0)), 37, 16)
    assert max_err(own, want) < tol


def prefill_batch(model, kv, bm, ref, rk, rv, lens, rng, cfg):
    """Prefill each sequence on both sides; returns the oracle's next tokens."""
    nxt = []
    for sid, n in enumerate(lens):
        bm.register_sequence(sid)
        toks = rng.integers(0, cfg.vocab_size, n)
        model.prefill(toks, kv, bm, sid, logits=None)
        want = ref.prefill(toks, rk, rv, np.array(bm.get_block_table(sid)), 0, kv.block_size)
        nxt.append(int(greedy_ref(want[-1])))
    return nxt


# (dim, n_heads, n_kv_heads): head_dim 32 takes the unfused path (qkv_rope +
# tv_paged_decode); head_dim 64 / 128 the fused MFMA step attention, with
# 2, 8 and 16 query heads per KV head
DECODE_SHAPES = [(128, 4, 2), (256, 4, 2), (512, 8, 1), (1024, 16, 1), (256, 2, 1)]


@pytest.mark.parametrize("dtype", ["float16", "float32"])
@pytest.mark.parametrize("shape", DECODE_SHAPES, ids=lambda s: f"dim{s[0]}-h{s[1]}-kv{s[2]}")
@pytest.mark.parametrize("write_before_attend", [True, False])
def test_decode_steps_match_oracle(write_before_attend, shape, dtype):
    """Engine convention (context = position + 1, engine.py:251) over several steps,
    teacher-forced with the oracle's greedy tokens; one context spans every wave
    of the fused kernel (16-bit models; fp32 models take qkv_rope +
    tv_paged_decode)."""
    dim, nh, nkv = shape
    cfg = small_config(dim=dim, n_heads=nh, n_kv_heads=nkv, max_seq_len=512, dtype=dtype)
    model, kv, bm, ref, rk, rv = build(cfg, seed=3, write_before_attend=write_before_attend)
    rng = np.random.default_rng(21)
    lens = [7, 16, 300, 1]
    toks = prefill_batch(model, kv, bm, ref, rk, rv, lens, rng, cfg)
    jit = model.create_jit_decode(16)
    max_blocks = 20
    for step in range(4):
        pos = [bm.seq_positions[s] for s in range(len(lens))]
        for s, p in enumerate(pos):
            bm.ensure_block_for_position(s, p)
        bt = np.zeros((len(lens), max_blocks), np.int32)
        for s in range(len(lens)):
            t = bm.get_block_table(s)
            bt[s, :len(t)] = t
        ctx = [p + 1 for p in pos]
        logits = model.decode(torch.tensor(toks).reshape(-1, 1), kv, bm, list(range(len(lens))), pos,
                              torch.from_numpy(bt), torch.tensor(ctx, dtype=torch.int32), jit, max_blocks)
        want = ref.decode(toks, pos, ctx, bt, rk, rv, 16, write_before_attend=write_before_attend)
        assert logits.shape == (len(lens), 1, cfg.vocab_size)
        assert max_err(logits[:, 0].cpu().numpy(), want) < LOGIT_TOL[dtype], step
        toks = [int(t) for t in greedy_ref(want)]
    check_caches(kv, rk, rv)


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_graph_replay_is_deterministic_and_equals_eager(dtype):
    from tinyvllm_amd.llama import DecodeGraph
    cfg = small_config(n_layers=3, dtype=dtype)
    model, kv, bm, ref, rk, rv = build(cfg, seed=5)
    rng = np.random.default_rng(22)
    toks = prefill_batch(model, kv, bm, ref, rk, rv, [9, 12, 20], rng, cfg)
    pos = [9, 12, 20]
    bt = np.zeros((3, 4), np.int32)
    for s in range(3):
        bm.ensure_block_for_position(s, pos[s])
        t = bm.get_block_table(s)
        bt[s, :len(t)] = t
    g = DecodeGraph(model, kv, 3, 4)
    outs = []
    for mode in ("eager", "graph", "graph"):
        g.set_inputs(toks, pos, [p + 1 for p in pos], bt)
        if mode == "eager":
            g.step_eager()
        else:
            g.step()
        torch.cuda.synchronize()
        outs.append((g.logits.clone(), g.tokens.clone(), g.positions.clone(), g.context_lens.clone()))
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            assert torch.equal(a, b)
    assert outs[0][2].tolist() == [p + 1 for p in pos] and outs[0][3].tolist() == [p + 2 for p in pos]
    assert outs[0][1].tolist() == np.argmax(outs[0][0].cpu().numpy(), axis=1).tolist()


def test_device_loop_matches_host_stepping():
    """run(n) with sampling, position advance and history on the device equals n
    steps fed from the host."""
    from tinyvllm_amd.llama import DecodeGraph
    cfg = small_config()
    model, kv, bm, ref, rk, rv = build(cfg, seed=6, num_blocks=32)
    rng = np.random.default_rng(23)
    lens = [4, 11]
    toks = prefill_batch(model, kv, bm, ref, rk, rv, lens, rng, cfg)
    steps = 6
    bt = np.zeros((2, 4), np.int32)
    for s in range(2):
        bm.ensure_block_for_position(s, lens[s] + steps)
        t = bm.get_block_table(s)
        bt[s, :len(t)] = t
    snapshot = [(k.clone(), v.clone()) for k, v in zip(kv.k_cache, kv.v_cache)]
    g = DecodeGraph(model, kv, 2, 4, history_len=32)
    g.set_inputs(toks, lens, [n + 1 for n in lens], bt)
    g.run(steps)
    torch.cuda.synchronize()
    hist = g.history.cpu().numpy()
    dev_tokens = [hist[s, lens[s] + 1:lens[s] + 1 + steps].tolist() for s in range(2)]
    for (k, v), (k0, v0) in zip(zip(kv.k_cache, kv.v_cache), snapshot):
        k.copy_(k0)
        v.copy_(v0)
    h = DecodeGraph(model, kv, 2, 4)
    cur = list(toks)
    host_tokens = [[], []]
    for i in range(steps):
        h.set_inputs(cur, [n + i for n in lens], [n + i + 1 for n in lens], bt)
        h.step()
        cur = h.tokens.cpu().tolist()
        for s in range(2):
            host_tokens[s].append(cur[s])
    assert dev_tokens == host_tokens
    assert g.positions.cpu().tolist() == [n + steps for n in lens]


def test_tinyllama_shape_matches_oracle():
    """TinyLlama-1.1B architecture (22 layers, dim 2048, 32/4 heads, MLP 5632,
    vocab 32000), random N(0, 0.02) fp16 weights: prefill + 2 decode steps."""
    from tinyvllm_amd.llama import LlamaConfig
    cfg = LlamaConfig.tinyllama_1b()
    model, kv, bm, ref, rk, rv = build(cfg, seed=7, std=0.02, num_blocks=16)
    rng = np.random.default_rng(24)
    lens = [8, 13, 16]
    nxt = []
    for sid, n in enumerate(lens):
        bm.register_sequence(sid)
        toks = rng.integers(0, cfg.vocab_size, n)
        logits = model.prefill(toks, kv, bm, sid, logits="last")[0, 0].cpu().numpy()
        want = ref.prefill(toks, rk, rv, np.array(bm.get_block_table(sid)), 0, 16)[-1]
        assert max_err(logits, want) < TOL, sid
        nxt.append(int(greedy_ref(want)))
    jit = model.create_jit_decode(16)
    for step in range(2):
        pos = [bm.seq_positions[s] for s in range(3)]
        bt = np.zeros((3, 2), np.int32)
        for s in range(3):
            bm.ensure_block_for_position(s, pos[s])
            t = bm.get_block_table(s)
            bt[s, :len(t)] = t
        ctx = [p + 1 for p in pos]
        logits = model.decode(torch.tensor(nxt).reshape(-1, 1), kv, bm, [0, 1, 2], pos, torch.from_numpy(bt),
                              torch.tensor(ctx, dtype=torch.int32), jit, 2)
        want = ref.decode(nxt, pos, ctx, bt, rk, rv, 16)
        err = max_err(logits[:, 0].cpu().numpy(), want)
        assert err < TOL, (step, err)
        top2 = np.sort(want, axis=1)[:, -2:]
        clear = top2[:, 1] - top2[:, 0] > 2 * TOL
        got_tok = logits[:, 0].cpu().numpy().argmax(1)
        assert np.array_equal(got_tok[clear], greedy_ref(want)[clear])
        nxt = [int(t) for t in greedy_ref(want)]


def engine_tables(bm, seq_ids, width):
    """LLMEngine._prepare_batch_tensors (engine.py:235-255): each sequence's
    current table, zero padded -- built before get_slot allocates."""
    bt = np.zeros((len(seq_ids), width), np.int32)
    for i, s in enumerate(seq_ids):
        t = bm.get_block_table(s)[:width]
        bt[i, :len(t)] = t
    return bt


@pytest.mark.parametrize("write_before_attend", [True, False])
def test_decode_allocates_the_new_block_like_get_slot(write_before_attend):
    """Driven the engine's way: tables from get_block_table with no allocation,
    context = position + 1 (engine.py:152-153, 235-255).  Prompts of 16 and 32
    tokens start their first decode position in a block the table does not list
    yet; Llama.decode must allocate it through get_slot (llama.py:381-386) and
    write the token's K/V there.  Block 0 -- the last one LIFO allocation hands
    out, so no sequence owns it here -- stays untouched, the logits and caches
    match the oracle given the table after the allocation, and the tables grow
    by one block per 16 positions.  (In the reference order the attended row of
    the new position is unwritten -- zero in a fresh cache -- as in the
    reference, quirk Q4.)"""
    cfg = small_config()
    model, kv, bm, ref, rk, rv = build(cfg, seed=9, num_blocks=24, write_before_attend=write_before_attend)
    rng = np.random.default_rng(26)
    lens = [16, 5, 32]
    toks = prefill_batch(model, kv, bm, ref, rk, rv, lens, rng, cfg)
    jit = model.create_jit_decode(16)
    max_blocks = 8
    seqs = [0, 1, 2]
    for step in range(18):
        pos = [bm.get_context_length(s) for s in seqs]
        before = [len(bm.get_block_table(s)) for s in seqs]
        bt = engine_tables(bm, seqs, max_blocks)
        ctx = [p + 1 for p in pos]
        logits = model.decode(torch.tensor(toks).reshape(-1, 1), kv, bm, seqs, pos, torch.from_numpy(bt),
                              torch.tensor(ctx, dtype=torch.int32), jit, max_blocks)
        after = [len(bm.get_block_table(s)) for s in seqs]
        assert after == [b + (p % 16 == 0 and p // 16 == b) for b, p in zip(before, pos)], step
        full = engine_tables(bm, seqs, max_blocks)
        want = ref.decode(toks, pos, ctx, full, rk, rv, 16, write_before_attend=write_before_attend)
        err = max_err(logits[:, 0].cpu().numpy(), want)
        assert err < TOL, (step, err)
        assert [bm.get_context_length(s) for s in seqs] == [p + 1 for p in pos]
        toks = [int(t) for t in greedy_ref(want)]
    assert all(0 not in bm.get_block_table(s) for s in seqs)
    for k, v in zip(kv.k_cache, kv.v_cache):
        assert not k[0].any() and not v[0].any()
    check_caches(kv, rk, rv)


def test_decode_bad_position_allocates_nothing():
    """A start position that is not the block manager's raises before any
    sequence of the batch allocates: sequence 0 sits on a block boundary (its
    get_slot would allocate), sequence 1's position is wrong."""
    cfg = small_config()
    model, kv, bm, ref, rk, rv = build(cfg, seed=11, num_blocks=16)
    rng = np.random.default_rng(28)
    toks = prefill_batch(model, kv, bm, ref, rk, rv, [16, 7], rng, cfg)
    jit = model.create_jit_decode(16)
    before = [list(bm.get_block_table(s)) for s in (0, 1)]
    free_before = bm.get_num_free_blocks()
    pos = [bm.get_context_length(0), bm.get_context_length(1) + 1]
    bt = engine_tables(bm, [0, 1], 4)
    with pytest.raises(ValueError, match="start position"):
        model.decode(torch.tensor(toks).reshape(-1, 1), kv, bm, [0, 1], pos, torch.from_numpy(bt),
                     torch.tensor([p + 1 for p in pos], dtype=torch.int32), jit, 4)
    assert [list(bm.get_block_table(s)) for s in (0, 1)] == before
    assert bm.get_num_free_blocks() == free_before
    assert [bm.get_context_length(s) for s in (0, 1)] == [16, 7]


def test_decode_past_the_table_width_writes_kv_and_truncates_attention():
    """Quirk Q5 (engine.py:81, llama.py:368-374): a position past max_blocks
    columns is still written to its block (get_slot, llama.py:382) while
    attention covers only the first max_blocks * block_size tokens."""
    cfg = small_config()
    model, kv, bm, ref, rk, rv = build(cfg, seed=10, num_blocks=16)
    rng = np.random.default_rng(27)
    lens = [40, 20]
    toks = prefill_batch(model, kv, bm, ref, rk, rv, lens, rng, cfg)
    jit = model.create_jit_decode(16)
    max_blocks = 2
    for step in range(2):
        pos = [bm.get_context_length(s) for s in (0, 1)]
        bt = engine_tables(bm, [0, 1], 3)
        ctx = [p + 1 for p in pos]
        logits = model.decode(torch.tensor(toks).reshape(-1, 1), kv, bm, [0, 1], pos, torch.from_numpy(bt),
                              torch.tensor(ctx, dtype=torch.int32), jit, max_blocks)
        full = engine_tables(bm, [0, 1], 3)
        want = ref.decode(toks, pos, ctx, full, rk, rv, 16, max_blocks=max_blocks)
        err = max_err(logits[:, 0].cpu().numpy(), want)
        assert err < TOL, (step, err)
        toks = [int(t) for t in greedy_ref(want)]
    check_caches(kv, rk, rv)
    slot = bm.get_block_table(0)[41 // 16] * 16 + 41 % 16
    assert kv.k_cache[1].reshape(-1, cfg.n_kv_heads * cfg.head_dim)[slot].abs().sum() > 0


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("block_size", [4, 32])
@pytest.mark.parametrize("ctx_convention", ["cached", "engine"])
def test_decode_block_sizes_match_oracle(ctx_convention, block_size, dtype):
    """Restates test_multiple_blocks_context (tests/test_jit_decode.py:259-294:
    block_size 4, contexts spanning several blocks) for 16-bit models at block
    sizes 4 (not a multiple of 16: the unfused RoPE + K/V write and the VALU
    paged decode) and 32 (the fused step attention), with the reference test's
    context (= tokens cached, ctx = position) and the engine's (position + 1)."""
    cfg = small_config(dim=256, n_heads=4, n_kv_heads=2, max_seq_len=256, dtype=dtype)
    model, kv, bm, ref, rk, rv = build(cfg, seed=12, num_blocks=128, block_size=block_size)
    rng = np.random.default_rng(28)
    lens = [10, 33, 90]
    toks = prefill_batch(model, kv, bm, ref, rk, rv, lens, rng, cfg)
    jit = model.create_jit_decode(block_size)
    max_blocks = -(-(max(lens) + 8) // block_size)
    seqs = [0, 1, 2]
    for step in range(4):
        pos = [bm.get_context_length(s) for s in seqs]
        for s, p in zip(seqs, pos):                       # _setup_seq pre-allocates (test_jit_decode.py:268)
            bm.ensure_block_for_position(s, p)
        bt = engine_tables(bm, seqs, max_blocks)
        ctx = pos if ctx_convention == "cached" else [p + 1 for p in pos]
        logits = model.decode(torch.tensor(toks).reshape(-1, 1), kv, bm, seqs, pos, torch.from_numpy(bt),
                              torch.tensor(ctx, dtype=torch.int32), jit, max_blocks)
        assert logits.shape == (3, 1, cfg.vocab_size) and not logits.isnan().any()
        want = ref.decode(toks, pos, ctx, bt, rk, rv, block_size)
        err = max_err(logits[:, 0].cpu().numpy(), want)
        # A bf16 model stores its activations (normalised x, q/k/v, attention
        # output, SwiGLU output) with 8 significant bits, which moves logits by
        # about 1% of their scale on its own: bf16 logits are held to 2e-2 of
        # the logit scale, fp16 logits to 2e-2 absolute.
        tol = TOL * max(1.0, float(np.abs(want).max())) if dtype == "bfloat16" else TOL
        assert err < tol, (step, err, tol)
        toks = [int(t) for t in greedy_ref(want)]
    check_caches(kv, rk, rv)


def _random_model_cases(n=None, seed=31):
    n = case_count(6) if n is None else n
    rng = np.random.Generator(np.random.PCG64(case_seed(seed)))
    cases = []
    for i in range(n):
        hd = int(rng.choice([32, 64, 64, 128]))
        nkv = int(rng.choice([1, 2, 4]))
        nh = nkv * int(rng.choice([1, 2, 4, 8, 16]))
        while nh * hd > 1024 and nh > nkv:
            nh //= 2
        hidden = int(rng.choice([64, 96, 160, 256, 352]))
        vocab = int(rng.choice([256, 300, 512, 1000]))
        layers = int(rng.integers(1, 3))
        dtype = ["float16", "bfloat16", "float32"][int(rng.integers(0, 3))]
        bs = int(rng.choice([4, 8, 16, 16, 32]))
        lens = [int(x) for x in rng.integers(1, 150, int(rng.integers(1, 9)))]
        wba = bool(rng.random() < 0.5)
        cases.append((i, hd, nh, nkv, hidden, vocab, layers, dtype, bs, lens, wba))
    return cases


@pytest.mark.parametrize("i,hd,nh,nkv,hidden,vocab,layers,dtype,bs,lens,wba", _random_model_cases())
def test_random_decode_models(i, hd, nh, nkv, hidden, vocab, layers, dtype, bs, lens, wba):
    """Seeded random models (head_dim 32-128, 1-16 query heads per KV head,
    hidden and vocabulary sizes, 1-2 layers, fp16 / bf16 / fp32), block sizes
    4-32, batches of 1-8 prompts of 1-149 tokens and both K/V write orders:
    three teacher-forced decode steps against the oracle's logits and caches
    (engine convention, context = position + 1).  fp32 and fp16 models are held
    to 1e-4 / 2e-2 against the reference's float32 activations; bf16 models to
    3e-2 (absolute) against the oracle that also stores the activations in
    bf16 where the model does (normalised inputs, q / k / v, attention and
    SwiGLU outputs): with 8 significant bits that storage alone moves two-layer
    logits by up to ~2.3% of their scale from float32 activations."""
    cfg = small_config(dim=nh * hd, n_layers=layers, n_heads=nh, n_kv_heads=nkv, vocab_size=vocab,
                       hidden_dim=hidden, max_seq_len=256, dtype=dtype)
    steps = 3
    num_blocks = sum(-(-(n + steps) // bs) for n in lens) + 4
    model, kv, bm, ref, rk, rv = build(cfg, seed=40 + i, write_before_attend=wba, num_blocks=num_blocks,
                                       block_size=bs, act_rounding=dtype == "bfloat16")
    rng = np.random.default_rng(case_seed(50 + i))
    toks = prefill_batch(model, kv, bm, ref, rk, rv, lens, rng, cfg)
    jit = model.create_jit_decode(bs)
    max_blocks = -(-(max(lens) + steps) // bs)
    seqs = list(range(len(lens)))
    for step in range(steps):
        pos = [bm.get_context_length(s) for s in seqs]
        for s, p in zip(seqs, pos):
            bm.ensure_block_for_position(s, p)
        bt = engine_tables(bm, seqs, max_blocks)
        ctx = [p + 1 for p in pos]
        logits = model.decode(torch.tensor(toks).reshape(-1, 1), kv, bm, seqs, pos, torch.from_numpy(bt),
                              torch.tensor(ctx, dtype=torch.int32), jit, max_blocks)
        want = ref.decode(toks, pos, ctx, bt, rk, rv, bs, write_before_attend=wba)
        err = max_err(logits[:, 0].cpu().numpy(), want)
        assert err < (BF16_MODEL_TOL if dtype == "bfloat16" else LOGIT_TOL[dtype]), (step, err)
        toks = [int(t) for t in greedy_ref(want)]
    check_caches(kv, rk, rv)


def test_load_weights_sets_found_names_and_keeps_the_rest():
    """Llama.load_weights follows llama.py:390-401: names are mapped (Meta, HF and
    the fallback rewrites), names the model lacks are ignored, and weights the
    dict does not hold keep their values.  The fused layouts (wq|wk|wv, the
    interleaved w1/w3) receive the parts in place; a wrong shape raises."""
    from tinyvllm_amd.llama import Llama, random_weights
    cfg = small_config()
    src = random_weights(cfg, seed=3)
    part = {"layers.0.feed_forward.w1.weight": src["layers.0.feed_forward.w1.weight"],
            "model.layers.1.self_attn.k_proj.weight": src["layers.1.attention.wk.weight"],
            "model.layers.1.mlp.up_proj.weight": src["layers.1.feed_forward.w3.weight"],
            "lm_head.weight": src["output.weight"],
            "model.layers.0.post_attention_layernorm.weight": src["layers.0.ffn_norm.weight"] * 2,
            "model.rotary_emb.inv_freq": torch.zeros(7)}
    expected = random_weights(cfg, seed=11)
    expected.update({"layers.0.feed_forward.w1.weight": src["layers.0.feed_forward.w1.weight"],
                     "layers.1.attention.wk.weight": src["layers.1.attention.wk.weight"],
                     "layers.1.feed_forward.w3.weight": src["layers.1.feed_forward.w3.weight"],
                     "output.weight": src["output.weight"],
                     "layers.0.ffn_norm.weight": src["layers.0.ffn_norm.weight"] * 2})
    want = Llama(cfg, expected)
    for model in (Llama(cfg, seed=11), Llama(cfg, part, seed=11)):
        model.load_weights(part)
        for a, b in zip([model.tok_embeddings, model.output, model.norm, *model.wqkv, *model.wo, *model.w13,
                         *model.w2, *model.attention_norm, *model.ffn_norm],
                        [want.tok_embeddings, want.output, want.norm, *want.wqkv, *want.wo, *want.w13,
                         *want.w2, *want.attention_norm, *want.ffn_norm]):
            assert torch.equal(a, b)
    with pytest.raises(ValueError):
        want.load_weights({"output.weight": torch.zeros(3, 3)})


def test_prefill_abi_rejects_a_table_short_of_the_prompt():
    """tv_llama_prefill checks, before any launch, that the block table covers
    positions 0 .. start_pos + n - 1 (Llama.prefill_table checks it in Python;
    a raw C caller gets TV_EINVAL instead of a read past the table)."""
    import ctypes
    from tinyvllm_amd import _lib
    from tinyvllm_amd.llama import _PrefillArgs
    cfg = small_config()
    model, kv, *_ = build(cfg, seed=8)
    lib = _lib.load()
    n = 20
    toks = torch.zeros(n, dtype=torch.int32, device="cuda")
    table = torch.zeros(1, dtype=torch.int32, device="cuda")       # one block of 16 positions
    need = lib.tv_llama_prefill_workspace_bytes(ctypes.byref(model._model), n)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    cache, keep = model.cache_struct(kv)
    for start, attend in ((0, 0), (10, 1)):
        args = _PrefillArgs(n, toks.data_ptr(), start, table.data_ptr(), table.numel(), None, 0, None,
                            ws.data_ptr(), ws.numel(), attend)
        rc = lib.tv_llama_prefill(ctypes.byref(model._model), ctypes.byref(cache), ctypes.byref(args),
                                  _lib.stream_ptr(model.device))
        assert rc == _lib.TV_EINVAL
        assert b"block table covers 16 positions" in lib.tv_last_error()
    del keep
