"""Pins of the LLaMA oracle (oracle/llama.py) on the CPU.

* RMSNorm: torch.nn.functional.rms_norm (float64) and the reference's own
  RMSNorm tests (test_llama.py:59-101: unit RMS, zero input, scale invariance).
* RoPE: the complex-multiplication form x_c * exp(i p theta_i) (the textbook
  Meta LLaMA statement, computed with torch.polar in float64); position 0 is the
  identity and norms are preserved (test_llama.py:131-186); the table at the
  unit frequency equals cos/sin(p); a half-split (GPT-NeoX) rotation -- the
  plausible mistake -- is rejected.
* The whole forward: an independent float64 torch model (F.rms_norm, torch.polar
  RoPE, F.scaled_dot_product_attention with repeated KV heads, F.silu).
* Caching: prefill + write-before-attend decode reproduce the dense causal
  forward position by position (paged cache in float32, shuffled blocks).
* Reference order (llama.py:378-386): equal to write-before-attend when the
  context excludes the new slot (test_jit_decode.py:102-107), different when it
  includes it, and the cache ends up identical either way.
* Greedy sampling: first maximum on ties (sampling.py:133-134).
* act_dtype (16-bit activation storage, no reference counterpart): the identity
  for float32; for bfloat16 every product input and attention operand is
  exactly representable.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.block_manager import BlockManagerRef
from oracle.llama import LlamaRef, apply_rope_ref, greedy_ref, rms_norm_ref, rope_tables_ref


class Cfg:
    def __init__(self, dim=64, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=96, hidden_dim=96,
                 norm_eps=1e-5, max_seq_len=64, rope_theta=10000.0):
        self.dim, self.n_layers, self.n_heads, self.n_kv_heads = dim, n_layers, n_heads, n_kv_heads
        self.vocab_size, self.hidden_dim, self.norm_eps = vocab_size, hidden_dim, norm_eps
        self.max_seq_len, self.rope_theta = max_seq_len, rope_theta
        self.head_dim = dim // n_heads


def rand_weights(cfg, seed=0, std=0.1, norm_jitter=True):
    rng = np.random.default_rng(seed)
    c, d = cfg, cfg.head_dim
    w = {"tok_embeddings.weight": rng.standard_normal((c.vocab_size, c.dim)).astype(np.float32),
         "norm.weight": (1 + 0.1 * rng.standard_normal(c.dim) * norm_jitter).astype(np.float32),
         "output.weight": (std * rng.standard_normal((c.vocab_size, c.dim))).astype(np.float32)}
    for i in range(c.n_layers):
        p = f"layers.{i}."
        for name, shape in (("attention.wq.weight", (c.n_heads * d, c.dim)),
                            ("attention.wk.weight", (c.n_kv_heads * d, c.dim)),
                            ("attention.wv.weight", (c.n_kv_heads * d, c.dim)),
                            ("attention.wo.weight", (c.dim, c.n_heads * d)),
                            ("feed_forward.w1.weight", (c.hidden_dim, c.dim)),
                            ("feed_forward.w2.weight", (c.dim, c.hidden_dim)),
                            ("feed_forward.w3.weight", (c.hidden_dim, c.dim))):
            w[p + name] = (std * rng.standard_normal(shape)).astype(np.float32)
        for name in ("attention_norm.weight", "ffn_norm.weight"):
            w[p + name] = (1 + 0.1 * rng.standard_normal(c.dim) * norm_jitter).astype(np.float32)
    return w


# ---- RMSNorm -------------------------------------------------------------------------

def test_rms_norm_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 48)).astype(np.float32) * 3
    w = rng.standard_normal(48).astype(np.float32)
    want = F.rms_norm(torch.from_numpy(x).double(), (48,), torch.from_numpy(w).double(), 1e-5).numpy()
    assert np.abs(rms_norm_ref(x, w) - want).max() < 1e-5


def test_rms_norm_reference_cases():
    x = np.random.default_rng(2).standard_normal(32).astype(np.float32)
    out = rms_norm_ref(x, np.ones(32, np.float32))
    assert 0.99 < np.sqrt(np.mean(out ** 2)) < 1.01
    assert np.abs(rms_norm_ref(np.zeros(8, np.float32), np.ones(8, np.float32))).max() < 0.01
    v = np.arange(1, 9, dtype=np.float32)
    assert np.allclose(rms_norm_ref(v, np.ones(8)), rms_norm_ref(2 * v, np.ones(8)), rtol=1e-5)


# ---- RoPE ----------------------------------------------------------------------------

def rope_complex(x, pos, theta=10000.0):
    """x_c * exp(i * pos * theta^(-2i/D)) in float64 (pairs (2i, 2i+1) as complex numbers)."""
    d = x.shape[-1]
    freqs = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = torch.as_tensor(pos, dtype=torch.float64)[:, None] * freqs[None]
    rot = torch.polar(torch.ones_like(ang), ang)[:, None, :]
    xc = torch.view_as_complex(torch.from_numpy(x).double().reshape(*x.shape[:-1], d // 2, 2).contiguous())
    return torch.view_as_real(xc * rot).reshape(x.shape).numpy()


def test_rope_matches_complex_rotation():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 3, 16)).astype(np.float32)
    pos = np.array([0, 1, 5, 17, 100, 1000])
    cos, sin = rope_tables_ref(16, 1024)
    got = apply_rope_ref(x, cos[pos][:, None], sin[pos][:, None])
    assert np.abs(got - rope_complex(x, pos)).max() < 2e-4


def test_rope_rejects_half_split_rotation():
    """A GPT-NeoX style rotation (pairs (i, i + D/2)) differs: the interleave is pinned."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 2, 16)).astype(np.float32)
    pos = np.array([1, 2, 3, 4])
    cos, sin = rope_tables_ref(16, 8)
    c, s = cos[pos][:, None], sin[pos][:, None]
    x0, x1 = x[..., :8], x[..., 8:]
    neox = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], -1)
    assert np.abs(neox - rope_complex(x, pos)).max() > 0.1
    assert np.abs(apply_rope_ref(x, c, s) - rope_complex(x, pos)).max() < 1e-5


def test_rope_position_zero_and_norm():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 1, 8)).astype(np.float32)
    cos, sin = rope_tables_ref(8, 10)
    assert np.array_equal(apply_rope_ref(x[:1], cos[:1][:, None], sin[:1][:, None]), x[:1])
    out = apply_rope_ref(x, cos[:4][:, None], sin[:4][:, None])
    assert np.allclose(np.linalg.norm(out, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


def test_rope_table_unit_frequency():
    cos, sin = rope_tables_ref(64, 4096)
    p = np.arange(4096, dtype=np.float64)
    assert np.abs(cos[:, 0] - np.cos(p)).max() < 1e-6 and np.abs(sin[:, 0] - np.sin(p)).max() < 1e-6
    assert cos.shape == (4096, 32) and np.all(np.abs(cos) <= 1) and np.all(np.abs(sin) <= 1)


def test_greedy_first_maximum():
    assert greedy_ref(np.array([[0.5, 2.0, 2.0, 1.0]]))[0] == 1


# ---- whole model ---------------------------------------------------------------------

def torch_forward(cfg, w, tokens):
    """Independent float64 LLaMA forward (causal, no cache)."""
    t = {k: torch.from_numpy(v).double() for k, v in w.items()}
    d = cfg.head_dim
    x = t["tok_embeddings.weight"][torch.as_tensor(tokens)]
    L = x.shape[0]
    pos = np.arange(L)
    for i in range(cfg.n_layers):
        p = f"layers.{i}."
        xn = F.rms_norm(x, (cfg.dim,), t[p + "attention_norm.weight"], cfg.norm_eps)
        q = (xn @ t[p + "attention.wq.weight"].T).reshape(L, cfg.n_heads, d)
        k = (xn @ t[p + "attention.wk.weight"].T).reshape(L, cfg.n_kv_heads, d)
        v = (xn @ t[p + "attention.wv.weight"].T).reshape(L, cfg.n_kv_heads, d)
        q = torch.from_numpy(rope_complex(q.numpy(), pos))
        k = torch.from_numpy(rope_complex(k.numpy(), pos))
        rep = cfg.n_heads // cfg.n_kv_heads
        k, v = k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)
        a = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                           is_causal=True).transpose(0, 1).reshape(L, -1)
        x = x + a @ t[p + "attention.wo.weight"].T
        hn = F.rms_norm(x, (cfg.dim,), t[p + "ffn_norm.weight"], cfg.norm_eps)
        x = x + (F.silu(hn @ t[p + "feed_forward.w1.weight"].T) * (hn @ t[p + "feed_forward.w3.weight"].T)) \
            @ t[p + "feed_forward.w2.weight"].T
    return (F.rms_norm(x, (cfg.dim,), t["norm.weight"], cfg.norm_eps) @ t["output.weight"].T).numpy()


def test_forward_matches_independent_torch_model():
    cfg = Cfg()
    w = rand_weights(cfg)
    tokens = np.random.default_rng(6).integers(0, cfg.vocab_size, 11)
    got = LlamaRef(cfg, w).forward(tokens)
    want = torch_forward(cfg, w, tokens)
    assert np.abs(got - want).max() < 2e-4 * max(1.0, np.abs(want).max())


def test_forward_planted_mistake_is_caught():
    """Dropping the layer-input residual (a plausible slip) moves the logits far beyond the tolerance."""
    cfg = Cfg(n_layers=1)
    w = rand_weights(cfg)
    tokens = np.arange(6)
    ref = LlamaRef(cfg, w)
    good = ref.forward(tokens)
    orig = ref._finish_layer
    ref._finish_layer = lambda i, x, attn: orig(i, x, attn) - x   # drop h = x + ...
    assert np.abs(ref.forward(tokens) - good).max() > 1e-2


def _cache(cfg, nb, bs):
    shape = (nb, bs, cfg.n_kv_heads, cfg.head_dim)
    return ([np.zeros(shape, np.float32) for _ in range(cfg.n_layers)],
            [np.zeros(shape, np.float32) for _ in range(cfg.n_layers)])


def test_prefill_then_decode_reproduce_forward():
    cfg = Cfg()
    w = rand_weights(cfg, seed=7)
    ref = LlamaRef(cfg, w, cache_dtype=np.float32)
    bs, nb = 4, 24
    kc, vc = _cache(cfg, nb, bs)
    rng = np.random.default_rng(8)
    table = rng.permutation(nb)[:8]                  # shuffled, non-contiguous blocks
    prompt = rng.integers(0, cfg.vocab_size, 7)
    logits = ref.prefill(prompt, kc, vc, table, 0, bs)
    assert np.abs(logits - ref.forward(prompt)).max() < 1e-4
    seq = list(prompt)
    for step in range(5):
        tok = int(greedy_ref(logits[-1:])[0])
        pos = len(seq)
        seq.append(tok)
        logits = ref.decode([tok], [pos], [pos + 1], table[None], kc, vc, bs)
        assert np.abs(logits[0] - ref.forward(seq)[-1]).max() < 1e-4, step


def test_reference_order_semantics():
    cfg = Cfg(n_layers=1)
    w = rand_weights(cfg, seed=9)
    ref = LlamaRef(cfg, w, cache_dtype=np.float32)
    bs, nb = 4, 16
    table = np.random.default_rng(10).permutation(nb)[:6][None]
    prompt = np.arange(9) % cfg.vocab_size
    caches = []
    for _ in range(4):
        kc, vc = _cache(cfg, nb, bs)
        ref.prefill(prompt, kc, vc, table[0], 0, bs)
        caches.append((kc, vc))
    pos = len(prompt)
    # context excludes the new slot: both orders agree
    a = ref.decode([3], [pos], [pos], table, *caches[0], bs, write_before_attend=True)
    b = ref.decode([3], [pos], [pos], table, *caches[1], bs, write_before_attend=False)
    assert np.array_equal(a, b)
    # context includes it (engine.py:251): the reference order reads the unwritten slot
    c = ref.decode([3], [pos], [pos + 1], table, *caches[2], bs, write_before_attend=True)
    d = ref.decode([3], [pos], [pos + 1], table, *caches[3], bs, write_before_attend=False)
    assert np.abs(c - d).max() > 1e-4
    for (k1, v1), (k2, v2) in ((caches[0], caches[1]), (caches[2], caches[3])):
        assert all(np.array_equal(x, y) for x, y in zip(k1 + v1, k2 + v2))


def test_prefill_slots_follow_block_manager():
    """The oracle's prefill places token p at table[p // bs] * bs + p % bs, as the
    reference's per-chunk loop does with BlockManager tables (llama.py:199-209)."""
    cfg = Cfg(n_layers=1)
    ref = LlamaRef(cfg, rand_weights(cfg, seed=11), cache_dtype=np.float32)
    bm = BlockManagerRef(1, 12, 4)
    bm.register_sequence(0)
    for p in range(10):
        bm.ensure_block_for_position(0, p)
    kc, vc = _cache(cfg, 12, 4)
    ref.prefill(np.arange(10), kc, vc, np.array(bm.get_block_table(0)), 0, 4)
    written = np.nonzero(np.abs(kc[0]).reshape(12 * 4, -1).sum(-1))[0]
    table = bm.get_block_table(0)
    assert sorted(written.tolist()) == sorted(table[p // 4] * 4 + p % 4 for p in range(10))


def test_round_bf16_matches_torch():
    """round_bf16 equals torch's float32 -> bfloat16 conversion (round to nearest,
    ties to even) bit for bit, including ties, subnormals and large values; a
    truncating conversion (the plausible mistake) differs."""
    from oracle.llama import round_bf16
    rng = np.random.default_rng(12)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 4096),
                        np.array([0.0, -0.0, 1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, 3e38, 1e-40, -1e-40],
                                 np.float32)]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = round_bf16(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    truncated = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)
    assert not np.array_equal(truncated, want)


def test_act_dtype_rounds_every_product_input():
    """act_dtype (no reference counterpart): float32 storage changes nothing,
    bit for bit; bfloat16 storage makes the input of every product (q / k / v,
    wo, w1 / w3, w2, the output head) and the attention operands exactly
    bfloat16-representable, and moves the logits by a small, non-zero amount."""
    from oracle.llama import round_bf16
    cfg = Cfg()
    w = rand_weights(cfg, seed=9)
    tokens = np.random.default_rng(10).integers(0, cfg.vocab_size, 9)
    plain = LlamaRef(cfg, w).forward(tokens)
    assert np.array_equal(LlamaRef(cfg, w, act_dtype=np.float32).forward(tokens), plain)
    ref = LlamaRef(cfg, w, act_dtype="bfloat16")
    seen = []
    lin = ref._lin

    def checked_lin(x, name):
        seen.append(name)
        assert np.array_equal(round_bf16(x), x), name
        return lin(x, name)

    ref._lin = checked_lin
    qkv = ref._qkv
    ref._qkv = lambda i, x, pos: tuple(t if np.array_equal(round_bf16(t), t) else pytest.fail("q/k/v")
                                       for t in qkv(i, x, pos))
    got = ref.forward(tokens)
    assert len(seen) == 7 * cfg.n_layers + 1
    err = np.abs(got - plain).max() / max(1.0, np.abs(plain).max())
    assert 0 < err < 5e-2


def test_decode_attention_width_truncates_context():
    """max_blocks = m attends to the first m*bs positions (llama.py:368-374 pad /
    truncate; the padded gather of llama.py:120-140): the same logits as a full
    table with the context clipped to m*bs.  The K/V write still goes to the
    block of the token's position."""
    cfg = Cfg(n_layers=1)
    ref = LlamaRef(cfg, rand_weights(cfg, seed=13), cache_dtype=np.float32)
    bs, nb = 4, 16
    table = np.random.default_rng(14).permutation(nb)[:5][None]
    prompt = np.arange(17) % cfg.vocab_size
    runs = []
    for _ in range(2):
        kc, vc = _cache(cfg, nb, bs)
        ref.prefill(prompt, kc, vc, table[0], 0, bs)
        runs.append((kc, vc))
    pos = 17
    a = ref.decode([5], [pos], [pos + 1], table, *runs[0], bs, max_blocks=3)
    b = ref.decode([5], [pos], [3 * bs], table, *runs[1], bs)
    assert np.abs(a - b).max() < 1e-5          # the gathers differ in width: float32 sum order only
    slot = table[0, pos // bs] * bs + pos % bs
    assert np.abs(runs[0][0][0].reshape(nb * bs, -1)[slot]).sum() > 0
    # a wider attention window changes the result (the truncation is real)
    kc, vc = _cache(cfg, nb, bs)
    ref.prefill(prompt, kc, vc, table[0], 0, bs)
    c = ref.decode([5], [pos], [pos + 1], table, kc, vc, bs, max_blocks=5)
    assert np.abs(a - c).max() > 1e-4
