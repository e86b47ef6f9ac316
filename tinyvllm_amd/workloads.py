"""Seeded synthetic workloads for the attention path (shapes of the benchmark configs).

Integer structure (context lengths, shuffled block pools, block tables, slot
mappings) always comes from numpy PCG64 with a fixed seed, so it is identical
on every machine.  Float data is N(0, 1): generated with numpy (and copied to
the device) when small enough for a CPU check of every element, otherwise
generated on the device with a seeded torch generator.
"""

from dataclasses import dataclass, field

import numpy as np
import torch

HOST_GEN_LIMIT = 64 << 20   # elements; above this float data is generated on the device


@dataclass
class DecodeWorkload:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    context_lens: np.ndarray          # [B] int32
    block_tables: np.ndarray          # [B, MB] int32, zero padded
    num_blocks: int
    dtype: torch.dtype
    seed: int
    q: torch.Tensor = None            # [B,1,Hq,D]
    k_cache: torch.Tensor = None      # [NB,bs,Hkv,D]
    v_cache: torch.Tensor = None
    bt_dev: torch.Tensor = None
    ctx_dev: torch.Tensor = None
    host: dict = field(default_factory=dict)   # numpy copies of q/k/v when generated on the host

    @property
    def batch(self):
        return int(self.context_lens.shape[0])

    def kv_bytes(self):
        """Algorithmic K+V bytes: every attended position once, per KV head."""
        es = torch.tensor([], dtype=self.dtype).element_size()
        return int(self.context_lens.astype(np.int64).sum()) * self.num_kv_heads * self.head_dim * 2 * es

    def algorithmic_bytes(self, out_elem=None):
        """K/V + q + out + block-table entries used + context lengths."""
        es = torch.tensor([], dtype=self.dtype).element_size()
        oe = es if out_elem is None else out_elem
        b = self.batch
        blocks = int(((self.context_lens.astype(np.int64) + self.block_size - 1) // self.block_size).sum())
        return (self.kv_bytes() + b * self.num_heads * self.head_dim * (es + oe) + blocks * 4 + b * 4)

    def flops(self):
        return 4 * int(self.context_lens.astype(np.int64).sum()) * self.num_heads * self.head_dim


def _tables_from_pool(rng, context_lens, block_size, pool, max_blocks):
    need = (context_lens.astype(np.int64) + block_size - 1) // block_size
    if need.sum() > pool:
        raise ValueError("block pool too small")
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.zeros((len(context_lens), max_blocks), dtype=np.int32)
    cur = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[cur:cur + n]
        cur += n
    return bt


def _normal(shape, dtype, device, seed, stream_id, host_ok):
    n = int(np.prod(shape))
    if host_ok and n <= HOST_GEN_LIMIT:
        rng = np.random.Generator(np.random.PCG64([seed, stream_id]))
        arr = rng.standard_normal(shape, dtype=np.float32)
        t = torch.from_numpy(arr).to(dtype)
        return t.to(device), t.float().numpy()
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 1000 + stream_id)
    t = torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(dtype)
    return t, None


def make_decode(name, context_lens, num_heads, num_kv_heads, head_dim, block_size, dtype,
                pool=None, pool_factor=1.1, max_blocks=None, seed=0, device="cuda", host_ok=True,
                rng=None):
    """Build a paged-decode workload; tables come from a shuffled pool of blocks."""
    rng = rng if rng is not None else np.random.Generator(np.random.PCG64(seed))
    context_lens = np.asarray(context_lens, dtype=np.int32)
    need = (context_lens.astype(np.int64) + block_size - 1) // block_size
    if pool is None:
        pool = int(np.ceil(pool_factor * need.sum()))
    if max_blocks is None:
        max_blocks = int(need.max())
    bt = _tables_from_pool(rng, context_lens, block_size, pool, max_blocks)
    wl = DecodeWorkload(name, num_heads, num_kv_heads, head_dim, block_size, context_lens, bt, pool, dtype, seed)
    b = len(context_lens)
    wl.q, hq = _normal((b, 1, num_heads, head_dim), dtype, device, seed, 1, host_ok)
    wl.k_cache, hk = _normal((pool, block_size, num_kv_heads, head_dim), dtype, device, seed, 2, host_ok)
    wl.v_cache, hv = _normal((pool, block_size, num_kv_heads, head_dim), dtype, device, seed, 3, host_ok)
    if hq is not None and hk is not None:
        wl.host = {"q": hq, "k_cache": hk, "v_cache": hv}
    wl.bt_dev = torch.from_numpy(bt).to(device)
    wl.ctx_dev = torch.from_numpy(context_lens).to(device)
    return wl


# ---- the benchmark configurations ---------------------------------------------

def decode_tinyllama_f32_b4(device="cuda", seed=0):
    """Paged decode, TinyLlama layer shape, fp32, B=4, ctx {17,64,128,250}, 64-block pool."""
    return make_decode("decode_tinyllama_f32_b4", [17, 64, 128, 250], 32, 4, 64, 16, torch.float32,
                       pool=64, seed=seed, device=device)


def decode_llama3_8b_b256(device="cuda", seed=0, batch=256, host_ok=False):
    """Paged decode, Llama-3-8B head shape, fp16, B=256, ctx ~ U[512, 4096], pool +10%."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ctx = rng.integers(512, 4097, batch).astype(np.int32)
    return make_decode("decode_llama3_8b_f16_b256", ctx, 32, 8, 128, 16, torch.float16,
                       max_blocks=4096 // 16, seed=seed, device=device, host_ok=host_ok, rng=rng)


def decode_long_bf16_b16(device="cuda", seed=0, batch=16, context=32768, host_ok=False):
    """Split-context paged decode, Llama-3-8B head shape, bf16, B=16 x ctx 32768."""
    return make_decode("decode_long_bf16_b16_32k", [context] * batch, 32, 8, 128, 16, torch.bfloat16,
                       max_blocks=context // 16, seed=seed, device=device, host_ok=host_ok)


@dataclass
class PrefillWorkload:
    name: str
    lengths: list
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    seed: int
    q: list = field(default_factory=list)      # per prompt [1, L, Hq, D]
    k: list = field(default_factory=list)      # per prompt [1, L, Hkv, D]
    v: list = field(default_factory=list)
    slots: list = field(default_factory=list)  # per prompt int32 numpy [L]
    slots_dev: list = field(default_factory=list)
    num_blocks: int = 0
    host: dict = field(default_factory=dict)

    def flops(self, causal=True):
        """Causal: 4*Hq*D per unmasked (query, key) pair = 2*Hq*D*L*(L+1) per prompt."""
        tot = 0
        for length in self.lengths:
            pairs = length * (length + 1) // 2 if causal else length * length
            tot += 4 * self.num_heads * self.head_dim * pairs
        return tot

    def io_bytes(self):
        es = torch.tensor([], dtype=self.dtype).element_size()
        return sum(l * (2 * self.num_heads + 2 * self.num_kv_heads) * self.head_dim * es for l in self.lengths)

    def kv_write_bytes(self):
        es = torch.tensor([], dtype=self.dtype).element_size()
        t = sum(self.lengths)
        return 2 * t * self.num_kv_heads * self.head_dim * es * 2 + t * 4


def prefill_tinyllama_l512_l1024(device="cuda", seed=0, lengths=(512, 1024), spare_blocks=8):
    """Causal prefill + KV write, TinyLlama shape, fp16, prompts of 512 and 1024 tokens."""
    rng = np.random.Generator(np.random.PCG64(seed))
    bs = 16
    need = [(l + bs - 1) // bs for l in lengths]
    pool = sum(need) + spare_blocks
    perm = rng.permutation(pool).astype(np.int64)
    wl = PrefillWorkload("prefill_tinyllama_f16", list(lengths), 32, 4, 64, bs, torch.float16, seed)
    wl.num_blocks = pool
    cur = 0
    for i, (length, n) in enumerate(zip(lengths, need)):
        table = perm[cur:cur + n]
        cur += n
        pos = np.arange(length)
        wl.slots.append((table[pos // bs] * bs + pos % bs).astype(np.int32))
        wl.slots_dev.append(torch.from_numpy(wl.slots[-1]).to(device))
        q, hq = _normal((1, length, 32, 64), torch.float16, device, seed, 10 + 3 * i, True)
        k, hk = _normal((1, length, 4, 64), torch.float16, device, seed, 11 + 3 * i, True)
        v, hv = _normal((1, length, 4, 64), torch.float16, device, seed, 12 + 3 * i, True)
        wl.q.append(q)
        wl.k.append(k)
        wl.v.append(v)
        wl.host[i] = (hq, hk, hv)
    return wl


class E2EWorkload:
    """Batched greedy decode of a random-init LLaMA model over a prefilled paged cache."""

    def __init__(self, model, kv_cache, tables, prompts, decode_steps, seed):
        self.model = model
        self.kv = kv_cache
        self.tables = tables                  # [B, blocks per sequence] int32, covers prompt + decode
        self.prompts = prompts                # [B, L] int32
        self.batch, self.prompt_len = prompts.shape
        self.decode_steps = decode_steps
        self.seed = seed

    def weight_bytes_per_step(self):
        """Weights read by one step: everything but the embedding table, of which only B rows are read."""
        m = self.model
        emb = m.tok_embeddings
        return m.weight_bytes() - emb.numel() * emb.element_size() + self.batch * emb.shape[1] * emb.element_size()

    def kv_bytes(self, ctx):
        """K and V rows attended by one step at context ctx per sequence, all layers (+ the write)."""
        c = self.model.config
        row = c.n_kv_heads * c.head_dim * self.kv.k_cache[0].element_size()
        return self.batch * c.n_layers * 2 * row * (ctx + 1)

    def bytes_for_steps(self, first_ctx, steps):
        return sum(self.weight_bytes_per_step() + self.kv_bytes(first_ctx + i) for i in range(steps))


def e2e_tinyllama_b64(device="cuda", seed=0, batch=64, prompt_len=1024, decode_steps=128, block_size=16,
                          pool_margin=0.1):
    """Random-init TinyLlama-1.1B (fp16 weights ~ N(0, 0.02), unit norms), ``batch``
    prompts of ``prompt_len`` seeded token ids, blocks for prompt + decode drawn from
    a shuffled pool sized to the need + 10%."""
    from .kv_cache import KVCache
    from .llama import Llama, LlamaConfig
    cfg = LlamaConfig.tinyllama_1b("float16")
    model = Llama(cfg, seed=seed, device=device)
    rng = np.random.Generator(np.random.PCG64(seed))
    per_seq = -(-(prompt_len + decode_steps) // block_size)
    num_blocks = int(np.ceil((1 + pool_margin) * batch * per_seq))
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = perm[:batch * per_seq].reshape(batch, per_seq)
    prompts = rng.integers(0, cfg.vocab_size, (batch, prompt_len)).astype(np.int32)
    kv = KVCache(cfg.n_layers, num_blocks, block_size, cfg.n_kv_heads, cfg.head_dim, cfg.dtype, device)
    return E2EWorkload(model, kv, tables, prompts, decode_steps, seed)
