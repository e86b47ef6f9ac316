"""numpy restatement of the reference's LLaMA forward passes (test infrastructure).

Follows tinyvllm/model/llama.py step by step:

* ``rms_norm_ref``      RMSNorm.__call__, llama.py:14-23: x * rsqrt(mean(x^2) + eps) * w
* ``rope_tables_ref``   precompute_freqs_cis, llama.py:26-31 (float32, as tinygrad's .float())
* ``apply_rope_ref``    apply_rope, llama.py:34-55: interleaved pairs (2i, 2i+1)
* ``silu_ref``          Tensor.silu = x * sigmoid(x), used by FeedForward, llama.py:220-221
* ``LlamaRef.prefill``  Llama.prefill + TransformerBlock + Attention, llama.py:147-285:
                        K/V written to the cache, attention over this chunk only (llama.py:184)
* ``LlamaRef.decode``   Llama.create_jit_decode + Llama.decode, llama.py:290-388:
                        ``write_before_attend=False`` is the reference's order (attention
                        first, K/V written at get_slot() afterwards, llama.py:378-386);
                        True writes first (the order of the HIP step's default)
* ``LlamaRef.forward``  the dense causal forward over a whole token list (no cache): what
                        prefill + decode must reproduce position by position
* greedy sampling       sample_tokens with temperature 0 -> argmax, sampling.py:131-134
* ``round_bf16``        storage rounding of a bfloat16 cache (no reference counterpart:
                        the reference has no bfloat16, weights.py:44)
* ``act_dtype``         (LlamaRef option, no reference counterpart) rounds the activations
                        a 16-bit model stores between its kernels -- each product's
                        normalised input, q / k / v after RoPE, the attention output and
                        the SwiGLU output -- through that dtype; unset, every activation
                        stays float32 as in the reference

Arithmetic is float32 (the precision the fp16 / bf16 kernels are held to); the paged cache stores
``cache_dtype`` (float16 by default, as KVCache(dtype=float16), kv_cache.py:25-32).
Weights use the reference's Meta-style names (``layers.{i}.attention.wq.weight``, ...,
llama.py:413-416).
"""

import numpy as np

from .attention import flash_prefill_ref, paged_decode_ref


def rms_norm_ref(x, weight, eps=1e-5):
    """llama.py:21-23."""
    x = np.asarray(x, dtype=np.float32)
    rms = np.float32(1.0) / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + np.float32(eps))
    return (x * rms * np.asarray(weight, dtype=np.float32)).astype(np.float32)


def rope_tables_ref(head_dim, seq_len, theta=10000.0):
    """llama.py:26-31: (cos, sin) of t * theta^(-arange(0, D, 2) / D), each [seq_len, D/2]."""
    expo = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    freqs = np.float32(1.0) / (np.float32(theta) ** expo)
    t = np.arange(seq_len, dtype=np.float32)
    ang = (t[:, None] * freqs[None, :]).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def apply_rope_ref(x, cos, sin):
    """llama.py:34-55 on x [..., H, D] with cos/sin broadcastable to [..., 1, D/2]."""
    x = np.asarray(x, dtype=np.float32)
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out0 = x0 * cos - x1 * sin
    out1 = x0 * sin + x1 * cos
    return np.stack([out0, out1], axis=-1).reshape(x.shape).astype(np.float32)


def round_bf16(x):
    """Round float32 values to the nearest bfloat16 (ties to even), returned as
    float32: the storage rounding of a bfloat16 cache or activation.  NaN is
    not expected here (finite model values only)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def silu_ref(x):
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def greedy_ref(logits):
    """sampling.py:133-134: argmax over the vocabulary (first maximum)."""
    return np.argmax(np.asarray(logits), axis=-1)


class LlamaRef:
    """The reference model's forward passes over numpy float32 weights."""

    def __init__(self, cfg, weights, cache_dtype=np.float16, act_dtype=None):
        """``cache_dtype``: a numpy dtype the cache rows are rounded through, or
        ``"bfloat16"`` (rounded with ``round_bf16``).  ``act_dtype`` (same forms;
        None keeps float32): the storage type of the activations between kernels."""
        self.cfg = cfg
        self.w = {k: np.asarray(v, dtype=np.float32) for k, v in weights.items()}
        self.cache_dtype = cache_dtype
        self.act_dtype = act_dtype
        self.head_dim = cfg.dim // cfg.n_heads
        self.cos, self.sin = rope_tables_ref(self.head_dim, cfg.max_seq_len * 2, cfg.rope_theta)

    def _round(self, x, dtype):
        if dtype is None:
            return np.asarray(x, dtype=np.float32)
        if isinstance(dtype, str) and dtype == "bfloat16":
            return round_bf16(x)
        return np.asarray(x).astype(dtype).astype(np.float32)

    def _act(self, x):
        return self._round(x, self.act_dtype)

    def _lin(self, x, name):
        return (x @ self.w[name].T).astype(np.float32)

    def _qkv(self, i, x, pos):
        """Projections + RoPE of tokens x [T, dim] at positions pos [T] (llama.py:178-182, 315-322)."""
        c, d = self.cfg, self.head_dim
        p = f"layers.{i}."
        xn = self._act(rms_norm_ref(x, self.w[p + "attention_norm.weight"], c.norm_eps))
        q = self._lin(xn, p + "attention.wq.weight").reshape(-1, c.n_heads, d)
        k = self._lin(xn, p + "attention.wk.weight").reshape(-1, c.n_kv_heads, d)
        v = self._lin(xn, p + "attention.wv.weight").reshape(-1, c.n_kv_heads, d)
        cos, sin = self.cos[pos][:, None, :], self.sin[pos][:, None, :]
        return self._act(apply_rope_ref(q, cos, sin)), self._act(apply_rope_ref(k, cos, sin)), self._act(v)

    def _finish_layer(self, i, x, attn):
        """wo, residual, FFN, residual (llama.py:186, 241-244, 334-338)."""
        c = self.cfg
        p = f"layers.{i}."
        h = x + self._lin(self._act(attn.reshape(attn.shape[0], -1)), p + "attention.wo.weight")
        hn = self._act(rms_norm_ref(h, self.w[p + "ffn_norm.weight"], c.norm_eps))
        g = self._act(silu_ref(self._lin(hn, p + "feed_forward.w1.weight")) * self._lin(hn, p + "feed_forward.w3.weight"))
        ff = self._lin(g, p + "feed_forward.w2.weight")
        return (h + ff).astype(np.float32)

    def _logits(self, x):
        return self._lin(self._act(rms_norm_ref(x, self.w["norm.weight"], self.cfg.norm_eps)), "output.weight")

    def _store(self, cache, slot, value, block_size):
        rounded = self._round(value, self.cache_dtype)
        cache.reshape(-1, *cache.shape[2:])[slot] = rounded.astype(cache.dtype)

    def forward(self, tokens):
        """Dense causal forward over tokens [L] from position 0: logits [L, vocab]."""
        tokens = np.asarray(tokens).reshape(-1)
        x = self.w["tok_embeddings.weight"][tokens]
        pos = np.arange(len(tokens))
        for i in range(self.cfg.n_layers):
            q, k, v = self._qkv(i, x, pos)
            attn = flash_prefill_ref(q[None], k[None], v[None], True, acc=np.float32)[0]
            x = self._finish_layer(i, x, attn)
        return self._logits(x)

    def prefill(self, tokens, k_caches, v_caches, block_table, start_pos, block_size):
        """llama.py:264-285 for one sequence; writes the caches in place; logits [L, vocab]."""
        tokens = np.asarray(tokens).reshape(-1)
        x = self.w["tok_embeddings.weight"][tokens]
        pos = start_pos + np.arange(len(tokens))
        slots = np.asarray(block_table)[pos // block_size] * block_size + pos % block_size
        for i in range(self.cfg.n_layers):
            q, k, v = self._qkv(i, x, pos)
            self._store(k_caches[i], slots, k, block_size)
            self._store(v_caches[i], slots, v, block_size)
            attn = flash_prefill_ref(q[None], k[None], v[None], True, acc=np.float32)[0]
            x = self._finish_layer(i, x, attn)
        return self._logits(x)

    def decode(self, tokens, positions, context_lens, block_tables, k_caches, v_caches, block_size,
               write_before_attend=True, max_blocks=None):
        """One batched decode step (llama.py:290-388); writes the caches; logits [B, vocab].

        ``block_tables`` lists every block of each sequence: the K/V of position p
        go to column p // block_size (the block get_slot returns, llama.py:382).
        Attention reads the first ``max_blocks`` columns (all when None), padded
        with block 0 when the table is narrower (llama.py:368-374)."""
        c, d = self.cfg, self.head_dim
        tokens = np.asarray(tokens).reshape(-1)
        positions = np.asarray(positions).reshape(-1)
        block_tables = np.asarray(block_tables)
        attend_tables = block_tables
        if max_blocks is not None:
            attend_tables = np.zeros((block_tables.shape[0], max_blocks), block_tables.dtype)
            n = min(max_blocks, block_tables.shape[1])
            attend_tables[:, :n] = block_tables[:, :n]
        x = self.w["tok_embeddings.weight"][tokens]
        slots = block_tables[np.arange(len(tokens)), positions // block_size] * block_size + positions % block_size
        for i in range(c.n_layers):
            q, k, v = self._qkv(i, x, positions)
            if write_before_attend:
                self._store(k_caches[i], slots, k, block_size)
                self._store(v_caches[i], slots, v, block_size)
            attn = paged_decode_ref(q[:, None], k_caches[i], v_caches[i], attend_tables, context_lens,
                                    c.n_heads, c.n_kv_heads, d, block_size, acc=np.float32)[:, 0]
            if not write_before_attend:
                self._store(k_caches[i], slots, k, block_size)
                self._store(v_caches[i], slots, v, block_size)
            x = self._finish_layer(i, x, attn.astype(np.float32))
        return self._logits(x)


def reference_weight_names(n_layers):
    """The per-model weight names of the reference's Meta-style map (llama.py:398-435)."""
    names = ["tok_embeddings.weight", "norm.weight", "output.weight"]
    for i in range(n_layers):
        p = f"layers.{i}."
        names += [p + s for s in ("attention.wq.weight", "attention.wk.weight", "attention.wv.weight",
                                  "attention.wo.weight", "feed_forward.w1.weight", "feed_forward.w2.weight",
                                  "feed_forward.w3.weight", "attention_norm.weight", "ffn_norm.weight")]
    return names

