"""LLaMA-architecture model with the reference's interface, running on libtvattn.so.

Mirrors tinyvllm/model/llama.py:347-453 and tinyvllm/model/weights.py:17-58:

* ``LlamaConfig``            -- weights.py:17-58 (same fields and defaults)
* ``Llama.prefill``          -- llama.py:264-285 (one sequence; K/V into the paged cache)
* ``Llama.create_jit_decode``-- llama.py:290-344; returns a ``JitDecode`` that captures
                                the whole batched step into a HIP graph per batch size,
                                the analogue of the engine's per-batch-size TinyJit cache
                                (engine.py:79-81, 157-159)
* ``Llama.decode``           -- llama.py:346-388 (pads / truncates tables to max_blocks,
                                RoPE at start_positions, attention over context_lens,
                                K/V written at each sequence's slot, positions advanced)
* ``Llama.load_weights``     -- llama.py:390-445 (Meta- and HF-style names)

Every forward operation runs in HIP kernels behind include/tv_llama.h; PyTorch
only owns buffers and copies inputs into them.  The model dtype is float32
(the reference's default), float16 or bfloat16; the products run on MFMA in all
three, and fp32 decode attention takes the separate RoPE and paged-decode
kernels (the fused step attention is 16-bit only).

K/V order: the reference attends first and writes the step's K/V afterwards
(llama.py:378-386), so with the engine's ``context_len = position + 1``
(engine.py:251) the last attended slot has not been written yet.  The default
here writes first (``write_before_attend=True``): identical results whenever
``context_len <= position`` (the reference tests' convention,
test_jit_decode.py:102-107), and the token attends to its own K/V otherwise.
``write_before_attend=False`` reproduces the reference's order.
"""

import ctypes

import numpy as np
import torch

from . import _lib
from .attention import default_partition_size
from .kv_cache import as_torch_dtype

_lib.load()

_P = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
_I = ctypes.c_int
_F = ctypes.c_float


class LlamaConfig:
    """Model configuration (weights.py:17-44)."""

    def __init__(self, dim=4096, n_layers=32, n_heads=32, n_kv_heads=None, vocab_size=32000, hidden_dim=None,
                 norm_eps=1e-5, max_seq_len=2048, rope_theta=10000.0, dtype="float32"):
        self.dim = dim
        self.n_layers = n_layers
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads or n_heads
        self.vocab_size = vocab_size
        self.hidden_dim = hidden_dim or 4 * dim
        self.norm_eps = norm_eps
        self.max_seq_len = max_seq_len
        self.rope_theta = rope_theta
        self.head_dim = dim // n_heads
        self.dtype = as_torch_dtype(dtype)

    @classmethod
    def from_dict(cls, d, dtype="float32"):
        """HF ``config.json`` or Meta ``params.json`` keys (weights.py:46-58)."""
        return cls(dim=d.get("hidden_size", d.get("dim", 4096)),
                   n_layers=d.get("num_hidden_layers", d.get("n_layers", 32)),
                   n_heads=d.get("num_attention_heads", d.get("n_heads", 32)),
                   n_kv_heads=d.get("num_key_value_heads", d.get("n_kv_heads")),
                   vocab_size=d.get("vocab_size", 32000),
                   hidden_dim=d.get("intermediate_size", d.get("hidden_dim")),
                   norm_eps=d.get("rms_norm_eps", d.get("norm_eps", 1e-5)),
                   max_seq_len=d.get("max_position_embeddings", d.get("max_seq_len", 2048)),
                   rope_theta=d.get("rope_theta", 10000.0), dtype=dtype)

    @classmethod
    def from_json(cls, path, dtype="float32"):
        """From a ``config.json`` / ``params.json`` file (weights.py:62-66)."""
        import json
        with open(path) as f:
            return cls.from_dict(json.load(f), dtype=dtype)

    @classmethod
    def tinyllama_1b(cls, dtype="float16"):
        """TinyLlama-1.1B: 22 layers, dim 2048, 32 q / 4 KV heads, MLP 5632, vocab 32000."""
        return cls(dim=2048, n_layers=22, n_heads=32, n_kv_heads=4, vocab_size=32000, hidden_dim=5632,
                   norm_eps=1e-5, max_seq_len=2048, rope_theta=10000.0, dtype=dtype)


def weight_shapes(config):
    """Reference (Meta-style) weight names -> shapes (llama.py:398-435)."""
    c = config
    qd, kd = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
    shapes = {"tok_embeddings.weight": (c.vocab_size, c.dim), "norm.weight": (c.dim,),
              "output.weight": (c.vocab_size, c.dim)}
    for i in range(c.n_layers):
        p = f"layers.{i}."
        shapes.update({p + "attention.wq.weight": (qd, c.dim), p + "attention.wk.weight": (kd, c.dim),
                       p + "attention.wv.weight": (kd, c.dim), p + "attention.wo.weight": (c.dim, qd),
                       p + "feed_forward.w1.weight": (c.hidden_dim, c.dim),
                       p + "feed_forward.w2.weight": (c.dim, c.hidden_dim),
                       p + "feed_forward.w3.weight": (c.hidden_dim, c.dim),
                       p + "attention_norm.weight": (c.dim,), p + "ffn_norm.weight": (c.dim,)})
    return shapes


def random_weights(config, seed=0, std=0.02, device="cuda"):
    """Random-init weights: projections and embeddings ~ N(0, std) in the model
    dtype, norm weights ones (RMSNorm init, llama.py:17-19).  Seeded on the device."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    out = {}
    for name, shape in weight_shapes(config).items():
        if len(shape) == 1:
            out[name] = torch.ones(shape, dtype=torch.float32, device=device)
        else:
            w = torch.randn(shape, generator=gen, dtype=torch.float32, device=device)
            out[name] = w.mul_(std).to(config.dtype)
    return out


_HF_MAP = {
    "self_attn.q_proj": "attention.wq", "self_attn.k_proj": "attention.wk", "self_attn.v_proj": "attention.wv",
    "self_attn.o_proj": "attention.wo", "mlp.gate_proj": "feed_forward.w1", "mlp.down_proj": "feed_forward.w2",
    "mlp.up_proj": "feed_forward.w3", "input_layernorm": "attention_norm", "post_attention_layernorm": "ffn_norm",
}


def _from_hf(name):
    if name == "model.embed_tokens.weight":
        return "tok_embeddings.weight"
    if name == "model.norm.weight":
        return "norm.weight"
    if name == "lm_head.weight":
        return "output.weight"
    if name.startswith("model.layers."):
        rest = name[len("model."):]
        for hf, meta in _HF_MAP.items():
            rest = rest.replace(hf, meta)
        return rest
    return name


def canonical_name(name):
    """Map a checkpoint name onto the Meta-style keys (llama.py:398-445): Meta
    names pass through, HF names are translated, and anything else gets the
    reference's fallback rewrites (llama.py:440-445) before translation."""
    if name.startswith("layers.") or name in ("tok_embeddings.weight", "norm.weight", "output.weight"):
        return name
    out = _from_hf(name)
    if out != name:
        return out
    for old, new in (("transformer.", "model."), ("h.", "layers."), ("attn.", "self_attn.")):
        name = name.replace(old, new)
    return _from_hf(name)


class _Model(ctypes.Structure):
    _fields_ = [("n_layers", _I), ("dim", _I), ("n_heads", _I), ("n_kv_heads", _I), ("head_dim", _I),
                ("hidden_dim", _I), ("vocab_size", _I), ("dtype", _I), ("norm_eps", _F),
                ("tok_embeddings", _P), ("wqkv", _PP), ("wo", _PP), ("w13", _PP), ("w2", _PP),
                ("attention_norm", _PP), ("ffn_norm", _PP), ("norm", _P), ("output", _P), ("rope", _P),
                ("rope_len", _I)]


class _Cache(ctypes.Structure):
    _fields_ = [("k_caches", _PP), ("v_caches", _PP), ("num_blocks", _I), ("block_size", _I)]


class _DecodeArgs(ctypes.Structure):
    _fields_ = [("batch", _I), ("tokens", _P), ("positions", _P), ("context_lens", _P), ("block_tables", _P),
                ("bt_stride", _I), ("max_blocks", _I), ("partition_size", _I), ("write_before_attend", _I),
                ("logits", _P), ("history", _P), ("history_len", _I), ("workspace", _P),
                ("workspace_bytes", ctypes.c_size_t)]


class _PrefillArgs(ctypes.Structure):
    _fields_ = [("num_tokens", _I), ("tokens", _P), ("start_pos", _I), ("block_table", _P), ("bt_width", _I),
                ("logits", _P), ("logits_last_only", _I), ("next_token", _P), ("workspace", _P),
                ("workspace_bytes", ctypes.c_size_t), ("attend_prefix", _I)]


def _ptr_array(tensors):
    return (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])


def _i32(x, device):
    if isinstance(x, torch.Tensor):
        return x.to(device=device, dtype=torch.int32).contiguous()
    return torch.as_tensor(np.asarray(x, dtype=np.int32), device=device)


class Llama:
    """LLaMA model on the HIP decode step (llama.py:347-453)."""

    def __init__(self, config, weights=None, *, seed=0, write_before_attend=True, device="cuda"):
        if config.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise ValueError("model dtype must be float32, float16 or bfloat16")
        if config.n_heads % config.n_kv_heads or config.hidden_dim % 2:
            raise ValueError("n_heads must be a multiple of n_kv_heads and hidden_dim even")
        self.config = config
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.write_before_attend = bool(write_before_attend)
        self.rope_len = config.max_seq_len * 2          # llama.py:258
        self.rope = torch.empty((self.rope_len, config.head_dim // 2, 2), dtype=torch.float32, device=self.device)
        lib = _lib.load()
        _lib.check(lib.tv_rope_table(self.rope.data_ptr(), self.rope_len, config.head_dim,
                                     float(config.rope_theta), _lib.stream_ptr(self.device)),
                   "tv_rope_table")
        known = self._known(weights) if weights is not None else {}
        if len(known) == len(weight_shapes(config)):
            self._build(known)
        else:
            # the reference's Llama(config) starts from random-init layers and
            # load_weights replaces only the names it finds (llama.py:390-401)
            self._build(random_weights(config, seed, device=self.device))
            if known:
                self.load_weights(known)
        self._prefill_ws = None

    # ---- weights -----------------------------------------------------------
    def _known(self, weights):
        """Canonical name -> tensor for the names of this model; others are dropped
        (llama.py:395-398: names outside the weight map are ignored)."""
        shapes = weight_shapes(self.config)
        out = {}
        for k, v in weights.items():
            n = canonical_name(k)
            if n in shapes:
                t = v if isinstance(v, torch.Tensor) else torch.as_tensor(np.asarray(v))
                if tuple(t.shape) != shapes[n]:
                    raise ValueError(f"{k}: shape {tuple(t.shape)} != {shapes[n]}")
                out[n] = t
        return out

    def load_weights(self, weights):
        """Load a name -> tensor dict (Meta or HF names, llama.py:390-445), cast to
        the model dtype.  As in the reference, names this model does not have are
        ignored and weights missing from the dict keep their current values; a
        tensor of the wrong shape raises ValueError.  Weights are copied into the
        existing device storage (fused layouts included), so captured decode
        graphs stay valid."""
        c = self.config
        qd, kd, h = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim, c.hidden_dim
        for name, t in self._known(weights).items():
            if name == "tok_embeddings.weight":
                dst = self.tok_embeddings
            elif name == "output.weight":
                dst = self.output
            elif name == "norm.weight":
                dst = self.norm
            else:
                layer, rest = name[len("layers."):].split(".", 1)
                i = int(layer)
                fused13 = self.w13[i].view(h // 2, 2, 2, c.dim)
                dst = {"attention.wq.weight": self.wqkv[i][:qd], "attention.wk.weight": self.wqkv[i][qd:qd + kd],
                       "attention.wv.weight": self.wqkv[i][qd + kd:], "attention.wo.weight": self.wo[i],
                       "feed_forward.w1.weight": fused13[:, 0], "feed_forward.w3.weight": fused13[:, 1],
                       "feed_forward.w2.weight": self.w2[i], "attention_norm.weight": self.attention_norm[i],
                       "ffn_norm.weight": self.ffn_norm[i]}[rest]
                if rest in ("feed_forward.w1.weight", "feed_forward.w3.weight"):
                    t = t.reshape(h // 2, 2, c.dim)
            dst.copy_(t.to(device=self.device, dtype=dst.dtype))

    def _build(self, w):
        """Allocate the device weights from a complete canonical-name dict and build
        the fused layouts the kernels read: wq|wk|wv rows stacked, and w1 / w3
        interleaved two rows at a time (rows 4j, 4j+1 = w1 rows 2j, 2j+1; rows
        4j+2, 4j+3 = w3 rows 2j, 2j+1)."""
        c = self.config

        def dev(name, dtype):
            return w[name].to(device=self.device, dtype=dtype).contiguous()

        dt = c.dtype
        self.tok_embeddings = dev("tok_embeddings.weight", dt)
        self.output = dev("output.weight", dt)
        self.norm = dev("norm.weight", torch.float32)
        self.wqkv, self.wo, self.w13, self.w2, self.attention_norm, self.ffn_norm = [], [], [], [], [], []
        for i in range(c.n_layers):
            p = f"layers.{i}."
            self.wqkv.append(torch.cat([dev(p + "attention.wq.weight", dt), dev(p + "attention.wk.weight", dt),
                                        dev(p + "attention.wv.weight", dt)], 0).contiguous())
            self.wo.append(dev(p + "attention.wo.weight", dt))
            w1 = dev(p + "feed_forward.w1.weight", dt).view(c.hidden_dim // 2, 2, c.dim)
            w3 = dev(p + "feed_forward.w3.weight", dt).view(c.hidden_dim // 2, 2, c.dim)
            self.w13.append(torch.stack([w1, w3], 1).reshape(2 * c.hidden_dim, c.dim).contiguous())
            self.w2.append(dev(p + "feed_forward.w2.weight", dt))
            self.attention_norm.append(dev(p + "attention_norm.weight", torch.float32))
            self.ffn_norm.append(dev(p + "ffn_norm.weight", torch.float32))
        self._arrays = [_ptr_array(x) for x in (self.wqkv, self.wo, self.w13, self.w2, self.attention_norm,
                                                 self.ffn_norm)]
        a = self._arrays
        self._model = _Model(c.n_layers, c.dim, c.n_heads, c.n_kv_heads, c.head_dim, c.hidden_dim, c.vocab_size,
                             _lib.dtype_code(dt), float(c.norm_eps), self.tok_embeddings.data_ptr(),
                             ctypes.cast(a[0], _PP), ctypes.cast(a[1], _PP), ctypes.cast(a[2], _PP),
                             ctypes.cast(a[3], _PP), ctypes.cast(a[4], _PP), ctypes.cast(a[5], _PP),
                             self.norm.data_ptr(), self.output.data_ptr(), self.rope.data_ptr(), self.rope_len)

    def weight_bytes(self):
        ts = [self.tok_embeddings, self.output, self.norm, *self.wqkv, *self.wo, *self.w13, *self.w2,
              *self.attention_norm, *self.ffn_norm]
        return sum(t.numel() * t.element_size() for t in ts)

    # ---- cache binding -------------------------------------------------------
    def cache_struct(self, kv_cache):
        c = self.config
        if kv_cache.num_layers != c.n_layers or kv_cache.n_kv_heads != c.n_kv_heads or \
                kv_cache.head_dim != c.head_dim or kv_cache.dtype != c.dtype:
            raise ValueError("KV cache shape / dtype does not match the model")
        keep = (_ptr_array(kv_cache.k_cache), _ptr_array(kv_cache.v_cache))
        s = _Cache(ctypes.cast(keep[0], _PP), ctypes.cast(keep[1], _PP), kv_cache.num_blocks, kv_cache.block_size)
        return s, keep

    # ---- prefill ---------------------------------------------------------------
    def prefill(self, tokens, kv_cache, block_manager, seq_id, start_pos=0, *, logits="all", attend_prefix=False):
        """Prompt pass of one sequence (llama.py:264-285).  Returns logits
        [1, L, vocab] float32 (``logits="last"``: [1, 1, vocab]; ``None``: no logits).
        ``attend_prefix`` (keyword-only, not in the reference): a chunk at
        ``start_pos > 0`` attends to the cached prefix as well; the reference's
        prefill attends within the chunk only (llama.py:184)."""
        toks = _i32(tokens, self.device).reshape(-1)
        n = toks.numel()
        for pos in range(start_pos, start_pos + n):            # llama.py:206, at layer 0
            block_manager.ensure_block_for_position(seq_id, pos)
        out = self.prefill_table(toks, kv_cache, block_manager.get_block_table(seq_id), start_pos, logits=logits,
                                 attend_prefix=attend_prefix)
        for _ in range(n):                                     # llama.py:282-283
            block_manager.advance_position(seq_id)
        return out

    def prefill_table(self, tokens, kv_cache, block_table, start_pos=0, *, logits="all", next_token=None,
                      attend_prefix=False):
        """Prompt pass over an explicit block table (the table must cover every
        position).  ``next_token``: an int32 device tensor slice that receives the
        greedy token after the last position."""
        c = self.config
        toks = _i32(tokens, self.device).reshape(-1)
        n = toks.numel()
        if n == 0:
            raise ValueError("prefill needs at least one token")
        table = _i32(block_table, self.device).reshape(-1)
        if (start_pos + n - 1) // kv_cache.block_size >= table.numel():
            raise ValueError("block table does not cover the prompt")
        lib = _lib.load()
        need = lib.tv_llama_prefill_workspace_bytes(ctypes.byref(self._model), n)
        if self._prefill_ws is None or self._prefill_ws.numel() < need:
            self._prefill_ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        rows = 0 if logits is None else (1 if logits == "last" else n)
        out = torch.empty((1, rows, c.vocab_size), dtype=torch.float32, device=self.device) if rows else None
        if next_token is not None and (next_token.dtype != torch.int32 or next_token.device != self.device):
            raise ValueError("next_token must be an int32 tensor on the model's device")
        cache, keep = self.cache_struct(kv_cache)
        args = _PrefillArgs(n, toks.data_ptr(), start_pos, table.data_ptr(), table.numel(),
                            out.data_ptr() if out is not None else None, 1 if logits == "last" else 0,
                            next_token.data_ptr() if next_token is not None else None,
                            self._prefill_ws.data_ptr(), self._prefill_ws.numel(), 1 if attend_prefix else 0)
        _lib.check(lib.tv_llama_prefill(ctypes.byref(self._model), ctypes.byref(cache), ctypes.byref(args),
                                        _lib.stream_ptr(self.device)), "tv_llama_prefill")
        del keep
        return out

    # ---- decode ------------------------------------------------------------------
    def create_jit_decode(self, block_size=16):
        """The decode-step compiler (llama.py:290-344): graphs are captured per
        batch size and table width on first use."""
        return JitDecode(self, block_size)

    def decode(self, tokens, kv_cache, block_manager, seq_ids, start_positions, block_tables_tensor,
               context_lens_tensor, jit_fn, max_blocks=64):
        """Batched single-token decode (llama.py:346-388).  Returns logits [B, 1, vocab].

        Each sequence's K/V go to the slot ``block_manager.get_slot(seq_id)``
        names, as in the reference (llama.py:381-386): when the position starts a
        new block, get_slot allocates it, although the engine built the tables
        before that allocation (engine.py:152, 235-255).  The step computes the
        write slot from the table, so the block is patched into the sequence's
        row at column position // block_size.  Attention still covers the first
        ``max_blocks`` columns only (llama.py:368-374); a position past them is
        written through extra columns that attention does not read, as the
        reference writes it to a block its truncated table does not list.
        ``start_positions[i]`` must be the block manager's position of
        ``seq_ids[i]`` (the engine passes ``len - 1``, engine.py:153), since the
        reference rotates by the one and writes at the other.
        """
        bt = _i32(block_tables_tensor, self.device)
        if bt.dim() != 2:
            raise ValueError("block_tables_tensor must be [batch, blocks]")
        batch = bt.shape[0]
        pos = [int(p) for p in np.asarray(start_positions).reshape(-1)]
        if len(seq_ids) != batch or len(pos) != batch:
            raise ValueError("seq_ids, start_positions and block_tables_tensor must have one entry per sequence")
        bs = kv_cache.block_size
        for sid, p in zip(seq_ids, pos):                      # every check before any allocation
            if block_manager.get_context_length(sid) != p:
                raise ValueError(f"sequence {sid}: start position {p} is not the block manager's position "
                                 f"{block_manager.get_context_length(sid)}")
        cols = []
        for sid, p in zip(seq_ids, pos):
            _, block_id, _ = block_manager.get_slot(sid)      # llama.py:382 (allocates on a block boundary)
            cols.append((p // bs, block_id))
        need = max(c for c, _ in cols) + 1
        width = max_blocks if need <= max_blocks else -(-need // 64) * 64
        table = torch.zeros((batch, width), dtype=torch.int32, device=self.device)
        n = min(bt.shape[1], max_blocks)                      # pad / truncate, llama.py:368-374
        table[:, :n] = bt[:, :n]
        rows = torch.arange(batch, device=self.device)
        table[rows, torch.tensor([c for c, _ in cols], device=self.device)] = \
            torch.tensor([b for _, b in cols], dtype=torch.int32, device=self.device)
        graph = jit_fn.graph_for(kv_cache, batch, max_blocks, width)
        graph.set_inputs(tokens, pos, context_lens_tensor, table)
        graph.step()
        logits = graph.logits.clone().unsqueeze(1)
        for sid in seq_ids:                                   # llama.py:387
            block_manager.advance_position(sid)
        return logits


class JitDecode:
    """Per-batch-size cache of captured decode steps (engine.py:79-81, 157-159)."""

    def __init__(self, model, block_size):
        self.model = model
        self.block_size = block_size
        self.graphs = {}

    def graph_for(self, kv_cache, batch, max_blocks, table_width=None):
        width = max_blocks if table_width is None else table_width
        key = (id(kv_cache), batch, max_blocks, width)
        if key not in self.graphs:
            if kv_cache.block_size != self.block_size:
                raise ValueError("KV cache block size differs from the one the decode was created for")
            self.graphs[key] = DecodeGraph(self.model, kv_cache, batch, max_blocks, table_width=width)
        return self.graphs[key]


class DecodeGraph:
    """Device-resident inputs of one batched decode step and its captured HIP graph.

    tokens / positions / context_lens / block_tables live in fixed device
    buffers; each replay reads them, samples the next token into ``tokens`` and
    advances ``positions`` and ``context_lens`` by one, so ``run(n)`` decodes n
    tokens per sequence with no host work between steps (``history`` records
    them when history_len > 0).  The tables are not extended on the device:
    before ``run(n)`` every row must already list the blocks of positions up to
    position + n - 1.  Attention reads the first ``max_blocks`` columns; the
    K/V write slot of position p is column p // block_size of a row of
    ``table_width`` (>= max_blocks) columns.
    """

    def __init__(self, model, kv_cache, batch, max_blocks, *, table_width=None, partition_size=None,
                 keep_logits=True, history_len=0):
        c = model.config
        dev = model.device
        self.model = model
        self.batch = batch
        self.max_blocks = max_blocks
        self.table_width = max_blocks if table_width is None else int(table_width)
        if self.table_width < max_blocks:
            raise ValueError("table_width must be at least max_blocks")
        self.tokens = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.positions = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.context_lens = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.block_tables = torch.zeros((batch, self.table_width), dtype=torch.int32, device=dev)
        self.logits = torch.zeros((batch, c.vocab_size), dtype=torch.float32, device=dev) if keep_logits else None
        self.history_len = history_len
        self.history = torch.zeros((batch, history_len), dtype=torch.int32, device=dev) if history_len else None
        self.partition_size = partition_size or default_partition_size(batch, c.n_heads, c.n_kv_heads, c.head_dim,
                                                                       max_blocks, kv_cache.block_size, c.dtype)
        lib = _lib.load()
        need = lib.tv_llama_decode_workspace_bytes(ctypes.byref(model._model), batch, max_blocks,
                                                   kv_cache.block_size, self.partition_size)
        if need == 0:
            raise ValueError("tv_llama_decode_workspace_bytes rejected the shape")
        self.workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        self._cache, self._keep = model.cache_struct(kv_cache)
        self._args = _DecodeArgs(batch, self.tokens.data_ptr(), self.positions.data_ptr(),
                                 self.context_lens.data_ptr(), self.block_tables.data_ptr(), self.table_width,
                                 max_blocks, self.partition_size, 1 if model.write_before_attend else 0,
                                 self.logits.data_ptr() if self.logits is not None else None,
                                 self.history.data_ptr() if self.history is not None else None,
                                 history_len, self.workspace.data_ptr(), need)
        self._graph = None
        # capture runs on a dedicated stream (the legacy default stream cannot be captured)
        self._stream = torch.cuda.Stream(device=dev)

    def set_inputs(self, tokens, positions, context_lens, block_tables):
        dev = self.model.device
        self.tokens.copy_(_i32(tokens, dev).reshape(-1))
        self.positions.copy_(_i32(positions, dev).reshape(-1))
        self.context_lens.copy_(_i32(context_lens, dev).reshape(-1))
        bt = _i32(block_tables, dev).reshape(self.batch, -1)
        if bt.shape[1] == self.table_width:
            self.block_tables.copy_(bt)
        elif bt.shape[1] == self.max_blocks:
            self.block_tables.zero_()
            self.block_tables[:, :self.max_blocks].copy_(bt)
        else:
            raise ValueError(f"block tables must have {self.max_blocks} or {self.table_width} columns")

    def step_eager(self):
        """Launch the step's kernels directly on the current stream."""
        lib = _lib.load()
        _lib.check(lib.tv_llama_decode_step(ctypes.byref(self.model._model), ctypes.byref(self._cache),
                                            ctypes.byref(self._args), _lib.stream_ptr(self.model.device)),
                   "tv_llama_decode_step")

    def capture(self):
        if self._graph is not None:
            return
        lib = _lib.load()
        handle = ctypes.c_void_p()
        torch.cuda.synchronize(self.model.device)
        _lib.check(lib.tv_llama_graph_create(ctypes.byref(self.model._model), ctypes.byref(self._cache),
                                             ctypes.byref(self._args), ctypes.c_void_p(self._stream.cuda_stream),
                                             ctypes.byref(handle)), "tv_llama_graph_create")
        self._graph = handle

    def step(self):
        """One step through the captured graph, ordered with torch's current stream."""
        self.run(1)

    def run(self, steps):
        """Replay the step ``steps`` times back to back on the current stream."""
        self.capture()
        lib = _lib.load()
        stream = _lib.stream_ptr(self.model.device)
        for _ in range(steps):
            _lib.check(lib.tv_llama_graph_launch(self._graph, stream), "tv_llama_graph_launch")

    def close(self):
        if self._graph is not None:
            _lib.load().tv_llama_graph_destroy(self._graph)
            self._graph = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

