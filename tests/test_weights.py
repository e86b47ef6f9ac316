"""On-disk weights (tinyvllm/model/weights.py:11-120) -> tinyvllm_amd.weights.

Host tests: the directory and single-file forms, config.json fields, the
reference's dtype detection and its errors.  GPU test: a model loaded from
safetensors files with HF names gives the same logits as the same weights
handed over in memory.
"""

import json

import numpy as np
import pytest
import torch

HF_CONFIG = {"hidden_size": 128, "num_hidden_layers": 2, "num_attention_heads": 4, "num_key_value_heads": 2,
             "vocab_size": 512, "intermediate_size": 256, "rms_norm_eps": 1e-6, "max_position_embeddings": 256,
             "rope_theta": 500000.0}

_TO_HF = {"attention.wq": "self_attn.q_proj", "attention.wk": "self_attn.k_proj", "attention.wv": "self_attn.v_proj",
          "attention.wo": "self_attn.o_proj", "feed_forward.w1": "mlp.gate_proj", "feed_forward.w2": "mlp.down_proj",
          "feed_forward.w3": "mlp.up_proj", "attention_norm": "input_layernorm", "ffn_norm": "post_attention_layernorm"}


def hf_name(meta):
    if meta == "tok_embeddings.weight":
        return "model.embed_tokens.weight"
    if meta == "norm.weight":
        return "model.norm.weight"
    if meta == "output.weight":
        return "lm_head.weight"
    for m, h in _TO_HF.items():
        meta = meta.replace(m, h)
    return "model." + meta


def host_weights(dtype=torch.float16, seed=0):
    """HF-named random weights of HF_CONFIG's shape, on the host."""
    from tinyvllm_amd.llama import LlamaConfig, random_weights
    cfg = LlamaConfig.from_dict(HF_CONFIG, dtype="float32")
    w = random_weights(cfg, seed=seed, device="cpu")
    return {hf_name(k): v.to(dtype).contiguous() for k, v in w.items()}


def save(tmp_path, weights, shards=1, config=True):
    from safetensors.torch import save_file
    names = sorted(weights)
    for i in range(shards):
        part = {n: weights[n] for n in names[i::shards]}
        save_file(part, str(tmp_path / f"model-{i + 1:05d}-of-{shards:05d}.safetensors"))
    if config:
        (tmp_path / "config.json").write_text(json.dumps(HF_CONFIG))


def test_directory_of_shards(tmp_path):
    from tinyvllm_amd.weights import load_llama_weights
    w = host_weights()
    save(tmp_path, w, shards=3)
    cfg, got = load_llama_weights(tmp_path, device="cpu")
    assert (cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.vocab_size, cfg.hidden_dim) == (128, 2, 4, 2, 512, 256)
    assert cfg.norm_eps == 1e-6 and cfg.max_seq_len == 256 and cfg.rope_theta == 500000.0
    assert cfg.dtype == torch.float16                      # auto: float16 weights
    assert set(got) == set(w) and all(torch.equal(got[k], w[k]) for k in w)


def test_single_file_with_config_beside(tmp_path):
    from tinyvllm_amd.weights import load_llama_weights
    w = host_weights(torch.float32)
    save(tmp_path, w)
    cfg, got = load_llama_weights(tmp_path / "model-00001-of-00001.safetensors", device="cpu")
    assert cfg.dtype == torch.float32 and len(got) == len(w)


@pytest.mark.parametrize("stored,asked,want", [
    (torch.float16, "auto", torch.float16), (torch.float32, "auto", torch.float32),
    (torch.bfloat16, "auto", torch.float32),               # the reference's rule: only float16 stays float16
    (torch.float16, "float32", torch.float32), (torch.float32, "float32", torch.float32)])
def test_dtype_detection(tmp_path, stored, asked, want):
    from tinyvllm_amd.weights import load_llama_weights
    save(tmp_path, host_weights(stored))
    cfg, _ = load_llama_weights(tmp_path, dtype=asked, device="cpu")
    assert cfg.dtype == want


def test_errors(tmp_path):
    from tinyvllm_amd.weights import load_llama_weights
    with pytest.raises(FileNotFoundError, match="No .safetensors"):
        load_llama_weights(tmp_path, device="cpu")
    save(tmp_path, host_weights(torch.float32), config=False)
    with pytest.raises(FileNotFoundError, match="config.json"):
        load_llama_weights(tmp_path, device="cpu")
    (tmp_path / "config.json").write_text(json.dumps(HF_CONFIG))
    with pytest.raises(ValueError, match="lose precision"):
        load_llama_weights(tmp_path, dtype="float16", device="cpu")
    with pytest.raises(ValueError, match="Unsupported"):
        load_llama_weights(tmp_path / "model.bin", device="cpu")


@pytest.mark.gpu
def test_loaded_model_matches_in_memory_weights(tmp_path):
    from tinyvllm_amd.block_manager import BlockManager
    from tinyvllm_amd.kv_cache import KVCache
    from tinyvllm_amd.llama import Llama
    from tinyvllm_amd.weights import load_llama_weights
    w = host_weights(torch.float16, seed=3)
    save(tmp_path, w, shards=2)
    cfg, loaded = load_llama_weights(tmp_path)
    assert all(t.is_cuda for t in loaded.values())
    toks = np.random.default_rng(4).integers(0, cfg.vocab_size, 19)
    logits = []
    for weights in (loaded, {k: v.cuda() for k, v in w.items()}):
        model = Llama(cfg, weights)
        kv = KVCache(cfg.n_layers, 8, 16, cfg.n_kv_heads, cfg.head_dim, cfg.dtype)
        bm = BlockManager(1, 8, 16)
        bm.register_sequence(0)
        logits.append(model.prefill(toks, kv, bm, 0))
    torch.cuda.synchronize()
    assert torch.isfinite(logits[0]).all() and torch.equal(logits[0], logits[1])
