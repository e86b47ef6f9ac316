"""On-disk LLaMA weights as the reference reads them (tinyvllm/model/weights.py:11-120).

``load_llama_weights(model_path, dtype="auto")`` takes a directory of
``*.safetensors`` shards with a ``config.json`` beside them, or one
``.safetensors`` file whose directory holds ``config.json``, and returns
``(LlamaConfig, {name: tensor})`` with the tensors on the GPU; ``Llama(config,
weights)`` takes the dict (Meta- or HF-style names, llama.py:390-445).  Files
are read with the safetensors library, which loads tensor data only.
"""

from pathlib import Path

import torch

from .llama import LlamaConfig


def load_safetensors(path, device="cuda"):
    """All tensors of one safetensors file, moved to ``device`` (weights.py:11-15)."""
    from safetensors.torch import load_file
    return {name: t.to(device) for name, t in load_file(str(path)).items()}


def detect_dtype(weights, dtype):
    """weights.py:69-83: "auto" picks float16 for float16 weights, else float32;
    asking for float16 with other weights is refused (it would lose precision)."""
    first = next(iter(weights.values()))
    if dtype == "auto":
        return "float16" if first.dtype == torch.float16 else "float32"
    if dtype == "float16" and first.dtype != torch.float16:
        raise ValueError(f"Cannot use dtype='float16' with {first.dtype} weights. "
                         "This would lose precision. Use dtype='float32' or dtype='auto'.")
    return dtype


def load_llama_weights(model_path, dtype="auto", device="cuda"):
    """weights.py:86-120: (config, weights) from a directory or one .safetensors file."""
    model_path = Path(model_path)
    if model_path.is_dir():
        weights = {}
        for sf in sorted(model_path.glob("*.safetensors")):
            weights.update(load_safetensors(sf, device))
        if not weights:
            raise FileNotFoundError(f"No .safetensors files found in {model_path}")
        config_path = model_path / "config.json"
    elif model_path.suffix == ".safetensors":
        weights = load_safetensors(model_path, device)
        config_path = model_path.parent / "config.json"
    else:
        raise ValueError(f"Unsupported model format: {model_path}")
    dtype = detect_dtype(weights, dtype)
    if not config_path.exists():
        raise FileNotFoundError(f"No config.json found for {model_path}")
    return LlamaConfig.from_json(config_path, dtype), weights
