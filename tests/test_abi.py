"""The C ABI: libtvattn.so loads on the host and exports exactly what include/*.h declares.

Only host-side entry points run here (no kernel launch): argument validation
paths return before any HIP call.
"""

import ctypes
import re
from pathlib import Path

import pytest

from tinyvllm_amd import _lib

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def header_text():
    return re.sub(r"/\*.*?\*/", "", "\n".join(h.read_text() for h in HEADERS), flags=re.S)


def declared_functions():
    return set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(tv_[a-z_0-9]+)\s*\(", header_text(), flags=re.M))


def test_header_parses():
    names = declared_functions()
    assert {"tv_paged_decode", "tv_flash_prefill", "tv_reshape_and_cache", "tv_write_kv",
            "tv_read_kv_blocks", "tv_last_error", "tv_abi_version",
            "tv_paged_decode_workspace_bytes", "tv_linear", "tv_rms_norm_residual", "tv_qkv_rope_cache",
            "tv_argmax_advance", "tv_llama_decode_step", "tv_llama_prefill", "tv_llama_graph_create"} <= names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    assert set(_lib.SIGNATURES) == declared_functions()
    assert lib.tv_abi_version() == _lib.ABI_VERSION


def test_argument_counts_match_header():
    text = header_text()
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(name + r"\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), name


def test_workspace_size_is_host_arithmetic():
    lib = _lib.load()
    # prefill: L=1024 causal, 32 heads, D=64, split into chunks of one key tile:
    # 16 query tiles x max_chunks x 64 rows x (64 + 2) floats
    ws = lib.tv_flash_prefill_workspace_bytes(1024, 1024, 32, 64, 64, 1, 1, 1)
    unit = 32 * 16 * 64 * 66 * 4
    assert ws > 0 and ws % unit == 0 and ws // unit in (8, 16)      # 128- or 64-key tiles
    assert lib.tv_flash_prefill_workspace_bytes(1024, 1024, 32, 64, 64, 1, 1, 0) == 0      # default: no split
    assert lib.tv_flash_prefill_workspace_bytes(1024, 1024, 32, 64, 64, 1, 0, 4) == 0      # fp32: generic kernel
    assert lib.tv_paged_decode_workspace_bytes(4, 32, 64, 16, 16, 512) == 0      # one partition
    # one partition: the schedule (KV heads per row + order) only, in 256-byte units
    assert lib.tv_paged_decode_workspace_bytes(256, 32, 128, 256, 16, 4096) == 1280
    assert lib.tv_paged_decode_workspace_bytes(255, 32, 128, 256, 16, 4096) == 1024
    assert lib.tv_paged_decode_workspace_bytes(300, 32, 128, 256, 16, 4096) == 1280
    # 256 seqs x 32 heads x 8 partitions x (128 + 2) floats
    assert lib.tv_paged_decode_workspace_bytes(256, 32, 128, 256, 16, 512) == 256 * 32 * 8 * 130 * 4


def test_validation_errors_are_reported_without_launch():
    lib = _lib.load()
    rc = lib.tv_paged_decode(None, None, None, None, None, None, 1, 32, 8, 128, 16, 10, 4, 4,
                             0.1, 1, 1, 512, None, 0, None)
    assert rc == _lib.TV_EINVAL
    assert b"null pointer" in lib.tv_last_error()
    with pytest.raises(ValueError, match="null pointer"):
        _lib.check(rc, "tv_paged_decode")
    fake = ctypes.c_void_p(16)      # never dereferenced: rejected before any launch
    rc = lib.tv_paged_decode(fake, fake, fake, fake, fake, fake, 1, 32, 8, 96, 16, 10, 4, 4,
                             0.1, 1, 1, 512, None, 0, None)
    assert rc == _lib.TV_EUNSUPPORTED and b"head_dim 96" in lib.tv_last_error()
    rc = lib.tv_paged_decode(fake, fake, fake, fake, fake, fake, 1, 32, 8, 128, 16, 10, 4, 4,
                             0.1, 1, 1, 500, None, 0, None)
    assert rc == _lib.TV_EINVAL and b"partition_size" in lib.tv_last_error()
    rc = lib.tv_paged_decode(fake, fake, fake, fake, fake, fake, 1, 32, 8, 128, 16, 10, 64, 64,
                             0.1, 1, 1, 512, None, 0, None)
    assert rc == _lib.TV_EINVAL and b"workspace" in lib.tv_last_error()
    rc = lib.tv_write_kv(fake, fake, fake, fake, 10, 0, 1, 4, 64, 16, 10, 256, 256, 1, None)
    assert rc == _lib.TV_EINVAL and b"block_id" in lib.tv_last_error()
    rc = lib.tv_write_kv(fake, fake, fake, fake, 0, 10, 7, 4, 64, 16, 10, 256, 256, 1, None)
    assert rc == _lib.TV_EINVAL and b"do not fit" in lib.tv_last_error()
    rc = lib.tv_flash_prefill(fake, fake, fake, fake, 0, 4, 8, 8, 64, 64, 512, 512, 512, 512,
                              1, 0.1, 1, 1, 0, None, 0, None)
    assert rc == _lib.TV_EINVAL and b"empty" in lib.tv_last_error()
    rc = lib.tv_flash_prefill(fake, fake, fake, fake, 2048, 2048, 8, 2, 128, 128, 1024, 256, 256, 1024,
                              1, 0.1, 1, 1, 0, ctypes.c_void_p(24), 1 << 20, None)
    assert rc == _lib.TV_EINVAL and b"16-byte aligned" in lib.tv_last_error()
    rc = lib.tv_read_kv_blocks(fake, fake, fake, fake, fake, 1, 17, 4, 64, 16, 10, 1, None)
    assert rc == _lib.TV_EINVAL and b"exceeds" in lib.tv_last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(ImportError, match="no fallback"):
        _lib.load()


def test_no_bit_cast_of_vector_element_lvalues():
    """hipcc (ROCm 7.2) reads element 0 when __builtin_bit_cast is applied to an
    element of an ext_vector_type lvalue (v[i]); sources must go through a
    by-value helper such as u32_as_f32 instead."""
    csrc = Path(__file__).resolve().parents[1] / "tinyvllm_amd" / "csrc"
    bad = []
    for f in sorted(csrc.glob("*")):
        for n, line in enumerate(f.read_text().splitlines(), 1):
            if re.search(r"__builtin_bit_cast\(\s*\w+\s*,\s*\w+(\[[^\]]*\])+\s*\)", line):
                bad.append(f"{f.name}:{n}: {line.strip()}")
    assert not bad, "\n".join(bad)


def test_linear_split_choice():
    """K splits the decode step uses: about 192 work-groups, whole 256-wide K
    chunks, and one split once the output tiles alone fill half of that."""
    lib = _lib.load()
    assert lib.tv_linear_k_split(64, 2560, 2048) == 512        # q|k|v: 40 tiles x 4 splits
    assert lib.tv_linear_k_split(64, 2048, 2048) == 256        # output projection: 32 tiles x 8 splits
    assert lib.tv_linear_k_split(64, 2048, 5632) == 1024       # down projection: 32 tiles x 6 splits
    assert lib.tv_linear_k_split(64, 11264, 2048) == 2048      # w1|w3: 176 tiles, one split
    assert lib.tv_linear_k_split(1024, 2560, 2048) == 2048     # prefill rows fill the GPU
    assert lib.tv_linear_k_split(4, 96, 64) % 32 == 0


def test_dense_entry_points_validate_on_host():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    # K not a multiple of 32, N not a multiple of 4, bad dtype, multi-split logits
    assert lib.tv_linear(p, p, p, 4, 64, 48, 48, 0, 48, 0, None, _lib.TV_F16, None) == _lib.TV_EUNSUPPORTED
    assert lib.tv_linear(p, p, p, 4, 66, 64, 64, 0, 64, 0, None, _lib.TV_F16, None) == _lib.TV_EUNSUPPORTED
    assert lib.tv_linear(p, p, p, 4, 64, 64, 64, 0, 64, 0, None, 7, None) == _lib.TV_EUNSUPPORTED   # no such dtype
    assert lib.tv_linear(p, p, p, 4, 64, 64, 64, 64, 32, 2, None, _lib.TV_F16, None) == _lib.TV_EINVAL
    assert b"one split" in lib.tv_last_error()
    assert lib.tv_qkv_rope_cache(p, None, None, p, None, p, 1, None, 0, p, 8, p, 0, 1, 16, 4, 1, 4, 2, 16,
                                 _lib.TV_F16, None, None, None) == _lib.TV_EINVAL
    assert lib.tv_llama_decode_step(None, None, None, None) == _lib.TV_EINVAL
    assert lib.tv_llama_graph_create(None, None, None, None, None) == _lib.TV_EINVAL


def test_decode_step_workspace_tinyllama():
    """Workspace of the TinyLlama-1.1B step at batch 64 (the end-to-end decode workload)."""
    from tinyvllm_amd.llama import LlamaConfig, _Model
    c = LlamaConfig.tinyllama_1b()
    m = _Model(c.n_layers, c.dim, c.n_heads, c.n_kv_heads, c.head_dim, c.hidden_dim, c.vocab_size, _lib.TV_F16,
               c.norm_eps)
    lib = _lib.load()
    ws = lib.tv_llama_decode_workspace_bytes(ctypes.byref(m), 64, 72, 16, 2048)
    # 8 split partials of the widest product + activations + 500 x 64 argmax keys
    assert 64 * 2560 * 8 * 4 < ws < 16 << 20
    assert lib.tv_llama_decode_workspace_bytes(ctypes.byref(m), 0, 72, 16, 2048) == 0


def test_noalloc_rejects_oversize_launch_on_the_host():
    """tv_paged_decode_noalloc checks the launch against its 16 MiB per-device
    scratch before any HIP call: a launch needing more fails with TV_EINVAL."""
    lib = _lib.load()
    assert lib.tv_paged_decode_workspace_bytes(64, 32, 128, 2048, 16, 256) > (16 << 20)
    rc = lib.tv_paged_decode_noalloc(None, None, None, None, None, None, 64, 32, 8, 128, 16, 100, 2048, 2048,
                                     0.1, _lib.TV_F16, _lib.TV_F16, 256, None)
    assert rc == _lib.TV_EINVAL and b"scratch" in lib.tv_last_error()
