"""ctypes binding of libtvattn.so (declarations: include/tv_attn.h, include/tv_llama.h).

The library is required: importing the ops without it raises immediately, and
there is no CPU or PyTorch fallback for any op.
"""

import ctypes
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("TV_ATTN_LIB", _PKG / "libtvattn.so"))

TV_F32, TV_F16, TV_BF16 = 0, 1, 2
TV_OK, TV_EINVAL, TV_EUNSUPPORTED, TV_EHIP = 0, 1, 2, 3

# name -> (restype, argtypes); mirrors include/tv_attn.h, tv_llama.h and tv_bench.h
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_S = ctypes.c_size_t
SIGNATURES = {
    "tv_abi_version": (_I, []),
    "tv_last_error": (ctypes.c_char_p, []),
    "tv_paged_decode_workspace_bytes": (_S, [_I, _I, _I, _I, _I, _I]),
    "tv_paged_decode_partition_size": (_I, [_I, _I, _I, _I, _I, _I, _I]),
    "tv_paged_decode": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _I, _P, _S, _P]),
    "tv_paged_decode_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _I, _P]),
    "tv_flash_prefill_workspace_bytes": (_S, [_I, _I, _I, _I, _I, _I, _I, _I]),
    "tv_flash_prefill": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _L, _L, _L, _L, _I, _F, _I, _I,
                              _I, _P, _S, _P]),
    "tv_flash_prefill_varlen": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _L, _I, _I, _I, _L, _L, _L, _L,
                                     _I, _F, _I, _I, _P]),
    "tv_flash_prefill_paged": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _L, _L, _I, _F, _I, _I, _P]),
    "tv_reshape_and_cache": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _L, _L, _I, _P, _P]),
    "tv_write_kv": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _L, _L, _I, _P]),
    "tv_read_kv_blocks": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    # include/tv_llama.h
    "tv_linear_k_split": (_I, [_I, _I, _I]),
    "tv_linear": (_I, [_P, _P, _P, _I, _I, _I, _L, _L, _I, _I, _P, _I, _P]),
    "tv_rms_norm_residual": (_I, [_P, _P, _P, _I, _P, _P, _I, _P, _I, _I, _F, _I, _P]),
    "tv_rope_table": (_I, [_P, _I, _I, _F, _P]),
    "tv_qkv_rope_cache": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _I, _P, _I, _P, _L, _I, _I, _I, _I, _I, _I, _I,
                               _I, _P, _P, _P]),
    "tv_argmax_advance": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _P]),
    "tv_llama_decode_workspace_bytes": (_S, [_P, _I, _I, _I, _I]),
    "tv_llama_decode_step": (_I, [_P, _P, _P, _P]),
    "tv_llama_graph_create": (_I, [_P, _P, _P, _P, _P]),
    "tv_llama_graph_launch": (_I, [_P, _P]),
    "tv_llama_graph_destroy": (_I, [_P]),
    "tv_llama_prefill_workspace_bytes": (_S, [_P, _I]),
    "tv_llama_prefill": (_I, [_P, _P, _P, _P]),
    # include/tv_bench.h
    "tv_stream_read": (_I, [_P, _L, _I, _I, _I, _I, _P, _P]),
}
ABI_VERSION = 9

_lib = None


class TVError(RuntimeError):
    """A libtvattn call returned a non-zero status."""


def load():
    """Load the library once and attach signatures; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} not found: build it with `python -m tinyvllm_amd.build` "
            "(the attention ops have no fallback path)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.tv_abi_version()
    if ver != ABI_VERSION:
        raise ImportError(f"{LIB_PATH}: ABI version {ver}, expected {ABI_VERSION}; rebuild the library")
    _lib = lib
    return lib


def check(rc, what):
    if rc != TV_OK:
        msg = _lib.tv_last_error().decode(errors="replace") if _lib is not None else ""
        if rc == TV_EINVAL:
            raise ValueError(f"{what}: {msg}")
        raise TVError(f"{what} failed (code {rc}): {msg}")


def dtype_code(dt):
    import torch
    if dt == torch.float32:
        return TV_F32
    if dt == torch.float16:
        return TV_F16
    if dt == torch.bfloat16:
        return TV_BF16
    raise ValueError(f"unsupported dtype {dt} (float32, float16, bfloat16)")


def stream_ptr(device):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
