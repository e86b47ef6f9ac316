"""tv_paged_decode_noalloc (include/tv_attn.h) against tv_paged_decode.

The no-allocation entry point runs the same kernels with the split partials /
schedule in the library's per-device scratch instead of a caller workspace, so
its output must equal tv_paged_decode's bit for bit at the same partition size.
Each case makes two calls in a row, the second with a smaller input (fewer
sequences, shorter contexts), so stale scratch contents from the first call
cannot leak into the second.  Both calls go through the C ABI with ctypes.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib():
    from tinyvllm_amd import _lib
    return _lib


def _case(seed, batch, hq, hkv, d, bs, ctx_max, dtype):
    rng = np.random.Generator(np.random.PCG64(seed))
    ctx = rng.integers(1, ctx_max + 1, batch).astype(np.int32)
    need = (ctx + bs - 1) // bs
    nb = int(need.sum()) + 5
    perm = rng.permutation(nb).astype(np.int32)
    mb = int(need.max())
    bt = np.zeros((batch, mb), np.int32)
    cur = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[cur:cur + n]
        cur += n
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((batch, 1, hq, d), generator=g, device="cuda").to(dtype)
    kc = torch.randn((nb, bs, hkv, d), generator=g, device="cuda").to(dtype)
    vc = torch.randn((nb, bs, hkv, d), generator=g, device="cuda").to(dtype)
    return q, kc, vc, torch.from_numpy(bt).cuda(), torch.from_numpy(ctx).cuda()


def _args(q, kc, vc, bt, ctx, out, partition):
    L = _lib()
    b, _, hq, d = q.shape
    nb, bs, hkv, _ = kc.shape
    mb = bt.shape[1]
    return [ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(kc.data_ptr()),
            ctypes.c_void_p(vc.data_ptr()), ctypes.c_void_p(bt.data_ptr()), ctypes.c_void_p(ctx.data_ptr()),
            b, hq, hkv, d, bs, nb, mb, mb, 1.0 / math.sqrt(d), L.dtype_code(q.dtype), L.dtype_code(out.dtype),
            partition]


def _with_workspace(q, kc, vc, bt, ctx, partition):
    L = _lib()
    lib = L.load()
    out = torch.empty_like(q)
    b, _, hq, d = q.shape
    ws_bytes = lib.tv_paged_decode_workspace_bytes(b, hq, d, bt.shape[1], kc.shape[1], partition)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    L.check(lib.tv_paged_decode(*_args(q, kc, vc, bt, ctx, out, partition), ctypes.c_void_p(ws.data_ptr()),
                                ws_bytes, L.stream_ptr(q.device)), "tv_paged_decode")
    return out


def _noalloc(q, kc, vc, bt, ctx, partition):
    L = _lib()
    lib = L.load()
    out = torch.full_like(q, float("nan"))
    L.check(lib.tv_paged_decode_noalloc(*_args(q, kc, vc, bt, ctx, out, partition), L.stream_ptr(q.device)),
            "tv_paged_decode_noalloc")
    return out


# (batch, Hq, Hkv, D, block_size, longest context, partition size, dtype):
# split launches (partials + merge in the scratch) and an unsplit batch of >= 32
# sequences (the longest-first schedule in the scratch)
CASES = [
    ((16, 32, 8, 128, 16, 8192, 1024, torch.bfloat16), (5, 32, 8, 128, 16, 3000, 1024, torch.bfloat16)),
    ((8, 32, 4, 64, 16, 2000, 256, torch.float16), (3, 32, 4, 64, 16, 700, 256, torch.float16)),
    ((96, 32, 8, 128, 16, 1024, 1024, torch.float16), (40, 32, 8, 128, 16, 512, 512, torch.float16)),
]


@pytest.mark.parametrize("first,second", CASES, ids=["split-bf16", "split-f16-d64", "scheduled-f16"])
def test_noalloc_equals_workspace_entry(first, second):
    for seed, spec in enumerate((first, second)):
        batch, hq, hkv, d, bs, ctx_max, partition, dtype = spec
        print(f"noalloc case seed {seed}: B{batch} Hq{hq} Hkv{hkv} D{d} bs{bs} ctx<={ctx_max} "
              f"P{partition} {dtype}", flush=True)
        q, kc, vc, bt, ctx = _case(100 + seed, batch, hq, hkv, d, bs, ctx_max, dtype)
        want = _with_workspace(q, kc, vc, bt, ctx, partition)
        got = _noalloc(q, kc, vc, bt, ctx, partition)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want)


def test_noalloc_replays_in_a_captured_graph():
    """Captured in a HIP graph after one eager call on the device (which looks
    the scratch address up), then replayed three times.  Between replays an
    eager no-allocation call on a different, smaller input overwrites the
    shared scratch, and the output is poisoned with NaN: every replay must still
    equal tv_paged_decode bit for bit (the kernels write every scratch element
    they read back, and the graph holds no memset node)."""
    L = _lib()
    lib = L.load()
    spec = (16, 32, 8, 128, 16, 8192, 1024, torch.bfloat16)
    other = (5, 32, 8, 128, 16, 3000, 1024, torch.bfloat16)
    batch, hq, hkv, d, bs, ctx_max, partition, dtype = spec
    q, kc, vc, bt, ctx = _case(200, batch, hq, hkv, d, bs, ctx_max, dtype)
    want = _with_workspace(q, kc, vc, bt, ctx, partition)
    first = _noalloc(q, kc, vc, bt, ctx, partition)         # the device's first call runs eagerly
    torch.cuda.synchronize()
    assert torch.equal(first, want)
    oq, okc, ovc, obt, octx = _case(201, *other[:6], other[7])
    owant = _with_workspace(oq, okc, ovc, obt, octx, other[6])
    out = torch.full_like(q, float("nan"))
    args = _args(q, kc, vc, bt, ctx, out, partition)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        L.check(lib.tv_paged_decode_noalloc(*args, L.stream_ptr(q.device)), "tv_paged_decode_noalloc (capture)")
    for replay in range(3):
        print(f"noalloc graph replay {replay}", flush=True)
        mid = _noalloc(oq, okc, ovc, obt, octx, other[6])     # overwrites the scratch between replays
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(mid, owant), replay
        assert torch.isfinite(out.float()).all(), replay
        assert torch.equal(out, want), replay


def test_noalloc_rejects_launches_beyond_the_scratch():
    """A launch needing more than 16 MiB of partials fails with TV_EINVAL."""
    L = _lib()
    lib = L.load()
    b, hq, d, mb, bs, part = 64, 32, 128, 2048, 16, 256
    assert lib.tv_paged_decode_workspace_bytes(b, hq, d, mb, bs, part) > (16 << 20)
    q = torch.zeros((b, 1, hq, d), dtype=torch.float16, device="cuda")
    kc = torch.zeros((4, bs, 8, d), dtype=torch.float16, device="cuda")
    bt = torch.zeros((b, mb), dtype=torch.int32, device="cuda")
    ctx = torch.ones(b, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    args = _args(q, kc, kc, bt, ctx, out, part)
    rc = lib.tv_paged_decode_noalloc(*args, L.stream_ptr(q.device))
    assert rc == L.TV_EINVAL
    assert b"scratch" in lib.tv_last_error()
