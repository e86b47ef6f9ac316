"""KVCache and the fused slot-mapping write on the GPU (tinyvllm/core/kv_cache.py:13-61).

Restates the reference's tests/test_kv_cache.py (shapes, parameters, exact-sum
known answers, reads across blocks, empty reads, memory size, layer isolation)
and checks the fused write bit-exact against the oracle placement.
"""

import numpy as np
import pytest
import torch

from oracle.kv_cache import reshape_and_cache_ref
from tests.random_cases import case_count, case_seed

pytestmark = pytest.mark.gpu


def _cache(*args, **kw):
    from tinyvllm_amd.kv_cache import KVCache
    return KVCache(*args, **kw)


def ones(*shape):
    return torch.ones(*shape, device="cuda")


def arange(n, shape, offset=0.0):
    return (torch.arange(n, dtype=torch.float32) + offset).reshape(shape).cuda()


def test_init_shapes_and_params():
    c = _cache(num_layers=4, num_blocks=10, block_size=16, n_kv_heads=8, head_dim=64, dtype=torch.float32)
    assert len(c.k_cache) == 4 and len(c.v_cache) == 4
    assert c.k_cache[0].shape == (10, 16, 8, 64) and c.v_cache[3].shape == (10, 16, 8, 64)
    assert (c.num_layers, c.num_blocks, c.block_size, c.n_kv_heads, c.head_dim) == (4, 10, 16, 8, 64)
    assert float(c.k_cache[2].abs().sum()) == 0.0


def test_write_kv_basic_and_offset():
    c = _cache(2, 4, 16, 2, 4, "float32")
    c.write_kv(layer_idx=0, block_id=0, start_offset=0, k=ones(5, 2, 4), v=ones(5, 2, 4) * 2)
    for i in range(5):
        assert c.k_cache[0][0, i].sum().item() == 8
        assert c.v_cache[0][0, i].sum().item() == 16
    c.write_kv(layer_idx=0, block_id=0, start_offset=5, k=ones(3, 2, 4) * 5, v=ones(3, 2, 4) * 5)
    for i in range(5, 8):
        assert c.k_cache[0][0, i].sum().item() == 40
    assert c.k_cache[0][0, 8:].abs().sum().item() == 0
    assert c.k_cache[1].abs().sum().item() == 0


def test_write_single_token_2d():
    c = _cache(2, 4, 8, 2, 4, torch.float16)
    c.write_kv(1, 3, 7, ones(2, 4).half(), ones(2, 4).half() * 3)
    assert c.k_cache[1][3, 7].float().sum().item() == 8
    assert c.v_cache[1][3, 7].float().sum().item() == 24


def test_read_single_and_multiple_blocks():
    c = _cache(2, 4, 8, 2, 4, torch.float32)
    c.write_kv(0, 0, 0, arange(40, (5, 2, 4)), arange(40, (5, 2, 4), 100))
    k, v = c.read_kv_blocks(layer_idx=0, block_ids=[0], context_len=5)
    assert k.shape == (5, 2, 4) and v.shape == (5, 2, 4)
    assert torch.equal(k, arange(40, (5, 2, 4))) and torch.equal(v, arange(40, (5, 2, 4), 100))
    c = _cache(2, 4, 4, 2, 4, torch.float32)
    c.write_kv(0, 0, 0, arange(32, (4, 2, 4)), arange(32, (4, 2, 4), 100))
    c.write_kv(0, 1, 0, arange(32, (4, 2, 4), 32), arange(32, (4, 2, 4), 132))
    k, v = c.read_kv_blocks(0, [0, 1], 6)
    assert k.shape == (6, 2, 4)
    assert torch.equal(k, arange(48, (6, 2, 4)))


def test_read_empty_blocks():
    c = _cache(2, 4, 8, 2, 4, torch.float32)
    k, v = c.read_kv_blocks(0, [], 0)
    assert k.shape == (0, 2, 4) and v.shape == (0, 2, 4)


def test_memory_bytes():
    assert _cache(2, 10, 16, 4, 64, torch.float32).get_memory_bytes() == 2 * 10 * 16 * 4 * 64 * 2 * 4
    assert _cache(1, 8, 16, 4, 64, torch.float16).get_memory_bytes() == 8 * 16 * 4 * 64 * 2 * 2


def test_sequence_lifecycle_and_multi_block_sums():
    c = _cache(1, 4, 4, 2, 4, torch.float32)
    for blk, base, n in ((0, 1, 4), (1, 5, 4), (2, 9, 2)):
        rows = torch.stack([ones(2, 4) * (base + i) for i in range(n)])
        c.write_kv(0, blk, 0, rows, rows)
    k, v = c.read_kv_blocks(0, [0, 1, 2], 10)
    assert k.shape == (10, 2, 4)
    for pos in range(10):
        assert k[pos].sum().item() == (pos + 1) * 8


def test_layer_isolation():
    c = _cache(4, 4, 8, 2, 4, torch.float32)
    for layer in range(4):
        c.write_kv(layer, 0, 0, ones(1, 2, 4) * (layer + 1), ones(1, 2, 4) * (layer + 1) * 10)
    for layer in range(4):
        k, v = c.read_kv_blocks(layer, [0], 1)
        assert k.sum().item() == (layer + 1) * 8
        assert v.sum().item() == (layer + 1) * 80


def test_write_kv_rejects_overflowing_chunk():
    c = _cache(1, 4, 8, 2, 4, torch.float32)
    with pytest.raises(ValueError, match="do not fit"):
        c.write_kv(0, 0, 6, ones(3, 2, 4), ones(3, 2, 4))
    with pytest.raises(ValueError, match="block_id"):
        c.write_kv(0, 4, 0, ones(1, 2, 4), ones(1, 2, 4))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hkv,d", [(4, 64), (8, 128), (1, 8), (3, 2)])
def test_fused_slot_write_bit_exact(dtype, hkv, d):
    from tinyvllm_amd.kv_cache import reshape_and_cache
    rng = np.random.Generator(np.random.PCG64(hkv * 1000 + d))
    nb, bs, t = 37, 16, 300
    slots = rng.permutation(nb * bs)[:t].astype(np.int32)
    slots[::17] = -1                                    # padding tokens
    k = torch.from_numpy(rng.standard_normal((t, hkv, d), dtype=np.float32)).to(dtype)
    v = torch.from_numpy(rng.standard_normal((t, hkv, d), dtype=np.float32)).to(dtype)
    kc = torch.from_numpy(rng.standard_normal((nb, bs, hkv, d), dtype=np.float32)).to(dtype)
    vc = torch.from_numpy(rng.standard_normal((nb, bs, hkv, d), dtype=np.float32)).to(dtype)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    kg, vg = kc.cuda(), vc.cuda()
    reshape_and_cache(kg, vg, k.cuda(), v.cuda(), torch.from_numpy(slots).cuda())
    # oracle placement on the raw bit patterns
    ib = torch.int16 if dtype != torch.float32 else torch.int32
    kc_bits = kc_ref.view(ib).numpy().copy()
    vc_bits = vc_ref.view(ib).numpy().copy()
    reshape_and_cache_ref(kc_bits, vc_bits, k.view(ib).numpy(), v.view(ib).numpy(), slots)
    assert np.array_equal(kg.cpu().view(ib).numpy(), kc_bits)
    assert np.array_equal(vg.cpu().view(ib).numpy(), vc_bits)


def test_fused_write_strided_rows_and_error_count():
    from tinyvllm_amd.kv_cache import reshape_and_cache
    nb, bs, hkv, d, t = 4, 8, 2, 64, 5
    qkv = torch.randn(t, 3 * hkv * d, device="cuda", dtype=torch.float16)
    k = qkv[:, :hkv * d].view(t, hkv, d)
    v = qkv[:, hkv * d:2 * hkv * d].view(t, hkv, d)
    kc = torch.zeros(nb, bs, hkv, d, device="cuda", dtype=torch.float16)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([0, 9, 31, 32, 1000], dtype=torch.int32, device="cuda")   # last two past the cache
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    reshape_and_cache(kc, vc, k, v, slots, err_count=err)
    assert err.item() == 2
    flat_k, flat_v = kc.view(nb * bs, hkv, d), vc.view(nb * bs, hkv, d)
    for i, s in enumerate([0, 9, 31]):
        assert torch.equal(flat_k[s], k[i]) and torch.equal(flat_v[s], v[i])
    assert flat_k.abs().sum(dim=(1, 2)).nonzero().flatten().tolist() == [0, 9, 31]


def _random_write_cases(n=None, seed=91):
    n = case_count(8) if n is None else n
    rng = np.random.Generator(np.random.PCG64(case_seed(seed)))
    cases = []
    for i in range(n):
        nb = int(rng.integers(1, 200))
        bs = int(rng.choice([1, 4, 8, 12, 16, 32]))
        hkv = int(rng.choice([1, 2, 3, 4, 8]))
        d = int(rng.choice([2, 8, 32, 64, 80, 128, 256]))
        t = int(rng.integers(1, min(600, nb * bs) + 1))
        dtype = [torch.float32, torch.float16, torch.bfloat16][int(rng.integers(0, 3))]
        cases.append((i, nb, bs, hkv, d, t, dtype))
    return cases


@pytest.mark.parametrize("i,nb,bs,hkv,d,t,dtype", _random_write_cases())
def test_random_fused_writes(i, nb, bs, hkv, d, t, dtype):
    """Seeded random pools (1-199 blocks of 1-32 rows), head shapes, token
    counts and dtypes; slots a random injective map with padding (-1) and
    out-of-range entries mixed in: the cache equals the oracle placement bit
    for bit, out-of-range slots are skipped and counted."""
    from tinyvllm_amd.kv_cache import reshape_and_cache
    rng = np.random.Generator(np.random.PCG64(case_seed(700 + i)))
    slots = rng.permutation(nb * bs)[:t].astype(np.int32)
    kind = rng.integers(0, 10, t)
    slots[kind == 0] = -1                                          # padding tokens
    bad = kind == 1
    slots[bad] = nb * bs + rng.integers(0, 1000, int(bad.sum()))   # past the cache
    k = torch.from_numpy(rng.standard_normal((t, hkv, d), dtype=np.float32)).to(dtype)
    v = torch.from_numpy(rng.standard_normal((t, hkv, d), dtype=np.float32)).to(dtype)
    kc = torch.from_numpy(rng.standard_normal((nb, bs, hkv, d), dtype=np.float32)).to(dtype)
    vc = torch.from_numpy(rng.standard_normal((nb, bs, hkv, d), dtype=np.float32)).to(dtype)
    ib = torch.int16 if dtype != torch.float32 else torch.int32
    kc_bits, vc_bits = kc.view(ib).numpy().copy(), vc.view(ib).numpy().copy()
    kg, vg = kc.cuda(), vc.cuda()
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    reshape_and_cache(kg, vg, k.cuda(), v.cuda(), torch.from_numpy(slots).cuda(), err_count=err)
    keep = np.where(bad, -1, slots).astype(np.int32)
    reshape_and_cache_ref(kc_bits, vc_bits, k.view(ib).numpy(), v.view(ib).numpy(), keep)
    assert err.item() == int(bad.sum())
    assert np.array_equal(kg.cpu().view(ib).numpy(), kc_bits)
    assert np.array_equal(vg.cpu().view(ib).numpy(), vc_bits)


def test_prefill_slot_mapping_drives_fused_write():
    """Prompt written through BlockManager slots == the reference's chunked write_kv loop."""
    from tinyvllm_amd.block_manager import BlockManager
    from tinyvllm_amd.kv_cache import KVCache
    bm = BlockManager(1, 32, 16)
    bm.register_sequence(0)
    L = 70
    slots = bm.prefill_slot_mapping(0, 0, L)
    k = torch.randn(L, 4, 64, device="cuda", dtype=torch.float16)
    v = torch.randn(L, 4, 64, device="cuda", dtype=torch.float16)
    fused = KVCache(1, 32, 16, 4, 64, torch.float16)
    fused.write_kv_slots(0, torch.from_numpy(slots).cuda(), k, v)
    looped = KVCache(1, 32, 16, 4, 64, torch.float16)
    table = bm.get_block_table(0)
    tok, pos = 0, 0
    while tok < L:
        off = pos % 16
        n = min(16 - off, L - tok)
        looped.write_kv(0, table[pos // 16], off, k[tok:tok + n], v[tok:tok + n])
        tok += n
        pos += n
    assert torch.equal(fused.k_cache[0], looped.k_cache[0])
    assert torch.equal(fused.v_cache[0], looped.v_cache[0])


def test_config2_slot_map_fused_write_bit_exact():
    """The bench's own config-2 workload (tinyvllm_amd.workloads.prefill_tinyllama_l512_l1024):
    1536 tokens of seeded fp16 K/V written through its seeded shuffled slot map
    (prompts of 512 and 1024 tokens, block 16, Hkv 4, head_dim 64), one fused
    write per prompt exactly as bench.py times it, then every cache element
    compared bit for bit with the oracle's placement (kv_cache.py:34-38 over
    the slots of llama.py:199-209)."""
    from tinyvllm_amd import workloads
    from tinyvllm_amd.kv_cache import reshape_and_cache
    wl = workloads.prefill_tinyllama_l512_l1024()
    assert sum(len(s) for s in wl.slots) == 1536
    kc = torch.zeros((wl.num_blocks, 16, 4, 64), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    for k, v, s in zip(wl.k, wl.v, wl.slots_dev):
        reshape_and_cache(kc, vc, k[0], v[0], s)
    torch.cuda.synchronize()
    kr = np.zeros((wl.num_blocks, 16, 4, 64), np.float16)
    vr = np.zeros_like(kr)
    for k, v, s in zip(wl.k, wl.v, wl.slots):
        reshape_and_cache_ref(kr, vr, k[0].cpu().numpy(), v[0].cpu().numpy(), s)
    assert np.array_equal(kc.cpu().numpy().view(np.uint16), kr.view(np.uint16))
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), vr.view(np.uint16))
    # the slots are distinct and every written row is a prompt row
    allslots = np.concatenate(wl.slots)
    assert len(np.unique(allslots)) == allslots.size
