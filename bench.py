"""Benchmark of the MI355X attention hot path (one GPU).

Primary line (``value``): large-batch paged decode at the Llama-3-8B head shape
(Hq 32, Hkv 8, D 128, block_size 16, fp16 KV, 256 sequences, context ~ U[512,
4096], shuffled block pool +10%), reported as achieved HBM GB/s over the
algorithmic bytes (every attended K/V row once + q + out + table entries).

The same JSON line also carries, under ``configs``, the other workloads of the
benchmark set measured the same way: TinyLlama fp32 decode (latency), causal
prefill fp16 L=512+1024 with the fused K/V write (TFLOP/s), long-context split
decode bf16 16 x 32768 (GB/s), and the end-to-end greedy decode of a
random-init TinyLlama-1.1B at batch 64 / context 1024 (tok/s over 128 steps).

Timing: W warm-up launches, then K launches back to back bracketed by
torch.cuda.synchronize() and HIP events on the stream the kernels run on
(torch's current stream).  Small workloads are captured in a HIP graph of K
launches so launch overhead is not measured.  Every workload carries a
``cpu_baseline``: the oracle's float32 numpy restatement of the reference
algorithm (CPU restatement, tinygrad unavailable) timed on the host cores on a
bounded sample -- the padded-gather decode (llama.py:97-144), the full L x L
prefill and per-chunk K/V write loop (llama.py:58-94, 199-209), and one batched
decode step of the model (llama.py:290-388), whose logits also check the GPU's
step 1.  ``traffic`` figures come from rocprofv3 FETCH_SIZE / WRITE_SIZE runs
recorded under profiles/.  ``hbm_read_ceiling`` is the part's measured
streaming-read rate (tv_stream_read over 2 GiB), which the HBM-bound decode
figures are also quoted against (``frac_of_read_ceiling``).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0

# HBM bytes per launch of the primary decode (longest-first order kernel +
# decode kernel) measured with two rocprofv3 --pmc passes (FETCH_SIZE x1.99993 +
# WRITE_SIZE x1.000, factors from a plain 1 GiB copy), recorded in
# profiles/paged_decode_llama3_8b_f16.md.
PRIMARY_TRAFFIC_BYTES = 2500746870
PRIMARY_TRAFFIC_SOURCE = "profiles/paged_decode_llama3_8b_f16.md"
# The same measurement for the split-context decode (decode + merge, per
# launch) and for one TinyLlama decode step (all 157 launches, context 1024).
LONG_TRAFFIC_BYTES = 2152432806
LONG_TRAFFIC_SOURCE = "profiles/paged_decode_long_bf16_b16.md"
STEP_TRAFFIC_BYTES = 4220932722
STEP_TRAFFIC_SOURCE = "profiles/decode_step_tinyllama_b64.md"

# MFMA counters per prefill launch, from one rocprofv3 --pmc pass over
# `bench.py --prefill-only` (SQ_VALU_MFMA_BUSY_CYCLES summed over the 1024
# SIMDs, SQ_INSTS_VALU_MFMA_MOPS_F16 in units of 512 FLOPs), recorded in
# profiles/prefill_tinyllama_f16.md.  Both depend only on the shape (the
# matrix instructions a launch issues), so this run's own time per launch
# turns them into a utilisation: busy cycles / 1024 SIMDs / (ms x 2.4 GHz, the
# clock of the 2.5 PF/s fp16 peak).
PREFILL_MFMA_COUNTERS = {
    "L512": (1327104, 2654208),
    "L1024": (5013504, 10027008),
    "one_launch": (6340608, 12681216),
    "llama3_8b_heads_f16_L2048": (34603008, 69206016),
    "llama3_8b_heads_f16_L4096": (136314880, 272629760),
    "llama3_8b_heads_f16_L8192": (541065216, 1082130432),
    "chunk_over_cached_prefix": (17842176, 35684352),
    "llama3_8b_tp4_shard_f16_L4096": (34078720, 68157440),
}
PREFILL_COUNTER_SOURCE = "profiles/prefill_tinyllama_f16.md"
MFMA_SIMDS = 1024
PEAK_CLOCK_GHZ = 2.4


def mfma_fields(key, ms, flops):
    """Counter-sourced MFMA utilisation of one prefill launch of ``ms`` ms and
    ``flops`` algorithmic FLOPs."""
    busy, mops = PREFILL_MFMA_COUNTERS[key]
    return {"mfma_busy": round(busy / MFMA_SIMDS / (ms * 1e-3 * PEAK_CLOCK_GHZ * 1e9), 4),
            "mfma_busy_cycles": busy,
            "executed_over_algorithmic_flops": round(mops * 512 / flops, 4),
            "counter_source": PREFILL_COUNTER_SOURCE}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def timed(fn, steps, warmup, graph=False):
    """Average ms per launch of ``fn`` over ``steps`` launches on the current stream."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(steps):
                fn()
        g.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        g.replay()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


CPU_LABEL = "CPU restatement, tinygrad unavailable"


def cpu_env():
    """Host threads the CPU baselines run on: numpy's BLAS pool (matrix products)
    and the process's CPU set; elementwise numpy work runs on one thread."""
    import numpy  # noqa: F401  (loads the BLAS library threadpoolctl inspects)
    from threadpoolctl import threadpool_info
    blas = [p for p in threadpool_info() if p.get("user_api") == "blas"]
    return {"blas_threads": max((int(p["num_threads"]) for p in blas), default=1),
            "blas": blas[0].get("internal_api", "?") if blas else "none",
            "sched_getaffinity": len(os.sched_getaffinity(0)), "cpu_count": os.cpu_count()}


def _cpu_entry(value, unit, sample, env, **extra):
    out = {"value": value, "unit": unit, "cores": env["blas_threads"], "kind": "port", "label": CPU_LABEL,
           "sample": sample, "threads": {**env, "note": "BLAS products on blas_threads threads; "
                                                            "elementwise numpy on one thread"}}
    out.update(extra)
    return out


def _time_cpu(fn, seconds, min_iters=1):
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= min_iters:
            return n, el


def _compact_decode(wl, idx):
    """q, caches and remapped tables of the sequences ``idx`` of a decode workload, on the host."""
    import torch
    bt = wl.block_tables[idx]
    used = sorted(set(bt.reshape(-1).tolist()))
    remap = {b: i for i, b in enumerate(used)}
    bt_s = np.vectorize(remap.get)(bt).astype(np.int32)
    sel = torch.tensor(used, dtype=torch.long, device=wl.k_cache.device)
    kc = wl.k_cache.index_select(0, sel).float().cpu().numpy()
    vc = wl.v_cache.index_select(0, sel).float().cpu().numpy()
    q = wl.q[list(idx)].float().cpu().numpy()
    return q, kc, vc, bt_s


def cpu_baseline_decode(wl, seconds=10.0, sample_seqs=16, env=None):
    """Time the oracle's float32 restatement of the reference's paged decode
    (llama.py:97-144: padded gather to the table width, GQA expand, full scores,
    -1e9 mask, softmax, PV) on the first ``sample_seqs`` sequences."""
    from oracle.attention import paged_decode_ref
    env = env or cpu_env()
    idx = np.arange(min(sample_seqs, wl.batch))
    q, kc, vc, bt_s = _compact_decode(wl, idx)
    ctx = wl.context_lens[idx]
    n, el = _time_cpu(lambda: paged_decode_ref(q, kc, vc, bt_s, ctx, wl.num_heads, wl.num_kv_heads, wl.head_dim,
                                               wl.block_size, acc=np.float32), seconds)
    es = wl.k_cache.element_size()
    b = len(idx)
    blocks = int(((ctx.astype(np.int64) + wl.block_size - 1) // wl.block_size).sum())
    sample_bytes = (int(ctx.astype(np.int64).sum()) * wl.num_kv_heads * wl.head_dim * 2 * es
                    + b * wl.num_heads * wl.head_dim * 2 * es + blocks * 4 + b * 4)
    return _cpu_entry(round(sample_bytes * n / el / 1e9, 4), "GB/s",
                      f"{b} of {wl.batch} sequences (sum ctx {int(ctx.sum())}), {n} passes in {el:.1f} s; numpy "
                      f"float32 restatement of llama.py:97-144 incl. the padded gather to the {bt_s.shape[1]}-block "
                      f"table width", env, ms_per_call=round(el / n * 1e3, 3), sample_bytes=sample_bytes)


def cpu_baseline_prefill(wl, seconds=6.0, env=None):
    """Time the oracle's float32 restatement of the reference's prefill attention
    (llama.py:58-94: GQA expand, full L x L scores, -1e9 causal mask, softmax, PV)
    on each prompt, and its per-chunk K/V write loop (llama.py:199-209 over
    KVCache.write_kv, kv_cache.py:34-38)."""
    from oracle.attention import flash_prefill_ref
    from oracle.kv_cache import KVCacheRef
    env = env or cpu_env()
    per, flops_each = [], []
    for i, length in enumerate(wl.lengths):
        hq, hk, hv = wl.host[i]
        n, el = _time_cpu(lambda: flash_prefill_ref(hq, hk, hv, True, acc=np.float32), seconds / 2 / len(wl.lengths))
        per.append(el / n)
        flops_each.append(4 * wl.num_heads * wl.head_dim * length * (length + 1) // 2)
    cache = KVCacheRef(1, wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim, np.float16)
    ks = [wl.host[i][1][0].astype(np.float16) for i in range(len(wl.lengths))]
    vs = [wl.host[i][2][0].astype(np.float16) for i in range(len(wl.lengths))]
    bs = wl.block_size

    def write_loop():
        for slots, k, v in zip(wl.slots, ks, vs):
            pos, t = 0, len(slots)
            while pos < t:                                   # llama.py:203-209
                off = pos % bs
                n = min(bs - off, t - pos)
                cache.write_kv(0, int(slots[pos]) // bs, off, k[pos:pos + n], v[pos:pos + n])
                pos += n

    nw, elw = _time_cpu(write_loop, seconds / 2, min_iters=3)
    tot = sum(per)
    return _cpu_entry(round(sum(flops_each) / tot / 1e12, 5), "TFLOP/s",
                      f"every prompt ({'+'.join(map(str, wl.lengths))} tokens), numpy float32 restatement of "
                      f"llama.py:58-94 with the full L x L scores; K/V write loop of llama.py:199-209 "
                      f"({sum(len(s) for s in wl.slots)} tokens, {nw} passes)", env,
                      ms_per_prompt=[round(x * 1e3, 2) for x in per], kv_write_ms=round(elw / nw * 1e3, 3))


def cpu_baseline_e2e(state, env=None):
    """The oracle's float32 restatement of one batched decode step
    (llama.py:290-388 over the reference layers; RMSNorm, interleaved RoPE,
    paged attention with the padded gather, SwiGLU, greedy) at the workload's
    batch, fed with the K/V the device wrote; one step timed, tok/s
    extrapolated from it.  Its logits are the parity reference for the GPU's
    step 1 (max-abs and the greedy match over the batch)."""
    import torch
    from oracle.llama import LlamaRef, greedy_ref
    from tinyvllm_amd.llama import random_weights
    env = env or cpu_env()
    wl = state["wl"]
    m, kv = wl.model, wl.kv
    B, L = wl.batch, wl.prompt_len
    t0 = time.perf_counter()
    w = {name: t.float().cpu().numpy() for name, t in random_weights(m.config, seed=wl.seed).items()}
    torch.cuda.empty_cache()
    ref = LlamaRef(m.config, w, cache_dtype=np.float16)
    ncols = L // kv.block_size + 1
    ids = torch.from_numpy(wl.tables[:, :ncols].reshape(-1).astype(np.int64)).cuda()
    kc = [k.index_select(0, ids).float().cpu().numpy() for k in kv.k_cache]
    vc = [v.index_select(0, ids).float().cpu().numpy() for v in kv.v_cache]
    tables = np.arange(B * ncols, dtype=np.int32).reshape(B, ncols)
    prep = time.perf_counter() - t0
    first = state["first"]
    t0 = time.perf_counter()
    want = ref.decode(first, [L] * B, [L + 1] * B, tables, kc, vc, kv.block_size)
    el = time.perf_counter() - t0
    got = state["step1_logits"]
    # teacher-forced: the oracle decodes every step of the run on the device's
    # tokens and K/V rows for the kept sequences (llama.py:346-388,
    # sampling.py:131-134); logits within 2e-2, greedy token equal where the
    # oracle's top two logits are more than 2 x 2e-2 apart
    seqs, steps = state["tf_seqs"], state["steps"]
    ncols = -(-(L + steps) // kv.block_size)
    ids = torch.from_numpy(wl.tables[seqs, :ncols].reshape(-1).astype(np.int64)).cuda()
    tkc = [k.index_select(0, ids).float().cpu().numpy() for k in kv.k_cache]
    tvc = [v.index_select(0, ids).float().cpu().numpy() for v in kv.v_cache]
    ttab = np.arange(len(seqs) * ncols, dtype=np.int32).reshape(len(seqs), ncols)
    n = len(seqs)
    worst, matches, clear_total, clear_match = 0.0, [], 0, 0
    t1 = time.perf_counter()
    for i in range(steps):
        want_i = ref.decode([int(t) for t in state["tf_inputs"][i]], [L + i] * n, [L + i + 1] * n, ttab, tkc, tvc,
                            kv.block_size)
        got_i = state["tf_logits"][i]
        worst = max(worst, float(np.abs(got_i - want_i).max()))
        top2 = np.sort(want_i, axis=1)[:, -2:]
        clear = top2[:, 1] - top2[:, 0] > 2 * 2e-2
        gt = np.argmax(got_i, 1)
        clear_total += int(clear.sum())
        clear_match += int((gt[clear] == greedy_ref(want_i)[clear]).sum())
        matches += (gt == greedy_ref(want_i)).tolist()
    state["tf_parity"] = {"sequences": seqs, "steps": steps, "logits_max_abs": round(worst, 6),
                          "token_match_rate_128": round(float(np.mean(matches)), 4),
                          "clear_margin_matches": f"{clear_match}/{clear_total}",
                          "clear_margin_match_rate": round(clear_match / max(1, clear_total), 4),
                          "tolerance": 2e-2, "clear_margin": 4e-2,
                          "seconds": round(time.perf_counter() - t1, 1)}
    return _cpu_entry(round(B / el, 3), "tok/s",
                      f"one step at batch {B}, context {L} (the GPU's step 1, K/V gathered from the device), "
                      f"numpy float32 restatement of llama.py:290-388; tok/s = {B} / step time "
                      f"(the 128-step run extrapolated from one step)", env,
                      ms_per_step=round(el * 1e3, 1), prep_s=round(prep, 1),
                      parity={"step1_logits_max_abs": round(float(np.abs(got - want).max()), 6),
                              "step1_greedy_match_rate": round(float(np.mean(np.argmax(got, 1) == greedy_ref(want))), 4),
                              "tolerance": 2e-2, "sequences": B})

def per_launch_ms(fn, launches):
    """Each of ``launches`` calls of ``fn`` timed alone (HIP events around one
    launch on the launch stream, the previous one finished): (median, min, max) ms."""
    import torch
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(launches)]
    for a, b in ev:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    t = sorted(a.elapsed_time(b) for a, b in ev)
    return t[len(t) // 2], t[0], t[-1]


def bench_decode(wl, steps, warmup, graph, per_launch=0):
    from tinyvllm_amd.attention import PagedDecodePlan
    plan = PagedDecodePlan(wl.q, wl.k_cache, wl.v_cache, wl.bt_dev, wl.ctx_dev, wl.num_heads,
                           wl.num_kv_heads, wl.head_dim, wl.block_size)
    ms = timed(plan.run, steps, warmup, graph)
    gbs = wl.algorithmic_bytes() / (ms * 1e-3) / 1e9
    out = {"ms": ms, "gbs": gbs, "bytes": wl.algorithmic_bytes(), "flops": wl.flops(),
           "partition_size": plan.partition_size}
    if per_launch:
        med, lo, hi = per_launch_ms(plan.run, per_launch)
        out["per_launch"] = {"launches": per_launch, "median_ms": round(med, 5), "min_ms": round(lo, 5),
                             "max_ms": round(hi, 5),
                             "median_gbs": round(wl.algorithmic_bytes() / (med * 1e-3) / 1e9, 1),
                             "median_frac_of_hbm_peak": round(wl.algorithmic_bytes() / (med * 1e-3) / 1e9
                                                              / HBM_PEAK_GBS, 4)}
    return out


def bench_prefill(steps, warmup):
    import torch
    from tinyvllm_amd.attention import PrefillPlan, VarlenPrefillPlan
    from tinyvllm_amd.kv_cache import reshape_and_cache
    from tinyvllm_amd.workloads import prefill_tinyllama_l512_l1024
    wl = prefill_tinyllama_l512_l1024()
    plans = [PrefillPlan(q, k, v, True) for q, k, v in zip(wl.q, wl.k, wl.v)]
    per = [timed(p.run, steps, warmup, graph=True) for p in plans]
    # the same two prompts packed into one launch (an extension: the reference
    # engine prefills one prompt per call, so the headline value is per call)
    packed = [torch.cat([t[0] for t in ts]) for ts in (wl.q, wl.k, wl.v)]
    lens = [t.shape[1] for t in wl.q]
    ms_packed = timed(VarlenPrefillPlan(*packed, lens, True).run, steps, warmup, graph=True)
    kc = torch.zeros((wl.num_blocks, 16, 4, 64), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)

    def write():
        for k, v, s in zip(wl.k, wl.v, wl.slots_dev):
            reshape_and_cache(kc, vc, k[0], v[0], s)
    wms = timed(write, steps, warmup, graph=True)
    tot = sum(per)
    flops = wl.flops()
    # Llama-3-8B heads (Hq 32 / Hkv 8, head_dim 128), one prompt of 2048, 4096
    # and 8192 tokens (the 128-row kernel; at 4096+ the grid holds more
    # work-groups than are resident at once).
    long_prompts = {}
    for L8 in (2048, 4096, 8192):
        g = torch.Generator(device="cuda").manual_seed(0)
        hq8, hkv8, d8 = 32, 8, 128
        q8 = torch.randn((1, L8, hq8, d8), generator=g, device="cuda").half()
        k8 = torch.randn((1, L8, hkv8, d8), generator=g, device="cuda").half()
        v8 = torch.randn((1, L8, hkv8, d8), generator=g, device="cuda").half()
        ms8 = timed(PrefillPlan(q8, k8, v8, True).run, steps, warmup, graph=True)
        flops8 = 2 * hq8 * d8 * L8 * (L8 + 1)
        long_prompts[f"llama3_8b_heads_f16_L{L8}"] = {
            "value": round(flops8 / (ms8 * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
            "ms": round(ms8, 5), "flops": flops8,
            "frac_of_fp16_mfma_peak": round(flops8 / (ms8 * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
            **mfma_fields(f"llama3_8b_heads_f16_L{L8}", ms8, flops8)}
        del q8, k8, v8
    # The same heads sharded over four GPUs (8 query / 2 KV heads each), one
    # prompt of 4096 tokens: a grid that leaves most resident slots empty,
    # where the longer causal query tiles run as two key halves and a second
    # kernel merges them.
    g = torch.Generator(device="cuda").manual_seed(0)
    hqs, hkvs, ds, Ls = 8, 2, 128, 4096
    qs = torch.randn((1, Ls, hqs, ds), generator=g, device="cuda").half()
    ks = torch.randn((1, Ls, hkvs, ds), generator=g, device="cuda").half()
    vs = torch.randn((1, Ls, hkvs, ds), generator=g, device="cuda").half()
    plan_s = PrefillPlan(qs, ks, vs, True)
    mss = timed(plan_s.run, steps, warmup, graph=True)
    flopss = 2 * hqs * ds * Ls * (Ls + 1)
    long_prompts["llama3_8b_tp4_shard_f16_L4096"] = {
        "value": round(flopss / (mss * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms": round(mss, 5), "flops": flopss,
        "frac_of_fp16_mfma_peak": round(flopss / (mss * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
        "split_key_halves": plan_s.ws_bytes > 0,
        **mfma_fields("llama3_8b_tp4_shard_f16_L4096", mss, flopss)}
    del qs, ks, vs, plan_s
    chunk = bench_chunk_over_prefix(steps, warmup)
    return wl, {
        "workload": "prefill_tinyllama_f16_L512+L1024 (Hq32 Hkv4 D64, causal) + fused KV write",
        "value": round(flops / (tot * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
        "ms_per_prompt": [round(x, 5) for x in per],
        "flops": flops,
        "frac_of_fp16_mfma_peak": round(flops / (tot * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
        "mfma_busy_per_prompt": [mfma_fields(k, ms, 4 * wl.num_heads * wl.head_dim * (n * (n + 1) // 2))["mfma_busy"]
                                 for k, ms, n in zip(("L512", "L1024"), per, wl.lengths)],
        "mfma_busy": round(sum(PREFILL_MFMA_COUNTERS[k][0] for k in ("L512", "L1024")) / MFMA_SIMDS
                           / (tot * 1e-3 * PEAK_CLOCK_GHZ * 1e9), 4),
        "executed_over_algorithmic_flops": round(
            sum(PREFILL_MFMA_COUNTERS[k][1] for k in ("L512", "L1024")) * 512 / flops, 4),
        "counter_source": PREFILL_COUNTER_SOURCE,
        "one_launch": {"value": round(flops / (ms_packed * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
                       "ms": round(ms_packed, 5), "note": "both prompts in one tv_flash_prefill_varlen launch",
                       **mfma_fields("one_launch", ms_packed, flops)},
        "kv_write_ms": round(wms, 5),
        "kv_write_gbs": round(wl.kv_write_bytes() / (wms * 1e-3) / 1e9, 1),
        **long_prompts,
        "chunk_over_cached_prefix": chunk,
    }


def calibration_copy(mib):
    """One plain device copy of ``mib`` MiB: the reference transfer the HBM
    counters (FETCH_SIZE, WRITE_SIZE) are scaled by."""
    import torch
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"bench: calibration copy of {n} bytes done")


def bench_read_ceiling(steps=20, warmup=5, gib=2):
    """The part's streaming-read ceiling: tv_stream_read over a 2 GiB buffer (8x
    the 256 MB memory-side cache), ordinary and non-temporal 16-byte loads, 4 or
    8 in flight per lane, 2-16 work-groups of 256 lanes per CU, each reading
    one contiguous range or strided over the whole grid.  The HBM-bound
    kernels are quoted against the 8 TB/s peak and against this ceiling."""
    import ctypes
    import torch
    from tinyvllm_amd import _lib
    lib = _lib.load()
    n = gib << 30
    buf = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(3)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(16 * cus, dtype=torch.int32, device="cuda")      # one word per work-group
    variants = {}
    for contig in (0, 1):
        for nt in (0, 1):
            for u in (4, 8):
                for per_cu in (2, 4, 8, 16):
                    wg = per_cu * cus

                    def fn(nt=nt, u=u, wg=wg, contig=contig):
                        rc = lib.tv_stream_read(ctypes.c_void_p(buf.data_ptr()), n, nt, u, wg, contig,
                                                ctypes.c_void_p(sink.data_ptr()),
                                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                        if rc != 0:
                            raise RuntimeError(lib.tv_last_error().decode())
                    ms = timed(fn, steps, warmup)
                    name = f"{'contig' if contig else 'strided'}_{'nt' if nt else 'plain'}_u{u}_wg{per_cu}x"
                    variants[name] = round(n / (ms * 1e-3) / 1e9, 1)
    best = max(variants, key=variants.get)
    del buf
    return {"value": variants[best], "unit": "GB/s", "frac_of_hbm_peak": round(variants[best] / HBM_PEAK_GBS, 4),
            "best": best, "bytes": n, "best_plain": max(v for k, v in variants.items() if "_plain_" in k),
            "variants": variants,
            "note": "read-only stream of 16-byte vectors; variant = layout (one contiguous range per "
                    "work-group or strided over the grid), load kind, loads in flight per lane, work-groups per CU"}


def bench_chunk_over_prefix(steps, warmup, prefix=3584, chunk=512):
    """A 512-token prompt chunk after a 3584-token cached prefix (TinyLlama heads,
    fp16, block 16, shuffled blocks): the MFMA pass through the block table
    (tv_flash_prefill_paged) against one paged decode query per chunk row over
    the same table (the previous chunked-prefill path)."""
    import ctypes
    import math
    import torch
    from tinyvllm_amd import _lib
    from tinyvllm_amd.attention import flash_prefill_paged
    hq, hkv, d, bs = 32, 4, 64, 16
    total = prefix + chunk
    nblk = total // bs
    rng = np.random.Generator(np.random.PCG64(3))
    table = torch.from_numpy(rng.permutation(nblk + 8)[:nblk].astype(np.int32)).cuda()
    g = torch.Generator(device="cuda").manual_seed(3)
    kc = torch.randn((nblk + 8, bs, hkv, d), generator=g, device="cuda").half()
    vc = torch.randn((nblk + 8, bs, hkv, d), generator=g, device="cuda").half()
    q = torch.randn((chunk, hq, d), generator=g, device="cuda").half()
    ms_new = timed(lambda: flash_prefill_paged(q, kc, vc, table, prefix), steps, warmup, graph=False)
    lib = _lib.load()
    ctx = torch.arange(prefix + 1, total + 1, dtype=torch.int32, device="cuda")
    out = torch.empty((chunk, 1, hq, d), dtype=torch.float16, device="cuda")
    part = (total + 15) // 16 * 16
    ws_bytes = lib.tv_paged_decode_workspace_bytes(chunk, hq, d, nblk, bs, part)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    args = (out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), table.data_ptr(), ctx.data_ptr(), chunk, hq,
            hkv, d, bs, kc.shape[0], 0, nblk, 1.0 / math.sqrt(d), _lib.TV_F16, _lib.TV_F16, part,
            ctypes.c_void_p(ws.data_ptr()), ws_bytes)

    def per_row():
        _lib.check(lib.tv_paged_decode(*args, _lib.stream_ptr(torch.device("cuda"))), "tv_paged_decode")
    ms_old = timed(per_row, steps, warmup, graph=False)
    new = flash_prefill_paged(q, kc, vc, table, prefix)[0]
    per_row()
    torch.cuda.synchronize()
    flops = 4 * hq * d * (chunk * prefix + chunk * (chunk + 1) // 2)
    return {"workload": f"chunk of {chunk} after {prefix} cached tokens, Hq32 Hkv4 D64 fp16, block 16 shuffled",
            "value": round(flops / (ms_new * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms": round(ms_new, 5),
            "frac_of_fp16_mfma_peak": round(flops / (ms_new * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
            **mfma_fields("chunk_over_cached_prefix", ms_new, flops),
            "per_row_decode_ms": round(ms_old, 5), "speedup": round(ms_old / ms_new, 2),
            "max_abs_diff_vs_per_row": round(float((new.float() - out[:, 0].float()).abs().max()), 6)}


def bench_e2e(decode_steps=128, warmup=3):
    """Batched greedy decode of random-init TinyLlama-1.1B: 64 prompts of 1024
    seeded tokens prefilled into the paged cache, then ``decode_steps`` steps
    replayed from one captured HIP graph (sampling and position advance on the
    device, no host work between steps)."""
    import torch
    from tinyvllm_amd import workloads
    from tinyvllm_amd.llama import DecodeGraph
    wl = workloads.e2e_tinyllama_b64(decode_steps=decode_steps)
    m, kv = wl.model, wl.kv
    B, L = wl.batch, wl.prompt_len
    first = torch.zeros(B, dtype=torch.int32, device="cuda")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for b in range(B):
        m.prefill_table(wl.prompts[b], kv, wl.tables[b], 0, logits=None, next_token=first[b:b + 1])
    e1.record()
    torch.cuda.synchronize()
    prefill_ms = e0.elapsed_time(e1)
    g = DecodeGraph(m, kv, B, wl.tables.shape[1], keep_logits=False, history_len=L + decode_steps + 2)

    def reset():
        g.set_inputs(first, [L] * B, [L + 1] * B, wl.tables)

    reset()
    g.run(warmup)                       # captures the graph; the steps' cache rows are rewritten below
    torch.cuda.synchronize()
    reset()
    torch.cuda.synchronize()
    e0.record()
    g.run(decode_steps)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    hist = g.history[:, L + 1:L + 1 + decode_steps].cpu().numpy().astype(np.int64)
    nbytes = wl.bytes_for_steps(L, decode_steps)
    g.close()
    # the same steps driven from the host (tokens copied in every step), keeping
    # the logits of two sequences for the CPU leg's teacher-forced parity check
    # over the whole run; their tokens must equal the timed device loop's
    tf_seqs = [0, B - 1]
    sel = torch.tensor(tf_seqs, device="cuda")
    hg = DecodeGraph(m, kv, B, wl.tables.shape[1])
    cur = first.clone()
    tf_inputs, tf_logits, host_equal = [], [], True
    for i in range(decode_steps):
        tf_inputs.append(cur.cpu().numpy()[tf_seqs])
        hg.set_inputs(cur, [L + i] * B, [L + i + 1] * B, wl.tables)
        hg.step()
        cur = hg.tokens.clone()
        tf_logits.append(hg.logits.index_select(0, sel).cpu().numpy())
        host_equal &= bool(np.array_equal(cur.cpu().numpy(), hist[:, i]))
    hg.close()
    # step 1 again from the prefilled state, keeping its logits for the parity
    # check of the CPU leg (rows written past position L are never attended by
    # step 1)
    g1 = DecodeGraph(m, kv, B, wl.tables.shape[1])
    g1.set_inputs(first, [L] * B, [L + 1] * B, wl.tables)
    g1.step()
    state = {"wl": wl, "first": first.cpu().numpy(), "step1_logits": g1.logits.cpu().numpy(),
             "tf_seqs": tf_seqs, "tf_inputs": tf_inputs, "tf_logits": tf_logits, "steps": decode_steps}
    g1.close()
    return state, {
        "workload": "tinyllama_1.1b_random_init_f16 decode: B64, prompts 1024 (seeded), 128 greedy steps, "
                    "block16, shuffled pool +10%, one HIP graph per step",
        "value": round(B * decode_steps / (ms * 1e-3), 1), "unit": "tok/s",
        "ms_per_step": round(ms / decode_steps, 4),
        "weight_bytes_per_step": wl.weight_bytes_per_step(),
        "algorithmic_bytes": nbytes,
        "achieved_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "traffic_per_step": STEP_TRAFFIC_BYTES,
        "traffic_over_algorithmic": round(STEP_TRAFFIC_BYTES / wl.bytes_for_steps(L, 1), 4),
        "traffic_source": STEP_TRAFFIC_SOURCE,
        "prefill_tok_s": round(B * L / (prefill_ms * 1e-3), 1),
        "prefill_ms": round(prefill_ms, 2),
        "tokens_checksum": int((hist * (np.arange(hist.size).reshape(hist.shape) % 9973 + 1)).sum()),
        "first_tokens_seq0": hist[0, :8].tolist(),
        "host_driven_steps_equal_device_loop": host_equal,
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU time of the primary workload's baseline (the others take a few seconds each)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--primary-only", action="store_true")
    ap.add_argument("--e2e-only", action="store_true",
                    help="run only the end-to-end TinyLlama decode and print its result (profiling)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the causal prefill + K/V write workload and print its result (profiling)")
    ap.add_argument("--decode-long-only", action="store_true",
                    help="run only the split-context decode B16 x 32768 and print its result (profiling)")
    ap.add_argument("--decode-small-only", action="store_true",
                    help="run only the TinyLlama fp32 B4 paged decode and print its result (profiling)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run one plain device copy of this many MiB (HBM counter calibration)")
    ap.add_argument("--read-ceiling-only", action="store_true",
                    help="run only the streaming-read ceiling and print its result (profiling)")
    ap.add_argument("--e2e-steps", type=int, default=128,
                    help="decode steps of the end-to-end run with --e2e-only (profiling runs use fewer)")
    args = ap.parse_args()
    if args.gpus != 1:
        sys.exit("bench.py measures one GPU only: this build has no multi-GPU path "
                 "(the attention hot path shards by sequence or KV head with no exchange)")

    import torch
    from tinyvllm_amd import workloads

    torch.cuda.set_device(0)
    cpu_on = not args.no_cpu_baseline
    env = cpu_env() if cpu_on else None
    if (args.e2e_only or args.prefill_only or args.decode_long_only or args.read_ceiling_only
            or args.decode_small_only):
        if args.calib_copy_mib:
            calibration_copy(args.calib_copy_mib)
        if args.read_ceiling_only:
            out = bench_read_ceiling()
        elif args.e2e_only:
            out = bench_e2e(decode_steps=args.e2e_steps)[1]
        elif args.prefill_only:
            out = bench_prefill(args.steps, args.warmup)[1]
        elif args.decode_small_only:
            r1 = bench_decode(workloads.decode_tinyllama_f32_b4(), args.steps, args.warmup, graph=True)
            out = {"value": round(r1["ms"] * 1e3, 3), "unit": "us", "gbs": round(r1["gbs"], 1), "bytes": r1["bytes"]}
        else:
            out = config_decode_long(args, None, False)
        print(json.dumps(out), flush=True)
        return
    log("bench: paged decode B256 Hq32 Hkv8 D128 fp16")
    wl3 = workloads.decode_llama3_8b_b256()
    torch.cuda.synchronize()
    r3 = bench_decode(wl3, args.steps, args.warmup, graph=False, per_launch=64)
    log(f"bench: paged decode B256 {r3['ms']:.4f} ms {r3['gbs']:.1f} GB/s")

    configs = {}
    if not args.primary_only:
        log("bench: paged decode TinyLlama fp32 B4")
        wl1 = workloads.decode_tinyllama_f32_b4()
        r1 = bench_decode(wl1, args.steps, args.warmup, graph=True)
        configs["decode_tinyllama_f32_b4"] = {
            "value": round(r1["ms"] * 1e3, 3), "unit": "us", "gbs": round(r1["gbs"], 1),
            "bytes": r1["bytes"], "note": "cache-resident (~1 MB): latency-bound, not an HBM figure"}
        if cpu_on:
            cb = cpu_baseline_decode(wl1, seconds=3.0, sample_seqs=wl1.batch, env=env)
            cb["us_per_call"] = round(cb["ms_per_call"] * 1e3, 1)
            configs["decode_tinyllama_f32_b4"]["cpu_baseline"] = cb
        del wl1
        log("bench: causal prefill TinyLlama shape L512 + L1024 (and Llama-3-8B heads L2048 / 4096 / 8192)")
        wl2, configs["prefill_tinyllama_f16"] = bench_prefill(args.steps, args.warmup)
        if cpu_on:
            configs["prefill_tinyllama_f16"]["cpu_baseline"] = cpu_baseline_prefill(wl2, env=env)
        del wl2
        log("bench: split-context decode B16 x 32768 bf16")
        configs["decode_long_bf16_b16_32k"] = config_decode_long(args, env, cpu_on)
        torch.cuda.empty_cache()
        log("bench: TinyLlama-1.1B greedy decode B64, prompts 1024, 128 steps")
        state, configs["e2e_tinyllama_decode"] = bench_e2e()
        log(f"bench: TinyLlama decode {configs['e2e_tinyllama_decode']['value']} tok/s")
        if cpu_on:
            log("bench: TinyLlama decode cpu baseline (one oracle step at B64)")
            configs["e2e_tinyllama_decode"]["cpu_baseline"] = cpu_baseline_e2e(state, env=env)
            configs["e2e_tinyllama_decode"]["parity"] = state["tf_parity"]
        del state
        torch.cuda.empty_cache()
        log("bench: streaming-read ceiling (2 GiB)")
        ceiling = bench_read_ceiling()
        configs["hbm_read_ceiling"] = ceiling
        for key in ("decode_long_bf16_b16_32k",):
            configs[key]["frac_of_read_ceiling"] = round(configs[key]["value"] / ceiling["value"], 4)
        torch.cuda.empty_cache()

    if args.calib_copy_mib:
        calibration_copy(args.calib_copy_mib)

    cpu = None
    if cpu_on:
        log("bench: cpu baseline (oracle float32 restatement)")
        cpu = cpu_baseline_decode(wl3, seconds=args.cpu_seconds, env=env)

    line = {
        "metric": "paged-decode HBM GB/s (% of peak), prefill TFLOP/s, TinyLlama decode tok/s",
        "value": round(r3["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r3["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) q/k/v; seeded context lengths and shuffled block tables)",
        "config": {"workload": "paged_decode Llama-3-8B head shape: B256 Hq32 Hkv8 D128 block16 fp16 KV, "
                               "ctx~U[512,4096] seed 0, pool +10% shuffled",
                   "sum_ctx": int(wl3.context_lens.astype(np.int64).sum()),
                   "partition_size": r3["partition_size"]},
        "roofline": {"bound": "hbm", "achieved": round(r3["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r3["gbs"] / HBM_PEAK_GBS, 4), "traffic": PRIMARY_TRAFFIC_BYTES,
                     "traffic_source": PRIMARY_TRAFFIC_SOURCE,
                     "algorithmic_bytes_per_launch": r3["bytes"],
                     "timing": "HIP events over K launches of decode+merge on the launch stream"},
        "per_launch": r3["per_launch"],
        "frac_of_read_ceiling": (round(r3["gbs"] / configs["hbm_read_ceiling"]["value"], 4)
                                 if "hbm_read_ceiling" in configs else None),
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


def config_decode_long(args, env, cpu_on):
    """Split-context decode, Llama-3-8B heads, bf16, 16 sequences x 32768."""
    from tinyvllm_amd import workloads
    wl5 = workloads.decode_long_bf16_b16()
    r5 = bench_decode(wl5, max(10, args.steps // 2), args.warmup, graph=False)
    out = {"value": round(r5["gbs"], 1), "unit": "GB/s", "ms": round(r5["ms"], 4),
           "frac_of_hbm_peak": round(r5["gbs"] / HBM_PEAK_GBS, 4), "bytes": r5["bytes"],
           "partition_size": r5["partition_size"],
           "traffic": LONG_TRAFFIC_BYTES, "traffic_over_algorithmic": round(LONG_TRAFFIC_BYTES / r5["bytes"], 4),
           "traffic_source": LONG_TRAFFIC_SOURCE}
    if cpu_on:
        out["cpu_baseline"] = cpu_baseline_decode(wl5, seconds=4.0, sample_seqs=1, env=env)
    del wl5
    return out


if __name__ == "__main__":
    main()
