"""CPU oracle for the tinyvllm attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``tinyvllm_amd``)
imports, links or executes anything in this directory.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the checker (or, for the baseline, as the timed CPU restatement of
the reference algorithm).

The reference (jonirajala/tinyvllm) is pure Python on top of tinygrad, which is
not installed here and is unpinned (requirements.txt:1).  The oracle is
therefore a numpy restatement of the reference's tensor expressions, file by
file:

=====================================  =========================================
oracle function                         reference it restates
=====================================  =========================================
attention.paged_decode_ref              tinyvllm/model/llama.py:97-144
attention.paged_decode_split_ref        (no reference counterpart; must equal
                                        llama.py:97-144 -- LSE merge algebra)
attention.flash_prefill_ref             tinyvllm/model/llama.py:58-94
kv_cache.KVCacheRef                     tinyvllm/core/kv_cache.py:13-61
kv_cache.reshape_and_cache_ref          kv_cache.py:34-38 driven per token by a
                                        slot mapping (llama.py:199-209, 381-386)
block_manager.BlockManagerRef           tinyvllm/core/block_manager.py:6-92
block_manager.write_kv_plan_ref         tinyvllm/model/llama.py:188-209
block_manager.prepare_batch_tensors_ref tinyvllm/core/engine.py:235-255 and
                                        tinyvllm/model/llama.py:368-374
=====================================  =========================================

Parity pinning (what each function is checked against, in tests/test_oracle.py):

* paged_decode_ref: torch ``scaled_dot_product_attention`` (float64, CPU) on the
  contiguous K/V trimmed to the context -- the reference test's own oracle
  (test_paged_attention.py:14-49, fixture :65-103); a scalar brute-force loop
  on tiny shapes; closed forms (ctx=1 -> V row; K=0 -> mean of V; ctx=0 -> mean
  of the padded gather); invariants (block-id permutation, padding contents).
* paged_decode_split_ref: equality with paged_decode_ref for every partition
  size (the merge is algebraically exact).
* flash_prefill_ref: torch SDPA causal / non-causal with GQA; the reference's
  known answers (test_flash_attention.py:123-139); L=1 -> V.
* KVCacheRef / reshape_and_cache_ref: the reference's exact-sum known answers
  (test_kv_cache.py:143-365) and brute-force element placement.
* BlockManagerRef / write_kv_plan_ref / prepare_batch_tensors_ref: integer
  functions, pinned by brute-force enumeration of positions and by the
  allocation order the reference code fixes (LIFO pop from list(range(N))).

Parity unpinned: tinygrad's ulp-level numerics (reduction order, exp lowering,
f16 rounding point of q@k^T, output-dtype promotion).  The reference ships no
golden vectors and tinygrad cannot be imported, so these stay unpinned; the
build is held to max-abs tolerances instead (f32 1e-4, f16/bf16 2e-2).
"""
