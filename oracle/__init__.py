"""CPU oracle for the ZoomKV quantized / sparse KV decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``zoomkv_revision_amd``)
imports, links or executes anything under ``oracle/``; only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use
it, and only as the checker (or the timed CPU baseline), never as the thing
measured or shipped.

Every function restates an algorithm of the reference
(amy-77/zoomkv_revision, runtime/zoomkv_urania_runtime_20261011) in plain
numpy, with each floating-point operation written out and rounded
explicitly, and cites the reference file:line it follows.  Citation prefixes:

  Z/  = runtime/zoomkv_urania_runtime_20261011/
  S   = Z/cache_hub/polar_cache_quest_density_single_layer_kivi.py
  PC  = Z/cache_hub/polar_cache.py

How each part is pinned (beyond the reference's own tests, which hold no
golden vectors for this path) is listed in ``PINNING`` below and checked by
``tests/test_oracle_*.py``.
"""

PINNING = {
    "numerics.bf16_round": "exhaustive against torch's float32->bfloat16 cast",
    "kivi.kivi_codes": "golden vectors of quant_pack.quantize_kcache_4bit "
                       "(g = 8 / 16 / 32, bit-exact, tests/test_golden.py); "
                       "op-by-op against torch-CPU bfloat16 ops mirroring "
                       "S:2003-2009 and quant_pack.py:112-121; exhaustive "
                       "divide-vs-reciprocal check over all bf16 diffs; "
                       "invariants (flat group -> 0, max -> 15, range)",
    "kivi.pack_last_dim": "golden vectors of quant_pack.pack_kcache_4bit + "
                          "the S:2017 relayout (bit-exact); closed form + "
                          "brute-force round trip of all 16 code values at "
                          "every nibble position",
    "kivi.chunk_minmax_mean / dequant_ref": "golden vectors of torch amin / "
                                            "amax / mean (S:2133-2135) and "
                                            "quant_pack.unpack_kcache_4bit",
    "kivi.kivi4_dequant / attention": "textbook softmax attention in float64 "
                                      "over dequantized K/V; LSE split "
                                      "invariance; GQA head independence",
    "quest.quest_chunk_score": "golden vectors of QuestPytorch (within the "
                               "bf16 product-rounding bound); upper-bound "
                               "invariant vs brute force "
                               "max_t q.k_t; order-independence where sums "
                               "are exact; torch-CPU product identity",
    "topk": "set equality with numpy argsort on tie-free inputs; planted "
            "selections",
    "stage2.kivi_qk_dense_sparse": "golden vectors of qk_dot."
                                   "partial_chunk_kivi_qk_ref (one bf16 unit, "
                                   "kept sets); op-by-op bf16 ladder vs torch-CPU "
                                   "(quant_pack/qk_dot ops); bitonic network "
                                   "vs stable sort on tie-free inputs",
    "density": "tree sum equals fsum within 1 ulp; exact on dyadic inputs",
    "kivi.lse_merge": "golden vectors of lse_merge.lse_merge_torch",
    "rabitq": "popcount identity vs brute-force +-1 dot products; FWHT vs "
              "explicit Hadamard matrix; correction factor closed form",
    "rabitq4": "golden vectors of the reference's own ParisKV code run on the CPU "
               "(tests/golden/make_golden_rabitq4.py: polar_cache.batch_encode / "
               "_encode_query_blocks / _pack_4bit_codes, rerank._unpack_4bit_codes, "
               "test_rerank_topk.python_rabitq_scores): codes, weights, query blocks "
               "and scores bit-exact; closed forms: sign bits and magnitude buckets "
               "vs an fp64 Hadamard-matrix rotation away from thresholds, weights vs "
               "(r / alpha) ||k|| in fp64, one-hot scores exact for every (block, "
               "dimension, 4-bit value); top-k vs a brute-force sort",
    "torch_cpu.decode_attention": "against kivi.kivi4_decode_attention (numpy, float64) on the same "
                                  "Format Q cache, 1e-5 (tests/test_oracle_kivi.py); it is the timed "
                                  "CPU baseline of bench.py, not a checker",
}
