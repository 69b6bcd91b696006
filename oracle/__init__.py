"""ORACLE -- test infrastructure, not product code.

A CPU restatement (PyTorch on CPU tensors) of nano-kvllm's attention hot path,
each function citing the reference lines it follows. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only to check results or as the timed CPU baseline -- never as a
compute path of the package (which has no CPU fallback).

Modules:
  attention_ref  store_kvcache, paged decode, varlen causal prefill
  compress_ref   window location, SnapKV (bf16 as the reference, or fp32),
                 deterministic top-k, two-phase compaction, events, the
                 compression schedule
  rope_ref       q/k RMSNorm, rotary table and rotation, the fused step
  metadata_ref   per-step positions, slots, cu_seqlens, padded block tables
  fp8_ref        OCP E4M3FN quantize / dequantize, fp8 store

How each function is pinned (tests/test_oracle_*.py):
  store_kvcache_ref         pure-Python slot loop on tiny inputs; -1 rows
                            skipped; untouched rows unchanged
  paged_decode_ref          torch scaled_dot_product_attention on the gathered
                            K/V; float64 Python loops; ctx=1 -> V[0]; equal
                            keys -> mean(V); block-permutation invariance;
                            GQA == MHA with repeated K/V heads
  varlen_prefill_ref        SDPA(is_causal) for Lq == Lk; last query row ==
                            decode; chunked == one-shot; float64 loops
  varlen_prefill_rows_ref   the same rows of varlen_prefill_ref; each row ==
                            decode over the keys it sees
  snapkv_ref / select_topk  float64 brute force on tiny windows with planted
                            sink / head-sum / scale / last-token cases;
                            bf16 path == fp32 path on well-separated scores
  compress_compact_ref      per-slot brute force on tiny blocks (B=4);
                            closed forms of new_len / keep_blocks / freed ids
  compress_schedule_ref     the host scheduler on random batch states
  rope_ref                  Hugging Face Qwen3 RMSNorm / rotary, bit for bit;
                            rotation invariants
  metadata_ref              hand-computed slots, positions and prefix sums
  fp8_ref                   the E4M3FN table from the format's definition and
                            a brute-force nearest-even search, against torch
No reference test, fixture or golden vector exists for this path (the
reference repository has no tests); flash-attn, which the reference calls for
decode and prefill, is not installed here, so those two are pinned by the
closed forms and library routines above, not by the reference's own outputs.
"""
