"""CPU oracle of the flash-mlm fused MLM attention path -- TEST INFRASTRUCTURE ONLY.

Plain numpy restatements of the reference's algorithm, used as the checker of the
HIP implementation.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package; the product
(``flash-mlm_amd/flash_mlm``) never does.

Modules:
  pack_ref       pack metadata, padded length, pack / pad / unpack (integer and copy
                 work, bit-exact contract)
  attention_ref  packed and dense MLM attention in float64 / float32
  cpu_baseline   the reference benchmark's per-sequence PyTorch SDPA path on the host
                 CPU (the reported CPU baseline, not a checker)

Parity pins (see tests/test_oracle_*.py):
  pack_ref       the reference's own known-answer tests (test_host_utils.py:19-151,
                 235-311), committed as tests/golden/reference_kats.json, plus closed-form
                 invariants (round trip, counts, monotonicity) on random inputs.
  attention_ref  closed forms that a wrong index, sign, dropped segment or swapped
                 operand breaks: zero queries give the mean of the attended values;
                 a single attended key returns its value row; very large logits select
                 the arg-max key; per-sequence no-context cases equal
                 torch.nn.functional.scaled_dot_product_attention; key-order permutation
                 invariance; linearity in V; the causal_query_seq_attn and cached-context
                 cases equal explicit concatenations checked against the same library
                 routine.
Nothing in this package is "parity unpinned".
"""
