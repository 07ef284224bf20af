"""CPU oracle for the KV-cache data path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's semantics for every op of the path
(swap, slot mapping, append, gather, pack/scatter, defrag, paged decode
attention).  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the reference that results are
compared with or as the timed CPU baseline; the product package
(``aegaeon_amd``) never imports it.

Pinning (what fixes each function independently of this file's formulas):
  swap_blocks, copy_blocks, pack/scatter  - brute-force per-byte loops in
      tests/golden/make_golden.py (fixtures cfg1_*.npz) and round-trip identities.
  slot_mapping, pad_block_tables           - hand-computed literals (15/16/17,
      length 1) in tests/test_oracle.py and the golden fixtures.
  reshape_and_cache_flash / append_layers  - literal-index checks on the
      [N, L, 2, 16, Hkv, D] storage, append->gather identity, poisoned-pool
      "untouched slots unchanged" test.
  gather_tokens                            - per-token brute force in the
      golden fixtures.
  plan_defrag / apply_defrag               - invariants (bijection, disjoint
      src/dst, dense prefix, per-sequence bytes unchanged).
  paged_decode_attention                   - torch.nn.functional
      scaled_dot_product_attention in float64 on the gathered K/V, plus the
      closed forms len=1 -> V0, equal keys -> mean(V), dominant logit -> V_argmax,
      GQA == MHA with repeated KV heads.
"""
